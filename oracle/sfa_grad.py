"""Oracle: sparse flash attention backward (MLA-absorb, MQA).

Test infrastructure only (see ``oracle/__init__.py``).

``sfa_bwd_bsnd`` restates ``sparse_flash_attention_grad_golden_bsnd``
(sparse_flash_attention_grad_numpy.py:34-143): per active row the
probabilities are rebuilt from the forward's softmax_max / softmax_sum
(line 121), dP = dO.v with v = key[..., :D] (122), delta = dO.O (123),
dS = P*(dP - delta)*scale (124); dq and dq_rope are per-row products
(127-128); dk, dk_rope and dv are scatter-adds over the gathered positions
(131-133); every gradient is rounded to the I/O dtype at the end (142-143).
Heads are evaluated together as matrix products.
"""
import numpy as np

from .common import BF16, INT64_MAX, band_bounds, gather_positions, kernel_positions, round_to


def sfa_bwd_bsnd(q, k, sparse_indices, d_out, out, softmax_max, softmax_sum,
                 q_rope, k_rope, scale, act_q, act_k, sparse_block_size=1,
                 sparse_mode=3, dtype=BF16, positions="golden", rows=None,
                 guard_sum=False, compute_dtype=np.float32, pre_tokens=INT64_MAX,
                 next_tokens=INT64_MAX):
    """Returns (d_query, d_key, d_value, d_query_rope, d_key_rope), fp32 arrays.

    ``guard_sum`` replaces a non-positive softmax_sum by 1, as the device
    kernel does (sparse_flash_attention_grad_triton.py:233-234); the golden
    divides unguarded, which only differs for rows with no valid token.
    ``pre_tokens`` / ``next_tokens`` add the band mask of ``band_bounds``
    (the forward oracle's rule).
    """
    ct = compute_dtype
    q = np.asarray(q, ct)
    k = np.asarray(k, ct)
    qr = np.asarray(q_rope, ct)
    kr = np.asarray(k_rope, ct)
    do = np.asarray(d_out, ct)
    o = np.asarray(out, ct)
    smax = np.asarray(softmax_max, ct)
    ssum = np.asarray(softmax_sum, ct)
    B, S1, N1, D = q.shape
    S2 = k.shape[1]
    Dr = qr.shape[-1]
    dq = np.zeros((B, S1, N1, D), ct)
    dqr = np.zeros((B, S1, N1, Dr), ct)
    dk = np.zeros((B, S2, 1, D), ct)
    dkr = np.zeros((B, S2, 1, Dr), ct)
    dv = np.zeros((B, S2, 1, D), ct)
    pos_fn = gather_positions if positions == "golden" else kernel_positions
    scale = ct(scale)
    if rows is None:
        rows = [(b, s1) for b in range(B) for s1 in range(S1)]
    for b, s1 in rows:
        aq, ak = int(act_q[b]), int(act_k[b])
        if s1 >= aq:
            continue
        if sparse_mode != 0 and s1 < aq - ak:
            continue
        lo, thr = band_bounds(sparse_mode, aq, ak, s1, pre_tokens, next_tokens)
        if thr <= 0:
            continue
        pos = pos_fn(sparse_indices[b, s1, 0, :], sparse_block_size, thr, ak, lo)
        if not pos:
            continue
        pos = np.asarray(pos, np.int64)
        kn = k[b, pos, 0, :]                                        # [P, D]
        krp = kr[b, pos, 0, :]                                      # [P, Dr]
        qn = q[b, s1]                                               # [N1, D]
        qrr = qr[b, s1]                                             # [N1, Dr]
        scores = (qn @ kn.T + qrr @ krp.T) * scale                  # [N1, P]
        den = ssum[b, 0, s1][:, None]
        if guard_sum:
            den = np.where(den > 0, den, ct(1.0))
        P = np.exp(scores - smax[b, 0, s1][:, None]) / den
        dP = do[b, s1] @ kn.T                                       # [N1, P]
        delta = np.sum(do[b, s1] * o[b, s1], axis=1, keepdims=True)
        dS = P * (dP - delta) * scale
        dq[b, s1] += dS @ kn
        dqr[b, s1] += dS @ krp
        np.add.at(dk[b, :, 0, :], pos, dS.T @ qn)
        np.add.at(dkr[b, :, 0, :], pos, dS.T @ qrr)
        np.add.at(dv[b, :, 0, :], pos, P.T @ do[b, s1])
    if ct is not np.float32:
        return dq, dk, dv, dqr, dkr
    return (round_to(dq, dtype), round_to(dk, dtype), round_to(dv, dtype),
            round_to(dqr, dtype), round_to(dkr, dtype))
