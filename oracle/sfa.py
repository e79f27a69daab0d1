"""Oracle: sparse flash attention forward (MLA-absorb, MQA).

Test infrastructure only (see ``oracle/__init__.py``).

``sfa_fwd_bsnd`` restates the reference CPU golden
``sparse_flash_attention_golden_bsnd`` (sparse_flash_attention_numpy.py:63-160):
for every batch ``b`` and active query row ``s1`` the selected key rows are
gathered, every head computes softmax((q_nope.k_nope + q_rope.k_rope)*scale)
in fp32, the probabilities are rounded to the I/O dtype before the P.V
product (sparse_flash_attention_numpy.py:108-115, 149), the output is rounded
once more at the end (155-159), and softmax_max / softmax_sum are the raw row
max and sum of exponentials (152-153).  Value is key[..., :D]; the value
tensor is ignored.  Heads are evaluated together as one matrix product
instead of the golden's per-head loop; the arithmetic per element is the same
fp32 dot product.

``sparse_flash_attention`` adds the layout handling of the public API
(sparse_flash_attention_triton.py:483-641): TND packing, paged KV through
``block_table``, block-wise index expansion.
"""
import numpy as np

from .common import (BF16, INT64_MAX, band_bounds, expand_block_indices, gather_positions,
                     kernel_positions, round_to,
                     cumsum_to_lengths, tnd_to_bsnd, bsnd_to_tnd, pa_to_bsnd)


def sfa_fwd_bsnd(q, k, sparse_indices, q_rope, k_rope, scale, act_q, act_k,
                 sparse_block_size=1, sparse_mode=3, return_lse=True,
                 dtype=BF16, positions="golden", rows=None, compute_dtype=np.float32,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """SFA forward on BSND arrays; inputs are fp32 arrays of dtype-rounded values.

    Args follow sparse_flash_attention_numpy.py:63-101.  ``positions`` picks
    the golden's scan ("golden", lines 38-60) or the kernels' per-entry
    masking ("kernel", sparse_flash_attention_triton.py:270-272); they agree
    on front-valid index rows.  ``rows`` optionally restricts evaluation to a
    list of (b, s1) pairs (other rows stay zero), used for sampled parity at
    full sizes.  ``compute_dtype=np.float64`` evaluates without any dtype
    rounding (used for finite differences and fp64 cross-checks).
    ``pre_tokens`` / ``next_tokens`` add the band mask of ``band_bounds``.

    Returns (out [B,S1,N1,D], softmax_max [B,1,S1,N1], softmax_sum [B,1,S1,N1]).
    """
    ct = compute_dtype
    q = np.asarray(q, ct)
    k = np.asarray(k, ct)
    qr = np.asarray(q_rope, ct)
    kr = np.asarray(k_rope, ct)
    B, S1, N1, D = q.shape
    out = np.zeros((B, S1, N1, D), ct)
    smax = np.zeros((B, 1, S1, N1), ct)
    ssum = np.zeros((B, 1, S1, N1), ct)
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
        k_sel = np.concatenate([k[b, pos, 0, :], kr[b, pos, 0, :]], axis=-1)   # [P, D+Dr]
        v_sel = k[b, pos, 0, :]                                                 # [P, D]
        q_full = np.concatenate([q[b, s1], qr[b, s1]], axis=-1)                # [N1, D+Dr]
        scores = (q_full @ k_sel.T) * scale                                     # [N1, P]
        mx = scores.max(axis=1, keepdims=True)
        e = np.exp(scores - mx)
        sm = e.sum(axis=1, keepdims=True)
        probs = e / sm if ct is not np.float32 else round_to(e / sm, dtype)
        out[b, s1] = probs @ v_sel
        if return_lse:
            smax[b, 0, s1] = mx[:, 0]
            ssum[b, 0, s1] = sm[:, 0]
    if ct is not np.float32:
        return out, smax, ssum
    return round_to(out, dtype), smax, ssum


def sparse_flash_attention(query, key, sparse_indices, scale_value, query_rope,
                           key_rope, block_table=None,
                           actual_seq_lengths_query=None,
                           actual_seq_lengths_kv=None, sparse_block_size=1,
                           layout_query="BSND", layout_kv="BSND", sparse_mode=0,
                           return_softmax_lse=False, dtype=BF16,
                           positions="kernel", pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Oracle of the public forward API (sparse_flash_attention_triton.py:483-641).

    Normalises TND / PA_BSND to dense BSND the way the reference's host code
    does (551-597), expands block ids (600), runs ``sfa_fwd_bsnd`` and packs
    TND results back (632-639).  Returns (out, softmax_max, softmax_sum) with
    the reference's shapes; stats are zeros unless requested.
    """
    is_tnd_q = layout_query == "TND"
    is_tnd_kv = layout_kv == "TND"
    is_pa = layout_kv == "PA_BSND"
    lq = lk = None
    if is_tnd_q:
        lq = cumsum_to_lengths(actual_seq_lengths_query)
        q = tnd_to_bsnd(query, lq)
        qr = tnd_to_bsnd(query_rope, lq)
        si = tnd_to_bsnd(sparse_indices, lq)
    else:
        q, qr, si = query, query_rope, sparse_indices
    if is_tnd_kv:
        lk = cumsum_to_lengths(actual_seq_lengths_kv)
        k = tnd_to_bsnd(key, lk)
        kr = tnd_to_bsnd(key_rope, lk)
    elif is_pa:
        max_s2 = np.asarray(block_table).shape[1] * key.shape[1]
        k = pa_to_bsnd(key, block_table, max_s2)
        kr = pa_to_bsnd(key_rope, block_table, max_s2)
    else:
        k, kr = key, key_rope
    B, S1 = q.shape[0], q.shape[1]
    S2 = k.shape[1]
    if is_tnd_q:
        act_q = lq
    else:
        act_q = (np.full(B, S1) if actual_seq_lengths_query is None
                 else np.asarray(actual_seq_lengths_query))
    if is_tnd_kv:
        act_k = lk
    elif is_pa:
        act_k = np.asarray(actual_seq_lengths_kv)
    else:
        act_k = (np.full(B, S2) if actual_seq_lengths_kv is None
                 else np.asarray(actual_seq_lengths_kv))
    si_tok = expand_block_indices(si, sparse_block_size)
    out, smax, ssum = sfa_fwd_bsnd(q, k, si_tok, qr, kr, scale_value, act_q, act_k,
                                   sparse_block_size=1, sparse_mode=sparse_mode,
                                   return_lse=return_softmax_lse, dtype=dtype,
                                   positions=positions, pre_tokens=pre_tokens,
                                   next_tokens=next_tokens)
    if is_tnd_q:
        out = bsnd_to_tnd(out, lq)
        smax = bsnd_to_tnd(smax.transpose(0, 2, 1, 3), lq).transpose(1, 0, 2)
        ssum = bsnd_to_tnd(ssum.transpose(0, 2, 1, 3), lq).transpose(1, 0, 2)
    return out, smax, ssum
