"""Oracle: dense lightning-indexer softmax LSE and dense KL-loss backward.

Test infrastructure only (see ``oracle/__init__.py``).

Restates the dense warm-up stage of the reference, the kernels
``_dense_indexer_stats_kernel``, ``_dense_loss_kernel``,
``_dense_main_grad_kernel`` and ``_dense_dkey_index_kernel``
(dense_loss_backward_triton.py:129-397), and the NumPy LSE baseline of its
test (test_dense_loss_backward_triton.py:101-138).  For every query row
(b, s1) with s1 < act_q, over the visible keys t < L, L = min(max(act_k -
act_q + s1 + 1, 0), S2) (lines 139-141):

  I[t]  = sum_g w_g ReLU(qi_g . ki_t)                                  (56-72)
  LSE:  imax = max_t I[t] (-inf if no key), isum = sum_t exp(I - imax)  (146-177)
  p[t]  = (1/N1) sum_h exp(s_h[t] - max_h) / (sum_h + 1e-8),
          s_h[t] = (q_h . k[t, h // G] + qr_h . kr[t, h // G]) * scale (75-126)
  student[t] = exp(I[t] - imax) / max(isum, 1e-8); both are 0 where the
          row is inactive or isum <= 0 (has_valid, 204-228)
  dI = student - p; loss += sum_t P (log P - log Q), P = max(p, 1e-8),
          Q = max(student, 1e-8)                                        (300-318)
  dW_g = sum_t dI ReLU_g; dQi_g = sum_t dI w_g 1[dot_g > 0] ki_t       (230-249)
  dKi[t] += sum_g dI w_g 1[dot_g > 0] qi_g                              (384-397)

softmax_max / softmax_sum are [B, N2, S1, G] (head h = n2 * G + g, the
reference's transpose at 474-475).  The index statistics are inputs of the
backward when given (the reference's ``*_with_index_core``, 547-655) and
computed by the LSE otherwise.
"""
import numpy as np


def _visible(act_q, act_k, s1, S2):
    return min(max(int(act_k) - int(act_q) + s1 + 1, 0), S2)


def dense_index_lse(qi, ki, w, act_q=None, act_k=None, compute_dtype=np.float64):
    """Returns (max_index, sum_index), each [B, 1, S1] (reference lines 146-177)."""
    ct = compute_dtype
    qi, ki, w = (np.asarray(x, ct) for x in (qi, ki, w))
    B, S1 = qi.shape[:2]
    S2 = ki.shape[1]
    aq = np.full(B, S1) if act_q is None else np.asarray(act_q)
    ak = np.full(B, S2) if act_k is None else np.asarray(act_k)
    imax = np.full((B, 1, S1), -np.inf, ct)
    isum = np.zeros((B, 1, S1), ct)
    for b in range(B):
        for s1 in range(S1):
            if s1 >= aq[b]:
                continue
            L = _visible(aq[b], ak[b], s1, S2)
            if L <= 0:
                continue
            I = w[b, s1] @ np.maximum(qi[b, s1] @ ki[b, :L, 0].T, 0.0)
            m = I.max()
            imax[b, 0, s1] = m
            isum[b, 0, s1] = np.exp(I - m).sum()
    return imax, isum


def dense_kl_bwd(q, k, qr, kr, qi, ki, w, softmax_max, softmax_sum, scale, imax=None, isum=None,
                 act_q=None, act_k=None, compute_dtype=np.float64):
    """q [B,S1,N1,D], k [B,S2,N2,D], qr / kr rope (or None), qi [B,S1,Nidx1,Di],
    ki [B,S2,1,Di], w [B,S1,Nidx1], softmax stats [B,N2,S1,G]; imax / isum
    ([B*S1] values in row order) or None to compute them.  Returns a dict
    with dQueryIndex, dKeyIndex, dW, loss [1], and the per-row p, student, dI
    ([B,S1,S2], zero past the visible range)."""
    ct = compute_dtype
    q, k, qi, ki, w = (np.asarray(x, ct) for x in (q, k, qi, ki, w))
    qr = None if qr is None else np.asarray(qr, ct)
    kr = None if kr is None else np.asarray(kr, ct)
    B, S1, N1, D = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    Ni = qi.shape[2]
    aq = np.full(B, S1) if act_q is None else np.asarray(act_q)
    ak = np.full(B, S2) if act_k is None else np.asarray(act_k)
    if imax is None:
        imax, isum = dense_index_lse(qi, ki, w, aq, ak, ct)
    imax = np.asarray(imax, ct).reshape(B, S1)
    isum = np.asarray(isum, ct).reshape(B, S1)
    smax = np.asarray(softmax_max, ct).reshape(B, N2, S1, G)
    ssum = np.asarray(softmax_sum, ct).reshape(B, N2, S1, G)
    eps = ct(1e-8)
    dqi = np.zeros(qi.shape, ct)
    dki = np.zeros(ki.shape, ct)
    dw = np.zeros(w.shape, ct)
    p_all = np.zeros((B, S1, S2), ct)
    st_all = np.zeros((B, S1, S2), ct)
    loss = ct(0.0)
    heads = np.arange(N1)
    kvh = heads // G
    for b in range(B):
        for s1 in range(S1):
            if s1 >= aq[b] or not isum[b, s1] > 0:
                continue
            L = _visible(aq[b], ak[b], s1, S2)
            if L <= 0:
                continue
            dots = qi[b, s1] @ ki[b, :L, 0].T                       # [Ni, L]
            relu = np.maximum(dots, 0.0)
            I = w[b, s1] @ relu
            student = np.exp(I - imax[b, s1]) / max(isum[b, s1], eps)
            # teacher: head h against key head h // G
            s = np.einsum("hd,thd->ht", q[b, s1], k[b, :L][:, kvh, :])
            if qr is not None:
                s = s + np.einsum("hd,thd->ht", qr[b, s1], kr[b, :L][:, kvh, :])
            s = s * ct(scale)
            m = smax[b, kvh, s1, heads % G][:, None]
            l = ssum[b, kvh, s1, heads % G][:, None]
            p = (np.exp(s - m) / (l + eps)).sum(0) / N1
            dI = student - p
            pc = np.maximum(p, eps)
            qc = np.maximum(student, eps)
            loss = loss + ct(np.sum(pc * (np.log(pc) - np.log(qc))))
            dw[b, s1] = relu @ dI
            ds = dI[None, :] * w[b, s1][:, None] * (dots > 0)        # [Ni, L]
            dqi[b, s1] = ds @ ki[b, :L, 0]
            dki[b, :L, 0] += ds.T @ qi[b, s1]
            p_all[b, s1, :L] = p
            st_all[b, s1, :L] = student
    return {"dQueryIndex": dqi, "dKeyIndex": dki, "dW": dw, "loss": np.array([loss], ct),
            "p": p_all, "student": st_all, "dI": st_all - p_all}
