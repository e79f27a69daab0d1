"""Oracle: sparse lightning-indexer KL-loss backward.

Test infrastructure only (see ``oracle/__init__.py``).

``kl_loss_bwd`` restates the reference golden ``numpy_reference``
(sli_grad_kl_loss_numpy.py:16-152) stage by stage, for every active row
(b, s1) over its first n = s2_real entries:

1. gather: idx clipped to [0, S2-1] (56-60)
2. I[k] = sum_g w_g * ReLU(qi_g . ki[idx_k]); ReLU values cached (64-75)
3. teacher p[k] = (1/N1) sum_h exp(s_hk - max_h) / (sum_h + 1e-8) with
   s_hk = (q_h.k[idx_k] + qr_h.kr[idx_k]) * scale (78-93)
4. softmax(I) with +1e-8 in the denominator (96-104); dI = softmax(I) - p
   (107-108); KL = sum max(p,1e-8)*(log max(p,1e-8) - log max(sI,1e-8)),
   summed over all rows into one scalar (111-117)
5. dW_g = sum_k dI*ReLU_g; dQi_g = sum_k dI*w_g*1[ReLU_g>0]*ki[idx_k] (120-131)
6. dKi[idx_k] += dI*w_g*1[ReLU_g>0]*qi_g (134-147)

The golden rounds inputs and dot products to fp16 to imitate the CANN
kernel (23-29, 72, 89).  The device kernels of the reference do neither
(sparse_lightning_indexer_grad_kl_loss_triton.py:119-177 accumulate in fp32),
so ``round_dots`` / ``input_dtype`` select the behaviour.  Row activity and
n follow the device kernel: rows with s1 >= act_q are skipped and
n = min(topK, max(act_k - act_q + s1 + 1, 0)) (kernel lines 107-111, 58),
which equals the golden's min(topK, S2 - S1 + s1 + 1) at full lengths.
Out-of-range targets in step 6 are skipped by the golden (142-144) and
clamped by the device scatter (kernel line 300); ``dki_oob`` selects.

``kl_loss_bwd_tnd`` and ``kl_loss_bwd_paged`` extend the computation to the
packed (TND) and paged key layouts the reference rejects (kernel file
534-535).  They are compositions of ``kl_loss_bwd``: TND runs each batch as
its own B = 1 problem with S1, S2 = the batch's lengths (so token ids clamp
to the batch's key length), and a paged cache is de-paged with
``pa_to_bsnd`` (sparse_flash_attention_triton.py:382-403; -1 pages read as
zero rows), run as BSND with S2 = max_blocks * page, and the key-index
gradient is summed back onto the cache rows (-1 pages receive nothing).
"""
import numpy as np

from .common import cumsum_to_lengths, pa_to_bsnd, round_to

EPS = np.float32(1e-8)


def kl_loss_bwd(q, k, qr, kr, qi, ki, w, sparse_indices, softmax_max, softmax_sum,
                scale, act_q=None, act_k=None, input_dtype=None, round_dots=False,
                dki_oob="clamp", rows=None, compute_dtype=np.float32):
    """Returns dict with dQueryIndex [B,S1,Nidx1,Di], dKeyIndex [B,S2,1,Di],
    dW [B,S1,Nidx1], loss [1] (fp32) and the intermediates p, softmax_I, dI, I."""
    ct = compute_dtype

    def prep(x):
        if input_dtype is None:
            return np.asarray(x, ct)
        return round_to(np.asarray(x, np.float32), input_dtype).astype(ct)

    q, k, qr, kr, qi, ki, w = (prep(x) for x in (q, k, qr, kr, qi, ki, w))
    si = np.asarray(sparse_indices).astype(np.int64)
    smax = np.asarray(softmax_max, ct)
    ssum = np.asarray(softmax_sum, ct)
    B, S1, N1, D = q.shape
    S2 = k.shape[1]
    Nidx1, Di = qi.shape[2], qi.shape[3]
    topK = si.shape[3]
    act_q = np.full(B, S1) if act_q is None else np.asarray(act_q)
    act_k = np.full(B, S2) if act_k is None else np.asarray(act_k)
    scale = ct(scale)
    eps = ct(EPS)

    def rdot(x):
        return x.astype(np.float16).astype(ct) if round_dots else x

    dqi = np.zeros((B, S1, Nidx1, Di), ct)
    dki = np.zeros((B, S2, 1, Di), ct)
    dw = np.zeros((B, S1, Nidx1), ct)
    p_all = np.zeros((B, S1, topK), ct)
    sI_all = np.zeros((B, S1, topK), ct)
    I_all = np.zeros((B, S1, topK), ct)
    loss = ct(0.0)
    if rows is None:
        rows = [(b, s1) for b in range(B) for s1 in range(S1)]
    for b, s1 in rows:
        aq, ak = int(act_q[b]), int(act_k[b])
        if s1 >= aq:
            continue
        n = min(topK, max(ak - aq + s1 + 1, 0))
        if n <= 0:
            continue
        raw = si[b, s1, 0, :n]
        idx = np.clip(raw, 0, S2 - 1)
        kig = ki[b, idx, 0, :]                                   # [n, Di]
        kg = k[b, idx, 0, :]                                     # [n, D]
        krg = kr[b, idx, 0, :]                                   # [n, Dr]
        relu = np.maximum(rdot(qi[b, s1] @ kig.T), 0.0)          # [Nidx1, n]
        I = w[b, s1] @ relu                                      # [n]
        s = rdot((q[b, s1] @ kg.T + qr[b, s1] @ krg.T) * scale)   # [N1, n]
        probs = np.exp(s - smax[b, 0, s1][:, None]) / (ssum[b, 0, s1][:, None] + eps)
        p = probs.sum(axis=0) * ct(1.0 / N1)
        e = np.exp(I - I.max())
        sI = e / (e.sum() + eps)
        dI = sI - p
        pc = np.maximum(p, eps)
        sc = np.maximum(sI, eps)
        loss = loss + ct(np.sum(pc * (np.log(pc) - np.log(sc))))
        mask = (relu > 0).astype(ct)                     # [Nidx1, n]
        dw[b, s1] = relu @ dI
        ds = dI[None, :] * w[b, s1][:, None] * mask              # [Nidx1, n]
        dqi[b, s1] = ds @ kig
        contrib = ds.T @ qi[b, s1]                               # [n, Di]
        if dki_oob == "skip":
            keep = (raw >= 0) & (raw < S2)
            np.add.at(dki[b, :, 0, :], raw[keep], contrib[keep])
        else:
            np.add.at(dki[b, :, 0, :], idx, contrib)
        p_all[b, s1, :n] = p
        sI_all[b, s1, :n] = sI
        I_all[b, s1, :n] = I
    return {"dQueryIndex": dqi, "dKeyIndex": dki, "dW": dw,
            "loss": np.array([loss], ct), "p": p_all,
            "softmax_I": sI_all, "dI": sI_all - p_all, "I": I_all}


def _batch_problem(x, start, n):
    """Rows [start, start + n) of a packed tensor as a B = 1 BSND tensor."""
    return None if x is None else np.asarray(x)[start:start + n][None]


def kl_loss_bwd_tnd(q, k, qr, kr, qi, ki, w, sparse_indices, softmax_max, softmax_sum, scale,
                    cu_q, cu_k, **kw):
    """TND: q [T1,N1,D], k [T2,1,D], qi [T1,Nidx1,Di], ki [T2,1,Di], w [T1,Nidx1],
    sparse_indices [T1,1,topK], softmax stats with T1*N1 entries, cumulative
    lengths cu_q / cu_k.  Returns dQueryIndex [T1,Nidx1,Di], dKeyIndex
    [T2,1,Di], dW [T1,Nidx1] and loss [1]."""
    lq, lk = cumsum_to_lengths(cu_q), cumsum_to_lengths(cu_k)
    T1, N1 = q.shape[0], q.shape[1]
    T2 = k.shape[0]
    Nidx1, Di = qi.shape[1], qi.shape[2]
    smax = np.asarray(softmax_max, np.float32).reshape(T1, N1)
    ssum = np.asarray(softmax_sum, np.float32).reshape(T1, N1)
    si = np.asarray(sparse_indices).reshape(T1, 1, -1)
    ct = kw.get("compute_dtype", np.float32)
    dqi = np.zeros((T1, Nidx1, Di), ct)
    dki = np.zeros((T2, 1, Di), ct)
    dw = np.zeros((T1, Nidx1), ct)
    loss = ct(0.0)
    sq = sk = 0
    for nq, nk in zip(lq, lk):
        nq, nk = int(nq), int(nk)
        if nq > 0 and nk > 0:
            r = kl_loss_bwd(
                _batch_problem(q, sq, nq), _batch_problem(k, sk, nk), _batch_problem(qr, sq, nq),
                _batch_problem(kr, sk, nk), _batch_problem(qi, sq, nq), _batch_problem(ki, sk, nk),
                _batch_problem(w, sq, nq), si[sq:sq + nq][None], smax[sq:sq + nq][None, None],
                ssum[sq:sq + nq][None, None], scale, **kw)
            dqi[sq:sq + nq] = r["dQueryIndex"][0]
            dki[sk:sk + nk] = r["dKeyIndex"][0]
            dw[sq:sq + nq] = r["dW"][0]
            loss = loss + r["loss"][0]
        sq += nq
        sk += nk
    return {"dQueryIndex": dqi, "dKeyIndex": dki, "dW": dw, "loss": np.array([loss], ct)}


def kl_loss_bwd_paged(q, k_cache, qr, kr_cache, qi, ki_cache, w, sparse_indices, softmax_max,
                      softmax_sum, scale, block_table, act_k, act_q=None, **kw):
    """BSND queries over paged caches [blocks, page, 1, X] addressed by
    block_table [B, max_blocks] (-1 = no page); act_k per-batch lengths.
    dKeyIndex comes back in the cache shape."""
    bt = np.asarray(block_table)
    page = k_cache.shape[1]
    S2 = bt.shape[1] * page

    def dense(c):
        return None if c is None else pa_to_bsnd(np.asarray(c), bt, S2)

    r = kl_loss_bwd(q, dense(k_cache), qr, dense(kr_cache), qi, dense(ki_cache), w, sparse_indices,
                    softmax_max, softmax_sum, scale, act_q=act_q, act_k=act_k, **kw)
    dk = r["dKeyIndex"]                                         # [B, S2, 1, Di]
    out = np.zeros(ki_cache.shape, dk.dtype)
    for b in range(bt.shape[0]):
        for i in range(bt.shape[1]):
            blk = int(bt[b, i])
            if blk >= 0:
                out[blk] += dk[b, i * page:(i + 1) * page]
    r = dict(r)
    r["dKeyIndex"] = out
    return r
