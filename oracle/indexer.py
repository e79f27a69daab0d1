"""Oracle: lightning indexer score and stable top-k.

Test infrastructure only (see ``oracle/__init__.py``).

``indexer_scores`` restates the score kernel
(lightning_indexer_triton.py:147-280): for every (b, s1, n2) row and key s2,
score = sum over the G = N1/N2 heads of the group of
ReLU(q[b,s1,n2*G+g] . k[b,s2,n2]) * w[b,s1,n2*G+g], in fp32 with no scale
(264-269); keys at or beyond act_k are -inf (274); in sparse_mode 3 keys at or
beyond min(max(act_k-act_q+s1+1, 0), S2) are -inf (219-224, 272-273); rows
with s1 >= act_q are all -inf (227, 275-276).

``stable_topk`` restates ``_stable_topk`` (339-357) with the stable order the
readme specifies (readme.md:69): score descending, index ascending on ties,
entries whose score is -inf reported as index -1.  When k exceeds S2 the row
is padded with index -1 / value -inf (the reference's reshape fails there).
"""
import numpy as np

from .common import cumsum_to_lengths, tnd_to_bsnd, bsnd_to_tnd, round_to, pa_to_bsnd


def visible_limit(sparse_mode, aq, ak, s1, S2):
    """Number of leading keys a query row may see (lightning_indexer_triton.py:219-224)."""
    if s1 >= aq:
        return 0
    if sparse_mode == 3:
        return min(ak, min(max(ak - aq + s1 + 1, 0), S2))
    return min(ak, S2)


def indexer_scores(q, k, w, act_q, act_k, sparse_mode=3, rows=None):
    """Returns fp32 scores [B, S1, N2, S2] (-inf where masked).

    q [B,S1,N1,D], k [B,S2,N2,D], w [B,S1,N1] as fp32 arrays of
    dtype-rounded values.  ``rows`` optionally restricts to (b, s1) pairs.
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    w = np.asarray(w, np.float32)
    B, S1, N1, D = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    out = np.full((B, S1, N2, S2), -np.inf, np.float32)
    if rows is None:
        rows = [(b, s1) for b in range(B) for s1 in range(S1)]
    for b, s1 in rows:
        lim = visible_limit(sparse_mode, int(act_q[b]), int(act_k[b]), s1, S2)
        if lim <= 0:
            continue
        for n2 in range(N2):
            qg = q[b, s1, n2 * G:(n2 + 1) * G]            # [G, D]
            dots = qg @ k[b, :lim, n2, :].T                # [G, lim]
            out[b, s1, n2, :lim] = np.maximum(dots, 0.0).T @ w[b, s1, n2 * G:(n2 + 1) * G]
    return out


def stable_topk(scores, k):
    """scores [R, S2] fp32 -> (indices int32 [R, k], values fp32 [R, k]).

    Order: score descending, then index ascending; -inf entries -> index -1.
    """
    scores = np.asarray(scores, np.float32)
    R, S2 = scores.shape
    idx = np.full((R, k), -1, np.int32)
    val = np.full((R, k), -np.inf, np.float32)
    kk = min(k, S2)
    cols = np.arange(S2)
    for r in range(R):
        order = np.lexsort((cols, -scores[r].astype(np.float64)))[:kk]
        v = scores[r, order]
        idx[r, :kk] = np.where(v == -np.inf, -1, order).astype(np.int32)
        val[r, :kk] = v
    return idx, val


def lightning_indexer(query, key, weights, actual_seq_lengths_query=None,
                      actual_seq_lengths_key=None, layout_query="BSND",
                      layout_key="BSND", sparse_count=2048, sparse_mode=3,
                      return_value=False, value_dtype="bfloat16", block_table=None):
    """Oracle of the public indexer API (lightning_indexer_triton.py:462-550).

    Returns (indices int32, values rounded to ``value_dtype``), BSND
    [B,S1,N2,k] or TND [T1,N2,k].  ``layout_key="PA_BSND"`` (the build's
    extension; the reference rejects a block_table, 497-498) de-pages the key
    cache the way the reference's SFA does (``pa_to_bsnd``,
    sparse_flash_attention_triton.py:382-403: -1 blocks stay zero rows) and
    takes per-batch ``actual_seq_lengths_key``.
    """
    is_tnd = layout_query == "TND"
    paged = layout_key == "PA_BSND"
    if paged:
        key = pa_to_bsnd(key, block_table, np.asarray(block_table).shape[1] * key.shape[1])
        ak_paged = np.asarray(actual_seq_lengths_key)
    if is_tnd:
        aq = cumsum_to_lengths(actual_seq_lengths_query)
        ak = ak_paged if paged else cumsum_to_lengths(actual_seq_lengths_key)
        q = tnd_to_bsnd(query, aq)
        w = tnd_to_bsnd(weights, aq)
        k = tnd_to_bsnd(key, ak) if layout_key == "TND" else key
    else:
        q, k, w = query, key, weights
        B = q.shape[0]
        aq = np.full(B, q.shape[1]) if actual_seq_lengths_query is None else np.asarray(actual_seq_lengths_query)
        ak = np.full(B, k.shape[1]) if actual_seq_lengths_key is None else np.asarray(actual_seq_lengths_key)
        if paged:
            ak = ak_paged
    B, S1 = q.shape[0], q.shape[1]
    S2, N2 = k.shape[1], k.shape[2]
    sc = indexer_scores(q, k, w, aq, ak, sparse_mode)
    idx, val = stable_topk(sc.reshape(B * S1 * N2, S2), sparse_count)
    idx = idx.reshape(B, S1, N2, sparse_count)
    val = val.reshape(B, S1, N2, sparse_count)
    val = round_to(val, value_dtype) if return_value else np.zeros_like(val)
    if is_tnd:
        idx = bsnd_to_tnd(idx, aq)
        val = bsnd_to_tnd(val, aq)
    return idx, val
