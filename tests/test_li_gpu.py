"""GPU parity of the HIP lightning indexer against the oracle.

* Top-k (``dsa_li_topk_from_scores``): bit-exact against ``oracle.indexer.
  stable_topk`` on the same fp32 scores (score descending, index ascending on
  ties, -inf -> -1), including heavy ties, all-masked rows, rows with fewer
  visible keys than K, K > S2, and rows wider than the LDS-resident limit.
* Scores (``dsa_li_scores``): against the oracle's fp32 scores; both sum
  exact bf16 x bf16 products in fp32, in different orders, so the tolerance
  is a few fp32 ulps of the magnitude of the terms: rtol 1e-5 plus an
  absolute 1e-5 * sum_g |w_g| * |q_g| * |k| bound.  Masked entries must be
  -inf at exactly the same places.
* The full operator (``lightning_indexer_triton``): indices equal to the
  oracle's top-k of the oracle's scores except at near-ties (two candidates
  whose oracle scores differ by less than the score tolerance); the number
  of such tie flips is printed and must be a small fraction.
"""
import numpy as np
import pytest
import torch

from oracle.indexer import indexer_scores, lightning_indexer, stable_topk
from tests.helpers import dev, to_dtype_np

pytestmark = pytest.mark.gpu


def _api():
    import dsa_triton_ascend_amd as dsa
    return dsa


def _inputs(B, S1, S2, N1, N2, D, dtype, wdtype=torch.float32, seed=42):
    """fp16-representable q / k for 16-bit dtypes; full fp32 values for fp32
    (so that its products are not exact in fp32)."""
    rng = np.random.RandomState(seed)
    via16 = (lambda x: x) if dtype == torch.float32 else (lambda x: x.astype(np.float16).astype(np.float32))
    q = to_dtype_np(via16(rng.randn(B, S1, N1, D).astype(np.float32)), dtype)
    k = to_dtype_np(via16(rng.randn(B, S2, N2, D).astype(np.float32)), dtype)
    w = to_dtype_np(rng.rand(B, S1, N1).astype(np.float32), wdtype)
    return q, k, w


# ---------------------------------------------------------------------------
# top-k
# ---------------------------------------------------------------------------
def _topk_gpu(scores_np, k):
    from dsa_triton_ascend_amd.lightning_indexer import stable_topk as gpu_topk
    idx, val = gpu_topk(torch.from_numpy(scores_np).cuda(), k)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), val.cpu().numpy()


@pytest.mark.parametrize("S2,k,kind", [
    (64, 16, "random"), (300, 64, "ties"), (1000, 2048, "k_gt_s2"), (4096, 2048, "mixed"),
    (4096, 2048, "ties"), (16384, 2048, "random"), (20000, 2048, "ties"), (32768, 2048, "random"),
    (32768, 4096, "mixed"), (5000, 1, "ties"), (2049, 2048, "masked_tail"), (3000, 100, "equal"),
    (32768, 2048, "narrow"), (32767, 2048, "random"), (40001, 2048, "ties"), (8191, 4096, "random"),
    # K above 4096: the general selection with a 16384-entry LDS sort
    (32768, 8192, "random"), (20000, 16384, "ties"), (40001, 8192, "mixed"), (12000, 16384, "k_gt_s2"),
])
def test_topk_bit_exact(S2, k, kind):
    print(f"[li topk] S2={S2} k={k} {kind}", flush=True)
    rng = np.random.RandomState(S2 + k)
    R = 6
    if kind == "ties":
        sc = rng.randint(0, 7, size=(R, S2)).astype(np.float32) * 0.5
    elif kind == "equal":
        sc = np.full((R, S2), 3.25, np.float32)
    elif kind == "narrow":
        # all scores within a few ulps: the radix digits come from the low bits
        sc = (np.float32(100.0) + rng.randint(0, 40, size=(R, S2)).astype(np.float32) * np.float32(2 ** -17))
        sc = sc.astype(np.float32)
    else:
        sc = (rng.randn(R, S2) * 10).astype(np.float32)
    if kind in ("mixed", "masked_tail", "k_gt_s2"):
        # visible prefixes of different lengths, -inf beyond; one all-masked row
        lens = [S2, S2 // 2, k - 1, 1, 0, S2 - 3]
        for r, L in enumerate(lens):
            sc[r, max(L, 0):] = -np.inf
    if kind == "mixed":
        sc[1, :100] = 0.0          # a block of exact ties inside a row
        sc[5, ::7] = -0.0          # signed zeros tie with +0
        sc[5, 1::7] = 0.0
    ie, ve = stable_topk(sc, k)
    ig, vg = _topk_gpu(sc, k)
    np.testing.assert_array_equal(ig, ie)
    # values: identical fp32 (-inf where the index is -1); -0.0 == 0.0 compares equal
    np.testing.assert_array_equal(vg, ve)


@pytest.mark.parametrize("S2,k", [(300, 64), (2049, 2048), (4096, 2048), (4096, 1), (8192, 2048), (1500, 2048)])
def test_topk_many_short_rows_bit_exact(S2, k):
    """More rows than CUs (the four-rows-per-workgroup selection): every row
    kind in one launch, so the four rows of a workgroup mix fast rows with
    rows that take the general path (all-equal keys crowd one bin), rows
    with few or no visible keys, exact ties, signed zeros and narrow ranges.
    Bit-exact against np.lexsort on the same fp32 scores."""
    print(f"[li topk many rows] S2={S2} k={k}", flush=True)
    rng = np.random.RandomState(S2 * 7 + k)
    R = 600
    sc = (rng.randn(R, S2) * 10).astype(np.float32)
    kinds = rng.randint(0, 7, R)
    for r in range(R):
        if kinds[r] == 1:      # ties
            sc[r] = rng.randint(0, 7, S2).astype(np.float32) * 0.5
        elif kinds[r] == 2:    # all equal: one crowded bin
            sc[r] = 3.25
        elif kinds[r] == 3:    # visible prefix of random length
            sc[r, rng.randint(0, S2 + 1):] = -np.inf
        elif kinds[r] == 4:    # narrow range (a few ulps)
            sc[r] = np.float32(100.0) + rng.randint(0, 40, S2).astype(np.float32) * np.float32(2 ** -17)
        elif kinds[r] == 5:    # signed zeros and a block of exact ties
            sc[r, ::5] = -0.0
            sc[r, 1::5] = 0.0
            sc[r, :50] = 1.5
        elif kinds[r] == 6:    # nothing visible
            sc[r] = -np.inf
    sc = sc.astype(np.float32)
    ie, ve = stable_topk(sc, k)
    ig, vg = _topk_gpu(sc, k)
    np.testing.assert_array_equal(ig, ie)
    np.testing.assert_array_equal(vg, ve)


# ---------------------------------------------------------------------------
# scores
# ---------------------------------------------------------------------------
def _score_tol(q, k, w, N2):
    """Per (b, s1, n2, s2) bound on fp32 reassociation error of the score."""
    B, S1, N1, D = q.shape
    G = N1 // N2
    aq = np.abs(q).reshape(B, S1, N2, G, D)
    ak = np.abs(k)                                   # [B, S2, N2, D]
    aw = np.abs(w).reshape(B, S1, N2, G)
    # sum_g |w_g| * sum_d |q_gd||k_d|
    t = np.einsum("bsngd,btnd->bsnt", aq * aw[..., None], ak)
    return 1e-5 * t + 1e-6


@pytest.mark.parametrize("B,S1,S2,N1,N2,D,mode,dtype,wdtype", [
    (2, 8, 300, 64, 1, 128, 3, torch.bfloat16, torch.float32),
    (2, 8, 300, 64, 1, 128, 0, torch.bfloat16, torch.float32),
    (1, 5, 1100, 32, 2, 64, 3, torch.float16, torch.bfloat16),
    (2, 3, 257, 8, 1, 256, 0, torch.bfloat16, torch.float16),
    (1, 4, 2100, 128, 1, 128, 3, torch.bfloat16, torch.float32),
    (1, 2, 333, 24, 1, 128, 0, torch.float16, torch.float32),
    # head dims other than 64 / 128 / 256 (zero-padded rows), odd N1, G = 3
    (1, 4, 256, 7, 1, 96, 0, torch.bfloat16, torch.bfloat16),
    (2, 3, 300, 12, 4, 256, 3, torch.float16, torch.float16),
    (1, 3, 290, 8, 1, 40, 3, torch.bfloat16, torch.float32),
    # fp32 query / key / weights: full-fp32 products
    (1, 3, 500, 16, 2, 64, 3, torch.float32, torch.float32),
    (1, 4, 256, 7, 1, 96, 3, torch.float32, torch.float32),
    (2, 2, 400, 64, 1, 128, 0, torch.float32, torch.float32),
    (1, 2, 300, 40, 1, 256, 3, torch.float32, torch.float32),
    (1, 3, 200, 8, 1, 20, 0, torch.float32, torch.float32),
])
def test_scores_match_oracle(B, S1, S2, N1, N2, D, mode, dtype, wdtype):
    print(f"[li scores] B={B} S1={S1} S2={S2} N1={N1} N2={N2} D={D} mode={mode} {dtype}", flush=True)
    q, k, w = _inputs(B, S1, S2, N1, N2, D, dtype, wdtype)
    act_q = [S1] * B
    act_k = [S2 - 7 * b for b in range(B)]
    if B > 1:
        act_q[1] = max(1, S1 - 2)
    e = indexer_scores(q, k, w, act_q, act_k, mode)            # [B,S1,N2,S2]
    from dsa_triton_ascend_amd.lightning_indexer import indexer_scores as gpu_scores
    g = gpu_scores(dev(q, dtype), dev(k, dtype), dev(w, wdtype), act_q, act_k, mode)
    torch.cuda.synchronize()
    g = g.cpu().numpy().reshape(e.shape)
    assert np.array_equal(np.isneginf(g), np.isneginf(e)), "masked positions differ"
    fin = np.isfinite(e)
    tol = _score_tol(q, k, w, N2)
    err = np.abs(g[fin] - e[fin])
    assert np.all(err <= tol[fin] + 1e-5 * np.abs(e[fin])), f"max err {err.max():.3g}"


# ---------------------------------------------------------------------------
# full operator
# ---------------------------------------------------------------------------
def _check_topk_with_ties(idx_g, sc_rows, k, score_tol_rows, what, max_flips=None):
    """idx_g [R, k] from the GPU; sc_rows [R, S2] oracle fp32 scores.  Every
    differing entry must be a near tie (score gap within twice the
    reassociation bound); the count of such flips only guards against a
    systematic mismatch (max_flips, default max(4, entries / 500))."""
    ie, _ = stable_topk(sc_rows, k)
    flips = 0
    for r in range(ie.shape[0]):
        if np.array_equal(idx_g[r], ie[r]):
            continue
        d = np.nonzero(idx_g[r] != ie[r])[0]
        for j in d:
            a, b = idx_g[r, j], ie[r, j]
            assert a >= 0 and b >= 0, f"{what}: row {r} pos {j}: -1 mismatch ({a} vs {b})"
            gap = abs(float(sc_rows[r, a]) - float(sc_rows[r, b]))
            assert gap <= 2 * score_tol_rows[r], f"{what}: row {r} pos {j}: {a} vs {b}, score gap {gap:.3g}"
        flips += len(d)
    print(f"  {what}: tie flips {flips} of {idx_g.size} entries", flush=True)
    assert flips <= (max(4, idx_g.size // 500) if max_flips is None else max_flips)


def _full_case(B, S1, S2, N1, N2, D, k, mode, dtype, rows=None, act_q=None, act_k=None, seed=42,
               wdtype=torch.float32, max_flips=None):
    dsa = _api()
    q, k_, w = _inputs(B, S1, S2, N1, N2, D, dtype, wdtype, seed=seed)
    idx, val = dsa.lightning_indexer_triton(
        dev(q, dtype), dev(k_, dtype), dev(w, wdtype), act_q, act_k,
        sparse_count=k, sparse_mode=mode, return_value=True)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()
    val = val.float().cpu().numpy()
    aq = [S1] * B if act_q is None else act_q
    ak = [S2] * B if act_k is None else act_k
    sc = indexer_scores(q, k_, w, aq, ak, mode, rows=rows)  # [B,S1,N2,S2]
    G = N1 // N2
    sel = rows if rows is not None else [(b, s) for b in range(B) for s in range(S1)]
    for (b, s) in sel:
        rs = sc[b, s]                                     # [N2, S2]
        # reassociation bound of each score: 1e-5 * sum_g |w_g| sum_d |q_gd||k_d|
        a = (np.abs(q[b, s]) * np.abs(w[b, s])[:, None]).reshape(N2, G, D).sum(axis=1)   # [N2, D]
        t = 1e-5 * np.einsum("nd,tnd->nt", a, np.abs(k_[b])) + 1e-6                       # [N2, S2]
        _check_topk_with_ties(idx[b, s], rs, k, (np.where(np.isfinite(rs), t, 0.0).max(axis=1)
                                                 + 1e-5 * np.abs(np.where(np.isfinite(rs), rs, 0)).max()),
                              f"row ({b},{s})", max_flips)
        # values: the query dtype rounding of the score at the returned index
        for n2 in range(N2):
            ii = idx[b, s, n2]
            exp_v = np.where(ii >= 0, rs[n2, np.maximum(ii, 0)], -np.inf)
            exp_v = to_dtype_np(exp_v, dtype)
            with np.errstate(invalid="ignore"):  # -inf - -inf at the -1 slots, which ii < 0 covers
                ok = (ii < 0) | (np.abs(val[b, s, n2] - exp_v) <= 1e-2 * np.abs(exp_v) + 1e-3)
            assert ok.all() and np.array_equal(np.isneginf(val[b, s, n2]), ii < 0)
    return idx


@pytest.mark.parametrize("B,S1,S2", [(4, 4, 16384), (2, 8, 9000), (16, 2, 8192), (8, 3, 5000)],
                         ids=["mtp4_16k", "s1_8_9000", "mtp2_b16", "s1_3_b8"])
def test_indexer_multi_token_decode(B, S1, S2):
    """A few query rows per batch over a long key range (multi-token
    decode): from four rows per batch the multi-row score kernel splits each
    row group's keys into chunks over the CUs; two or three rows per batch
    run the one-row kernel with a batch's rows placed on one XCD (the
    remapped workgroup order); every row against the oracle (top-k with the
    tie rule, values)."""
    print(f"[li mtp] B={B} S1={S1} S2={S2}", flush=True)
    # every differing index is a near tie (checked); up to 16 per row of
    # 2048 (0.8 %) are allowed, where the 32K decode batch sees about one
    _full_case(B, S1, S2, 64, 1, 128, 2048, 3, torch.bfloat16, act_k=[S2 - 5 * b for b in range(B)],
               max_flips=16)


def test_indexer_small_mode3_hidden_rows():
    print("[li full] small mode3 with actual lengths", flush=True)
    idx = _full_case(2, 12, 40, 64, 1, 128, 16, 3, torch.bfloat16, act_q=[12, 9], act_k=[40, 20])
    # rows s1 >= act_q see nothing: all -1
    assert (idx[1, 9:] == -1).all()
    # mode 3: row s1 of batch 1 sees min(max(20 - 9 + s1 + 1, 0), 40) keys
    for s in range(9):
        vis = min(max(20 - 9 + s + 1, 0), 20)
        assert (idx[1, s, 0, :min(vis, 16)] >= 0).all() and (idx[1, s, 0, min(vis, 16):] == -1).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("B", [1, 2, 3])
@pytest.mark.parametrize("S1,S2,N1,N2,D,k", [
    (1, 128, 8, 1, 128, 32), (4, 256, 7, 1, 96, 32), (8, 128, 16, 2, 64, 64), (3, 256, 12, 4, 256, 32),
])
def test_indexer_reference_small_grid(S1, S2, N1, N2, D, k, B, mode, dtype):
    """The small shapes of the reference's test_basic grid (test_li_triton.py:42-57):
    odd N1, D = 96, GQA groups, fp16 and fp32 inputs with weights of the same
    dtype, against the oracle."""
    print(f"[li full] reference grid S1={S1} S2={S2} N1={N1} N2={N2} D={D} k={k} B={B} mode={mode} {dtype}",
          flush=True)
    idx = _full_case(B, S1, S2, N1, N2, D, k, mode, dtype, wdtype=dtype, seed=7 + B)
    assert idx.shape == (B, S1, N2, k) and ((idx >= 0) & (idx < S2)).any()


def test_indexer_gqa_fp16_mode0():
    print("[li full] gqa fp16 mode0", flush=True)
    _full_case(1, 6, 700, 32, 2, 64, 64, 0, torch.float16)


def test_indexer_cfg2_sampled_rows():
    """cfg2 (B=2, S1=S2=4096, N1=64, D=128, k=2048, mode 3), 16 sampled rows."""
    print("[li full] cfg2 sampled rows", flush=True)
    rng = np.random.RandomState(3)
    rows = [(int(b), int(s)) for b, s in zip(rng.randint(0, 2, 16), rng.randint(0, 4096, 16))]
    rows += [(0, 0), (1, 4095), (0, 2047), (1, 2048)]
    _full_case(2, 4096, 4096, 64, 1, 128, 2048, 3, torch.bfloat16, rows=rows)


def test_indexer_decode_32k_bench_batch():
    """Decode at 32K context with the bench batch (B=32, S1=1, S2=32768,
    N1=64, D=128, k=2048, mode 3): every row against the oracle."""
    print("[li full] decode 32k, B=32", flush=True)
    _full_case(32, 1, 32768, 64, 1, 128, 2048, 3, torch.bfloat16)


def test_indexer_tnd_matches_bsnd():
    """TND packing (cumulative lengths) gives the per-sequence BSND results."""
    print("[li full] TND vs BSND", flush=True)
    dsa = _api()
    dtype = torch.bfloat16
    lens_q, lens_k = [5, 9], [30, 50]
    N1, D, K = 64, 128, 24
    rng = np.random.RandomState(5)
    qs = [to_dtype_np(rng.randn(L, N1, D).astype(np.float32), dtype) for L in lens_q]
    ks = [to_dtype_np(rng.randn(L, 1, D).astype(np.float32), dtype) for L in lens_k]
    ws = [rng.rand(L, N1).astype(np.float32) for L in lens_q]
    cq, ck = list(np.cumsum(lens_q)), list(np.cumsum(lens_k))
    idx_t, val_t = dsa.lightning_indexer_triton(
        dev(np.concatenate(qs), dtype), dev(np.concatenate(ks), dtype), dev(np.concatenate(ws), torch.float32),
        cq, ck, layout_query="TND", layout_key="TND", sparse_count=K, sparse_mode=3, return_value=True)
    torch.cuda.synchronize()
    idx_t = idx_t.cpu().numpy()
    exp_i, _ = lightning_indexer(np.concatenate(qs), np.concatenate(ks), np.concatenate(ws), cq, ck,
                                 layout_query="TND", layout_key="TND", sparse_count=K, sparse_mode=3)
    # the oracle uses the same scores up to reassociation; these sizes have no near-ties
    np.testing.assert_array_equal(idx_t, exp_i)
    off = 0
    for b in range(2):
        i_b, _ = dsa.lightning_indexer_triton(
            dev(qs[b][None], dtype), dev(ks[b][None], dtype), dev(ws[b][None], torch.float32),
            sparse_count=K, sparse_mode=3)
        np.testing.assert_array_equal(idx_t[off:off + lens_q[b]], i_b.cpu().numpy()[0])
        off += lens_q[b]


@pytest.mark.parametrize("lens_q,extra_k", [
    ([300, 0, 1, 517, 2, 1200], [0, 5, 0, 40, 3, 0]),   # groups of four rows that span sequences, an empty one
    ([4096, 4096], [0, 0]),                              # cfg2 packed
])
def test_indexer_tnd_multirow_matches_per_sequence(lens_q, extra_k):
    """Packed (TND) queries run the multi-row kernel in groups of four
    consecutive rows (a group spanning sequences runs once per sequence):
    bit-identical to each sequence run on its own in BSND."""
    print(f"[li tnd] lens {lens_q}", flush=True)
    dsa = _api()
    dtype = torch.bfloat16
    lens_k = [a + e for a, e in zip(lens_q, extra_k)]
    N1, D, K = 64, 128, 256
    rng = np.random.RandomState(sum(lens_q))
    qs = [to_dtype_np(rng.randn(L, N1, D).astype(np.float32), dtype) for L in lens_q]
    ks = [to_dtype_np(rng.randn(L, 1, D).astype(np.float32), dtype) for L in lens_k]
    ws = [rng.rand(L, N1).astype(np.float32) for L in lens_q]
    cq, ck = [int(x) for x in np.cumsum(lens_q)], [int(x) for x in np.cumsum(lens_k)]
    idx_t, val_t = dsa.lightning_indexer_triton(
        dev(np.concatenate(qs), dtype), dev(np.concatenate(ks), dtype), dev(np.concatenate(ws), torch.float32),
        cq, ck, layout_query="TND", layout_key="TND", sparse_count=K, sparse_mode=3, return_value=True)
    torch.cuda.synchronize()
    idx_t, val_t = idx_t.cpu().numpy(), val_t.float().cpu().numpy()
    off = 0
    for b, L in enumerate(lens_q):
        if L > 0:
            i_b, v_b = dsa.lightning_indexer_triton(
                dev(qs[b][None], dtype), dev(ks[b][None], dtype), dev(ws[b][None], torch.float32),
                sparse_count=K, sparse_mode=3, return_value=True)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(idx_t[off:off + L], i_b.cpu().numpy()[0])
            np.testing.assert_array_equal(val_t[off:off + L].view(np.uint32),
                                          v_b.float().cpu().numpy()[0].view(np.uint32))
        off += L


def test_indexer_guards():
    dsa = _api()
    q = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(1, 4, 3, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(1, 2, 8, device="cuda")
    with pytest.raises(ValueError):
        dsa.lightning_indexer_triton(q, k, w, sparse_count=2)      # N1 % N2
    with pytest.raises(ValueError):
        dsa.lightning_indexer_triton(q, k[:, :, :1], w, block_table=torch.zeros(1, 1, dtype=torch.int32))


def test_indexer_repeatable():
    dsa = _api()
    q, k, w = _inputs(1, 4, 5000, 64, 1, 128, torch.bfloat16)
    a = dsa.lightning_indexer_triton(dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(w, torch.float32),
                                     sparse_count=512, return_value=True)
    b = dsa.lightning_indexer_triton(dev(q, torch.bfloat16), dev(k, torch.bfloat16), dev(w, torch.float32),
                                     sparse_count=512, return_value=True)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ---------------------------------------------------------------------------
# paged key cache (PA_BSND; an extension, the reference rejects block_table)
# ---------------------------------------------------------------------------
def _paged_case(B, page, max_blocks, N2, D, dtype, seed, holes=True):
    """A key cache of random blocks, each batch's table a random choice of
    physical blocks, optionally with -1 holes; returns (cache, table, dense)."""
    from oracle.common import pa_to_bsnd
    rng = np.random.RandomState(seed)
    nblk = B * max_blocks + 3
    cache = to_dtype_np(rng.randn(nblk, page, N2, D).astype(np.float16).astype(np.float32), dtype)
    table = rng.permutation(nblk)[:B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    if holes:
        table[0, 1] = -1
        table[B - 1, max_blocks - 1] = -1
    dense = pa_to_bsnd(cache, table, max_blocks * page)
    return cache, table, dense


# page 24: not a power of two (the kernels divide instead of shifting)
@pytest.mark.parametrize("layout_q,page", [("BSND", 16), ("TND", 16), ("BSND", 24)])
def test_indexer_paged_matches_depaged(layout_q, page):
    print(f"[li paged] query {layout_q} page {page}", flush=True)
    dsa = _api()
    dtype = torch.bfloat16
    B, S1, N1, N2, D, mb, K = 3, 4, 16, 1, 128, 8, 48
    cache, table, dense = _paged_case(B, page, mb, N2, D, dtype, seed=41)
    S2 = mb * page
    q, _, w = _inputs(B, S1, S2, N1, N2, D, dtype, seed=43)
    act_k = [100, S2, 37]
    if layout_q == "TND":
        lens_q = [4, 2, 3]
        cu_q = list(np.cumsum(lens_q))
        qt = np.concatenate([q[b, :lens_q[b]] for b in range(B)])
        wt = np.concatenate([w[b, :lens_q[b]] for b in range(B)])
        args = (dev(qt, dtype), dev(wt, torch.float32))
        kw = dict(actual_seq_lengths_query=cu_q, layout_query="TND")
        # the BSND-on-dense comparison per sequence
        exp = []
        for b in range(B):
            i_b, _ = dsa.lightning_indexer_triton(dev(q[b:b + 1, :lens_q[b]], dtype), dev(dense[b:b + 1], dtype),
                                                   dev(w[b:b + 1, :lens_q[b]], torch.float32),
                                                   actual_seq_lengths_query=[lens_q[b]],
                                                   actual_seq_lengths_key=[act_k[b]], sparse_count=K, sparse_mode=3)
            exp.append(i_b.cpu().numpy()[0])
        exp = np.concatenate(exp)
        ref, _ = lightning_indexer(qt, cache, wt, actual_seq_lengths_query=cu_q, actual_seq_lengths_key=act_k,
                                   layout_query="TND", layout_key="PA_BSND", sparse_count=K, sparse_mode=3,
                                   block_table=table)
    else:
        args = (dev(q, dtype), dev(w, torch.float32))
        kw = dict()
        e, _ = dsa.lightning_indexer_triton(dev(q, dtype), dev(dense, dtype), dev(w, torch.float32),
                                            actual_seq_lengths_key=act_k, sparse_count=K, sparse_mode=3)
        exp = e.cpu().numpy()
        ref, _ = lightning_indexer(q, cache, w, actual_seq_lengths_key=act_k, layout_key="PA_BSND",
                                   sparse_count=K, sparse_mode=3, block_table=table)
    got, val = dsa.lightning_indexer_triton(args[0], dev(cache, dtype), args[1], actual_seq_lengths_key=act_k,
                                            block_table=dev(table, torch.int32), layout_key="PA_BSND",
                                            sparse_count=K, sparse_mode=3, return_value=True, **kw)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    # bit-exact against the BSND kernel on the de-paged keys (same scores, same order)
    np.testing.assert_array_equal(got, exp)
    # and against the oracle up to near-ties of its fp32 scores
    flips = int((got != ref).sum())
    print(f"[li paged] tie flips vs oracle: {flips}", flush=True)
    assert flips <= max(2, got.size // 200)


@pytest.mark.parametrize("page", [64, 48])
def test_indexer_paged_decode_scores(page):
    print(f"[li paged] decode scores page {page}", flush=True)
    dsa = _api()
    from dsa_triton_ascend_amd import _lib
    dtype = torch.bfloat16
    B, N1, D, mb = 4, 64, 128, 16
    cache, table, dense = _paged_case(B, page, mb, 1, D, dtype, seed=47)
    S2 = mb * page
    q, _, w = _inputs(B, 1, S2, N1, 1, D, dtype, seed=49)
    act_k = [S2, 700, 65, 1]
    sc = torch.empty(B, S2, dtype=torch.float32, device="cuda")
    ak = torch.tensor(act_k, dtype=torch.int32, device="cuda")
    qd, cd, wd, td = dev(q, dtype), dev(cache, dtype), dev(w, torch.float32), dev(table, torch.int32)
    lib = _lib.load()
    st = lib.dsa_li_scores_paged(qd.data_ptr(), cd.data_ptr(), wd.data_ptr(), None, ak.data_ptr(), td.data_ptr(),
                                 sc.data_ptr(), B, 1, N1, 1, D, B, cache.shape[0], page, mb, 3,
                                 _lib.LAYOUT["BSND"], _lib.DTYPE_BF16, _lib.DTYPE_FP32, _lib.stream_handle(qd.device))
    _lib.check(st, "dsa_li_scores_paged")
    torch.cuda.synchronize()
    ref = indexer_scores(q, dense, w, [1] * B, act_k, 3).reshape(B, S2)
    got = sc.cpu().numpy()
    assert np.array_equal(np.isinf(got), np.isinf(ref)), "masked entries differ"
    fin = np.isfinite(ref)
    tol = _score_tol(q, dense, w, 1).reshape(B, S2)
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-5 * np.abs(ref[fin]) + tol[fin])
    # the -1 block of batch 0 (keys 64..127) scores exactly zero
    assert np.all(got[0, page:2 * page] == 0.0)


# ---------------------------------------------------------------------------
# the reference's large grid (test_li_triton.py:47-56): (S1, S2) = (4096, 8192)
# and (16384, 16384), N1 = 64, N2 = 1, D = 128, k = 2048, B in {1, 3}, modes
# 0 and 3, fp16 and fp32 inputs (fp16-representable values, weights of the
# input dtype, test_li_triton.py:28-34)
# ---------------------------------------------------------------------------
def _every_row_layout(idx, val, S1, S2, k, mode):
    """Device-side checks of every row: the first min(visible, k) entries are
    distinct in-range indices with non-increasing values, the rest -1 with
    -inf values."""
    B = idx.shape[0]
    s1 = torch.arange(S1, device=idx.device)
    lim = torch.full_like(s1, S2) if mode == 0 else torch.clamp(S2 - S1 + s1 + 1, 0, S2)
    nval = torch.clamp(lim, max=k)                                    # [S1]
    i = idx[:, :, 0].long()                                           # [B, S1, k]
    v = val[:, :, 0].float()
    j = torch.arange(k, device=idx.device)
    want = (j[None, None, :] < nval[None, :, None]).expand(B, S1, k)
    assert torch.equal(i >= 0, want), "valid entries are not exactly the row's first min(visible, k) slots"
    assert bool((i < lim[None, :, None]).all()), "index beyond the row's visible keys"
    assert bool(torch.isneginf(v[~want]).all()), "padding values must be -inf"
    assert not bool(torch.isnan(v).any())
    dec = (v[..., 1:] <= v[..., :-1]) | ~want[..., 1:]
    assert bool(dec.all()), "values are not non-increasing"
    srt = torch.sort(torch.where(want, i, -1 - j[None, None, :]), dim=-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all()), "duplicate index within a row"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("B", [1, 3])
@pytest.mark.parametrize("S1,S2", [(4096, 8192), (16384, 16384)], ids=["4k_8k", "16k_16k"])
def test_indexer_reference_large_grid(S1, S2, B, mode, dtype):
    dsa = _api()
    N1, D, K = 64, 128, 2048
    print(f"[li large grid] S1={S1} S2={S2} B={B} mode={mode} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(1000 * B + 10 * mode + (dtype == torch.float32))
    rnd = lambda *s: torch.randn(*s, generator=g, device="cuda").half().to(dtype)  # noqa: E731
    q, k, w = rnd(B, S1, N1, D), rnd(B, S2, 1, D), rnd(B, S1, N1)
    idx, val = dsa.lightning_indexer_triton(q, k, w, sparse_count=K, sparse_mode=mode, return_value=True)
    torch.cuda.synchronize()
    assert idx.shape == (B, S1, 1, K) and idx.dtype == torch.int32
    _every_row_layout(idx, val, S1, S2, K, mode)
    # sampled rows (edges included) against the oracle's top-k of its fp32 scores
    rng = np.random.RandomState(S1 + B + mode)
    rows = sorted({(b, int(s)) for b in range(B) for s in list(rng.randint(0, S1, 3)) + [0, S1 - 1]})
    kh = k.float().cpu().numpy()
    ih, vh = idx.cpu().numpy(), val.float().cpu().numpy()
    flips = 0
    for b, s in rows:
        qb = q[b, s].float().cpu().numpy()[None, None]                 # [1, 1, N1, D]
        wb = w[b, s].float().cpu().numpy()[None, None]                 # [1, 1, N1]
        lim = S2 if mode == 0 else min(S2, S2 - S1 + s + 1)
        sc = np.full((1, S2), -np.inf, np.float32)
        sc[0, :lim] = indexer_scores(qb, kh[b:b + 1, :lim], wb, [1], [lim], 0)[0, 0, 0]
        a = np.abs(qb[0, 0]) * np.abs(wb[0, 0])[:, None]                # [N1, D]
        tol = 1e-5 * (a.sum(0) @ np.abs(kh[b, :lim, 0]).T).max() + 1e-6 + 1e-5 * np.abs(sc[0, :lim]).max()
        ie, _ = stable_topk(sc, K)
        d = np.nonzero(ih[b, s, 0] != ie[0])[0]
        for jj in d:
            x, y = ih[b, s, 0, jj], ie[0, jj]
            assert x >= 0 and y >= 0, f"row ({b},{s}) slot {jj}: -1 mismatch ({x} vs {y})"
            assert abs(float(sc[0, x]) - float(sc[0, y])) <= 2 * tol, f"row ({b},{s}) slot {jj}: {x} vs {y}"
        flips += len(d)
        ok = ie[0] >= 0
        ev = sc[0, np.maximum(ie[0], 0)]
        ev = ev.astype(np.float16).astype(np.float32) if dtype == torch.float16 else ev
        gv = vh[b, s, 0]
        same = ih[b, s, 0] == ie[0]
        assert np.all(np.abs(gv[ok & same] - ev[ok & same]) <= 2e-3 * np.abs(ev[ok & same]) + 1e-3)
    print(f"  tie flips {flips} of {len(rows) * K} sampled entries", flush=True)
    assert flips <= max(4, len(rows) * K // 500)


# ---------------------------------------------------------------------------
# one-launch scores + top-k against the two launches
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,S1,S2,N1,K,mode,dtype,kind,paged", [
    (2, 2048, 4096, 64, 2048, 3, torch.bfloat16, "random", False),
    (1, 1024, 2048, 64, 512, 0, torch.float16, "random", False),
    (1, 1280, 1536, 48, 2048, 3, torch.bfloat16, "random", False),
    (1, 1024, 1024, 64, 2048, 0, torch.bfloat16, "random", False),   # K > S2: -1 padding
    (1, 1024, 2048, 64, 1024, 3, torch.bfloat16, "zeros", False),    # every score 0: general selection
    (1, 1024, 2048, 64, 700, 0, torch.float16, "ties", False),       # 8 distinct key rows: heavy ties
    (2, 1024, 2048, 64, 2048, 3, torch.bfloat16, "random", True),    # paged keys with a -1 page
], ids=["cfg2_half", "fp16_k512", "g48", "k_over_s2", "zeros", "ties", "paged"])
def test_indexer_fused_matches_two_launches(B, S1, S2, N1, K, mode, dtype, kind, paged):
    """dsa_li_fwd runs scores and top-k in one launch when the rows share key
    tiles (BSND, S1 >= 4, several query rows per batch), D = 128, 33-64 heads
    per key head, S2 <= 4096, K <= 2048 and there are at least four rows per
    CU (every case here on a 256-CU MI355X); the test flag forces the two
    launches.  Indices and values must be bit-identical, including rows
    that need the general selection (all-zero scores) and heavy ties."""
    from dsa_triton_ascend_amd import _lib as L
    dsa = _api()
    lib = L.load()
    print(f"[li fused] B={B} S1={S1} S2={S2} N1={N1} K={K} mode={mode} {dtype} {kind} paged={paged}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(S1 + S2 + K + mode)
    rnd = lambda *s: torch.randn(*s, generator=g, device="cuda").half().to(dtype)  # noqa: E731
    q, k, w = rnd(B, S1, N1, 128), rnd(B, S2, 1, 128), torch.rand(B, S1, N1, generator=g, device="cuda")
    if kind == "zeros":
        q = torch.zeros_like(q)
    elif kind == "ties":
        k = k[:, torch.arange(S2, device="cuda") % 8].contiguous()
    kw = dict(sparse_count=K, sparse_mode=mode, return_value=True)
    if paged:
        page = 64
        nblk = B * S2 // page
        perm = torch.randperm(nblk, generator=g, device="cuda")
        table = perm.to(torch.int32).reshape(B, S2 // page).contiguous()
        cache = torch.empty(nblk, page, 1, 128, dtype=dtype, device="cuda")
        cache[perm.long()] = k.reshape(nblk, page, 1, 128)
        table[1, 3] = -1
        kw.update(block_table=table, layout_key="PA_BSND",
                  actual_seq_lengths_key=torch.full((B,), S2, dtype=torch.int32, device="cuda"))
        k = cache
    outs = []
    for flags in (0, L.TEST_LI_UNFUSED):
        lib.dsa_set_test_flags(flags)
        try:
            idx, val = dsa.lightning_indexer_triton(q, k, w, **kw)
            torch.cuda.synchronize()
        finally:
            lib.dsa_set_test_flags(0)
        outs.append((idx.cpu().numpy(), val.float().cpu().numpy()))
    (i1, v1), (i2, v2) = outs
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(v1.view(np.uint32), v2.view(np.uint32))
    assert (i1 >= -1).all() and (i1 < S2).all()
    if kind == "zeros":
        # all visible scores tie at 0: the first K visible keys in index order
        vis = S2 if mode == 0 else None
        if vis is not None:
            np.testing.assert_array_equal(i1[0, 0, 0, :min(K, S2)], np.arange(min(K, S2)))


@pytest.mark.parametrize("B,S2,N1,D,mode,paged,acts", [
    (16, 8192, 64, 128, 3, False, False),   # multi-token decode shape
    (4, 3000, 32, 128, 0, False, True),     # row lengths: the two rows see different ranges
    (8, 5056, 64, 64, 3, True, False),      # paged keys (79 pages of 64) with a -1 page, D = 64
    (2, 700, 16, 256, 3, False, True),      # D = 256, short rows, act_q hiding the second row
])
def test_indexer_two_rows_per_batch_match_one_row_kernel(B, S2, N1, D, mode, paged, acts):
    """S1 = 2 runs the two-row score kernel (each key fragment serves both
    rows); bit-identical indices and values against the one-row kernel
    (test flag), and the indices against the oracle on every row."""
    from dsa_triton_ascend_amd import _lib as L
    dsa = _api()
    lib = L.load()
    print(f"[li pair] B={B} S2={S2} N1={N1} D={D} mode={mode} paged={paged} acts={acts}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(B + S2 + N1 + D)
    bf = torch.bfloat16
    q = torch.randn(B, 2, N1, D, generator=g, device="cuda").half().to(bf)
    k = torch.randn(B, S2, 1, D, generator=g, device="cuda").half().to(bf)
    w = torch.rand(B, 2, N1, generator=g, device="cuda")
    K = 512
    kw = dict(sparse_count=K, sparse_mode=mode, return_value=True)
    if acts:
        kw.update(actual_seq_lengths_query=[2 if b % 2 == 0 else 1 for b in range(B)],
                  actual_seq_lengths_key=[S2 - 37 * b for b in range(B)])
    kin = k
    if paged:
        page = 64
        nblk = B * S2 // page
        perm = torch.randperm(nblk, generator=g, device="cuda")
        table = perm.to(torch.int32).reshape(B, S2 // page).contiguous()
        cache = torch.empty(nblk, page, 1, D, dtype=bf, device="cuda")
        cache[perm.long()] = k.reshape(nblk, page, 1, D)
        table[1, 3] = -1
        kw.update(block_table=table, layout_key="PA_BSND", actual_seq_lengths_key=[S2] * B)
        kin = cache
    outs = []
    for flags in (0, L.TEST_LI_NO_PAIR):
        lib.dsa_set_test_flags(flags)
        try:
            idx, val = dsa.lightning_indexer_triton(q, kin, w, **kw)
            torch.cuda.synchronize()
        finally:
            lib.dsa_set_test_flags(0)
        outs.append((idx.cpu().numpy(), val.float().cpu().numpy()))
    (i1, v1), (i2, v2) = outs
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(v1.view(np.uint32), v2.view(np.uint32))
    assert (i1 >= -1).all() and (i1 < S2).all()
    if not paged:
        # every row against the oracle (near-tie flips allowed as in the full cases)
        _full_case(B, 2, S2, N1, 1, D, K, mode, bf, act_q=kw.get("actual_seq_lengths_query"),
                   act_k=kw.get("actual_seq_lengths_key"), max_flips=16, seed=B + S2 + N1 + D)
