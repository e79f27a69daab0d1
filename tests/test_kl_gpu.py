"""GPU parity of the HIP indexer KL-loss backward against the oracle.

Inputs follow the reference test recipe (test_sli_grad_kl_loss_triton.py:
26-70): RandomState(42) randn rounded to fp16 and then to the I/O dtype,
|randn| weights, and its index patterns (random, causal_random, continuous,
repeated, causal_continuous).  The teacher statistics are the dense causal
softmax max / sum over all S2 keys (test_sli_grad_kl_loss_triton.py:79-116;
computed here in fp64 without the fp16 rounding of the scores: the stats
are inputs of the operator, and the oracle is fed the same arrays).

Expected values: ``oracle.kl.kl_loss_bwd`` in fp64 with the device kernel's
semantics (no rounding of dot products, out-of-range targets clamped:
sparse_lightning_indexer_grad_kl_loss_triton.py:63, 300).  Tolerances: the
outputs are computed in fp32 with split-precision MFMA operands, so dW
(fp32 out) and the loss are checked at rtol 1e-3, and dQi / dKi (rounded
to the I/O dtype) at rtol 1e-2 with atol 1e-3 of the tensor's largest
magnitude (their entries span several orders of magnitude; the reference's
own comparison uses atol = rtol = 1e-2 absolute, lines 9-10).  An
absolute floor covers fp32's resolution of dI = softmax(I) - p: both terms
are O(1) probabilities with an ulp near 6e-8, so a row whose exact dI is
~1e-8 (a single slot: sI = 1/(1 + 1e-8) rounds to 1 in fp32) gets dI = 0;
dQi / dKi carry dI times |w|.|ki| (<~ 10), dW carries dI times ReLU scores
(<~ 100).
"""
ATOL_DQ = 1e-6
ATOL_DW = 1e-5
import math

import numpy as np
import pytest
import torch

from oracle.common import pa_to_bsnd
from oracle.kl import kl_loss_bwd, kl_loss_bwd_paged, kl_loss_bwd_tnd
from tests.helpers import assert_close, to_dtype_np

pytestmark = pytest.mark.gpu


def _indices(B, S1, S2, topK, pattern, rng):
    if pattern == "random":
        return rng.randint(0, S2, (B, S1, 1, topK)).astype(np.int32)
    si = np.zeros((B, S1, 1, topK), np.int32)
    if pattern == "causal_random":
        for b in range(B):
            for s1 in range(S1):
                vis = min(max(S2 - S1 + s1 + 1, 1), S2)
                n = min(topK, vis)
                si[b, s1, 0, :n] = rng.choice(vis, size=n, replace=False)
    elif pattern == "continuous":
        si[:] = (np.arange(topK) % S2).astype(np.int32)
    elif pattern == "repeated":
        row = np.zeros(topK, np.int32)
        row[1::2] = min(S2 - 1, 7)
        si[:] = row
    elif pattern == "causal_continuous":
        for s1 in range(S1):
            vis = min(max(S2 - S1 + s1 + 1, 1), S2)
            n = min(topK, vis)
            si[:, s1, 0, :n] = np.arange(n)
    else:
        raise ValueError(pattern)
    return si


def _dense_stats(q, k, qr, kr, scale, act_q, act_k):
    B, S1, N1, _ = q.shape
    S2 = k.shape[1]
    smax = np.full((B, 1, S1, N1), -np.inf, np.float32)
    ssum = np.zeros((B, 1, S1, N1), np.float32)
    for b in range(B):
        for s1 in range(S1):
            if s1 >= act_q[b]:
                continue
            lim = min(max(act_k[b] - act_q[b] + s1 + 1, 0), S2)
            if lim <= 0:
                continue
            s = q[b, s1].astype(np.float64) @ k[b, :lim, 0].T.astype(np.float64)
            if qr is not None:
                s = s + qr[b, s1].astype(np.float64) @ kr[b, :lim, 0].T.astype(np.float64)
            s = s * scale
            m = s.max(1)
            smax[b, 0, s1] = m
            ssum[b, 0, s1] = np.exp(s - m[:, None]).sum(1)
    return smax, ssum


def _gpu_stats(q, k, qr, kr, scale):
    """Dense causal stats (full lengths) in fp32 on the GPU, for shapes where
    the host loop is too slow."""
    B, S1, N1, _ = q.shape
    S2 = k.shape[1]
    smax = np.zeros((B, 1, S1, N1), np.float32)
    ssum = np.zeros((B, 1, S1, N1), np.float32)
    for b in range(B):
        kk = torch.from_numpy(np.concatenate([k[b, :, 0], kr[b, :, 0]], 1)).cuda()
        for r0 in range(0, S1, 64):
            qq = torch.from_numpy(np.concatenate([q[b, r0:r0 + 64], qr[b, r0:r0 + 64]], 2)).cuda()
            s = torch.matmul(qq, kk.T) * scale                      # [rows, N1, S2]
            lim = torch.arange(r0, r0 + qq.shape[0], device="cuda") + (S2 - S1) + 1
            mask = torch.arange(S2, device="cuda")[None, :] >= lim[:, None]
            s = s.masked_fill(mask[:, None, :], float("-inf"))
            m = s.amax(-1)
            smax[b, 0, r0:r0 + qq.shape[0]] = m.cpu().numpy()
            ssum[b, 0, r0:r0 + qq.shape[0]] = torch.exp(s - m[..., None]).sum(-1).cpu().numpy()
    return smax, ssum


def _case(B, S1, S2, N1, D, Ni, topK, dtype, pattern="causal_random", rope=True, w_dtype=torch.float32,
          act_q=None, act_k=None, seed=42, gpu_stats=False, Di=128):
    rng = np.random.RandomState(seed)
    f = lambda *s: to_dtype_np(rng.randn(*s).astype(np.float16).astype(np.float32), dtype)  # noqa: E731
    q, k = f(B, S1, N1, D), f(B, S2, 1, D)
    qr, kr = (f(B, S1, N1, 64), f(B, S2, 1, 64)) if rope else (None, None)
    qi, ki = f(B, S1, Ni, Di), f(B, S2, 1, Di)
    w = to_dtype_np(np.abs(rng.randn(B, S1, Ni)).astype(np.float32), w_dtype)
    si = _indices(B, S1, S2, topK, pattern, rng)
    aq = [S1] * B if act_q is None else list(act_q)
    ak = [S2] * B if act_k is None else list(act_k)
    scale = 1.0 / math.sqrt(D + (64 if rope else 0))
    if gpu_stats:
        smax, ssum = _gpu_stats(q, k, qr, kr, scale)
    else:
        smax, ssum = _dense_stats(q, k, qr, kr, scale, aq, ak)
    return dict(q=q, k=k, qr=qr, kr=kr, qi=qi, ki=ki, w=w, si=si, smax=smax, ssum=ssum, scale=scale,
                aq=aq, ak=ak, dtype=dtype, w_dtype=w_dtype, explicit_len=act_q is not None or act_k is not None)


def _run_gpu(c):
    import dsa_triton_ascend_amd as dsa
    d = lambda x, dt: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(  # noqa: E731
        device="cuda", dtype=dt)
    dt = c["dtype"]
    res = dsa.sparse_lightning_indexer_grad_kl_loss_triton(
        d(c["q"], dt), d(c["k"], dt), d(c["qi"], dt), d(c["ki"], dt), d(c["w"], c["w_dtype"]),
        d(c["si"], torch.int32), d(c["smax"], torch.float32), d(c["ssum"], torch.float32),
        query_rope=d(c["qr"], dt), key_rope=d(c["kr"], dt),
        actual_seq_qlen=c["aq"] if c["explicit_len"] else None,
        actual_seq_klen=c["ak"] if c["explicit_len"] else None, scale_value=c["scale"])
    torch.cuda.synchronize()
    return [r.float().cpu().numpy() for r in res]


def _oracle(c, rows=None):
    B, S1, N1 = c["q"].shape[:3]
    S2 = c["k"].shape[1]
    qr = c["qr"] if c["qr"] is not None else np.zeros((B, S1, N1, 1), np.float32)
    kr = c["kr"] if c["kr"] is not None else np.zeros((B, S2, 1, 1), np.float32)
    return kl_loss_bwd(c["q"], c["k"], qr, kr, c["qi"], c["ki"], c["w"], c["si"], c["smax"], c["ssum"],
                       c["scale"], c["aq"], c["ak"], input_dtype=None, round_dots=False, dki_oob="clamp",
                       rows=rows, compute_dtype=np.float64)


def _check(got, exp, what, w_dtype=torch.float32):
    dqi, dki, dw, loss = got
    rt_w = 1e-3 if w_dtype == torch.float32 else 1e-2  # dW is stored in the weights dtype
    assert np.isfinite(dqi).all() and np.isfinite(dki).all() and np.isfinite(dw).all()
    for g, e, nm in ((dqi, exp["dQueryIndex"], "dQueryIndex"), (dki, exp["dKeyIndex"], "dKeyIndex")):
        assert_close(g, e, 1e-2, 1e-3 * float(np.abs(e).max()) + ATOL_DQ, f"{what} {nm}")
    assert_close(dw, exp["dW"], rt_w, 1e-5 * float(np.abs(exp["dW"]).max()) + ATOL_DW, f"{what} dW")
    assert_close(loss, exp["loss"], 1e-3, 1e-6, f"{what} loss")


CASES = [
    # B, S1, S2, N1, D, Nidx1, topK, pattern
    (1, 4, 256, 32, 512, 8, 128, "causal_random"),
    (1, 8, 192, 16, 128, 16, 64, "random"),
    (1, 6, 96, 8, 256, 12, 64, "continuous"),
    (1, 5, 64, 32, 128, 8, 40, "repeated"),
    (2, 7, 80, 64, 512, 64, 48, "causal_continuous"),
    (1, 33, 33, 128, 512, 64, 32, "causal_random"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}s{c[1]}k{c[2]}n{c[3]}d{c[4]}i{c[5]}K{c[6]}{c[7]}"
                                             for c in CASES])
def test_kl_matches_oracle(case, dtype):
    B, S1, S2, N1, D, Ni, topK, pattern = case
    print(f"[kl_bwd] {case} {dtype}", flush=True)
    c = _case(B, S1, S2, N1, D, Ni, topK, dtype, pattern)
    _check(_run_gpu(c), _oracle(c), f"case {case}")


def test_kl_no_rope_bf16_weights_and_lengths():
    """Missing rope (zeros, API lines 543-546), bf16 weights, shorter actual
    lengths (inactive rows and rows with no visible key)."""
    print("[kl_bwd] no rope / bf16 weights / act lengths", flush=True)
    c = _case(2, 9, 70, 16, 256, 16, 48, torch.bfloat16, "random", rope=False, w_dtype=torch.bfloat16,
              act_q=[9, 6], act_k=[70, 4])
    got = _run_gpu(c)
    exp = _oracle(c)
    _check(got, exp, "no-rope", torch.bfloat16)
    assert np.all(got[0][1, 6:] == 0) and np.all(got[2][1, 6:] == 0)  # rows s1 >= act_q


def test_kl_topk_larger_than_window():
    """topK above the visible window: only the first n slots count (kernel line 107)."""
    print("[kl_bwd] topK > window", flush=True)
    c = _case(1, 6, 40, 16, 128, 8, 64, torch.bfloat16, "causal_random")
    _check(_run_gpu(c), _oracle(c), "topK>window")


@pytest.mark.parametrize("topk", [3072, 6144])
def test_kl_long_topk_smaller_tile_ring(topk):
    """At D = 512 the pass-A tile ring shrinks with topK (the row's arrays
    share the LDS): two buffers up to about 5000 slots (topK 3072 and every
    other test), one above (topK 6144)."""
    print(f"[kl_bwd] topK {topk}, smaller tile ring", flush=True)
    c = _case(1, 4, topk + 56, 16, 512, 64, topk, torch.bfloat16, "causal_random")
    _check(_run_gpu(c), _oracle(c), f"topK={topk}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_kl_many_contributions_per_token(dtype):
    """600 rows over the same 64 tokens ("continuous": every row attends
    tokens 0..63): each token receives 600 contributions, so its dKeyIndex
    sum is split over three waves and finished from the int64 accumulator."""
    print(f"[kl_bwd] 600 contributions per token, {dtype}", flush=True)
    c = _case(1, 600, 64, 16, 128, 16, 64, dtype, "continuous")
    _check(_run_gpu(c), _oracle(c), "600 per token")


def test_kl_deterministic():
    """Two calls give bit-identical outputs (no atomics in the dKi reduction)."""
    print("[kl_bwd] determinism", flush=True)
    c = _case(1, 40, 48, 32, 128, 16, 32, torch.bfloat16, "causal_random")
    a = _run_gpu(c)
    b = _run_gpu(c)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_kl_large_rows_sampled():
    """A larger shape (N1=128, D=512, Nidx1=64, topK=1024): dQi / dW of
    sampled rows against the oracle, loss finite and >= 0."""
    print("[kl_bwd] large sampled", flush=True)
    c = _case(1, 1100, 1100, 128, 512, 64, 1024, torch.bfloat16, "causal_continuous", gpu_stats=True)
    got = _run_gpu(c)
    rows = [(0, 0), (0, 517), (0, 1023), (0, 1099)]
    exp = _oracle(c, rows=rows)
    for _, s1 in rows:
        e = exp["dQueryIndex"][0, s1]
        assert_close(got[0][0, s1], e, 1e-2, 1e-3 * float(np.abs(e).max()) + ATOL_DQ, f"row {s1} dQueryIndex")
        e = exp["dW"][0, s1]
        assert_close(got[2][0, s1], e, 1e-3, 1e-5 * float(np.abs(e).max()) + ATOL_DW, f"row {s1} dW")
    assert np.isfinite(got[1]).all() and float(got[3][0]) >= 0.0


# ---------------------------------------------------------------------------
# the generic path: index shapes outside the fused row kernel (d_idx != 128,
# Nidx1 > 64, topK > 7168), which the reference's loops take
# (sparse_lightning_indexer_grad_kl_loss_triton.py:119-136, 219-262)
# ---------------------------------------------------------------------------
GEN_CASES = [
    # B, S1, S2, N1, D, Nidx1, D_idx, topK, pattern
    (1, 6, 96, 16, 128, 96, 64, 48, "causal_random"),
    (1, 5, 80, 32, 512, 128, 256, 40, "random"),
    (2, 7, 80, 16, 256, 24, 96, 48, "causal_continuous"),
    (1, 4, 64, 8, 128, 8, 40, 32, "repeated"),
    (1, 9, 120, 64, 512, 72, 128, 64, "continuous"),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", GEN_CASES, ids=[f"s{c[1]}k{c[2]}n{c[3]}d{c[4]}i{c[5]}di{c[6]}K{c[7]}{c[8]}"
                                                 for c in GEN_CASES])
def test_kl_generic_index_shapes(case, dtype):
    B, S1, S2, N1, D, Ni, Di, topK, pattern = case
    print(f"[kl_bwd generic] {case} {dtype}", flush=True)
    c = _case(B, S1, S2, N1, D, Ni, topK, dtype, pattern, Di=Di)
    _check(_run_gpu(c), _oracle(c), f"generic {case}")


def test_kl_generic_topk_above_fused_limit():
    """topK = 9000 (> 7168, the fused kernel's limit), no rope, bf16 weights, act lengths."""
    print("[kl_bwd generic] topK 9000", flush=True)
    c = _case(2, 3, 9100, 16, 128, 16, 9000, torch.bfloat16, "causal_random", rope=False,
              w_dtype=torch.bfloat16, act_q=[3, 2], act_k=[9100, 5000])
    _check(_run_gpu(c), _oracle(c), "topK 9000", torch.bfloat16)


def _with_flags(flags, fn):
    from dsa_triton_ascend_amd import _lib
    lib = _lib.load()
    lib.dsa_set_test_flags(flags)
    try:
        return fn()
    finally:
        lib.dsa_set_test_flags(0)


@pytest.mark.parametrize("case", [CASES[0], CASES[4], CASES[5]], ids=["n32d512", "b2n64", "s33n128"])
def test_kl_generic_path_at_fused_shapes(case):
    """The generic path forced at shapes the fused kernel takes: both match
    the oracle and each other (to the tolerance: their fp32 sums differ in
    order and the generic path keeps dS in fp32), and the generic path is
    bit-identical between two runs."""
    from dsa_triton_ascend_amd import _lib
    B, S1, S2, N1, D, Ni, topK, pattern = case
    print(f"[kl_bwd generic forced] {case}", flush=True)
    c = _case(B, S1, S2, N1, D, Ni, topK, torch.bfloat16, pattern)
    fused = _run_gpu(c)
    gen = _with_flags(_lib.TEST_KL_GENERIC, lambda: _run_gpu(c))
    gen2 = _with_flags(_lib.TEST_KL_GENERIC, lambda: _run_gpu(c))
    exp = _oracle(c)
    _check(gen, exp, "generic (forced)")
    for name, a, b in zip(("dQueryIndex", "dKeyIndex", "dW", "loss"), gen, fused):
        assert_close(a, b, 1e-2, 2e-3 * float(np.abs(b).max()) + 1e-5, f"generic vs fused {name}")
    for a, b in zip(gen, gen2):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("generic", [False, True], ids=["fused", "generic"])
def test_kl_nan_weight_poisons_exactly_its_tokens(generic):
    """A NaN weight in one query row makes that row's dS NaN, so the dKi of
    exactly the tokens the row attends is NaN (as in the reference, whose
    fp32 atomics add the NaN in); every other dKi entry stays finite and
    matches the clean run.  The reduction sums in fixed point, where NaN has
    no representation: a non-finite contribution marks its row maximum
    infinite, which the reduction turns into NaN for the row's tokens."""
    from dsa_triton_ascend_amd import _lib
    print(f"[kl_bwd] NaN weight generic={generic}", flush=True)
    c = _case(1, 24, 96, 32, 128, 16, 48, torch.bfloat16, "causal_random")
    run = (lambda: _with_flags(_lib.TEST_KL_GENERIC, lambda: _run_gpu(c))) if generic else (lambda: _run_gpu(c))
    clean = run()
    s = 20
    c["w"] = c["w"].copy()
    c["w"][0, s, 3] = np.nan
    got = run()
    dki, dki0 = got[1][0, :, 0], clean[1][0, :, 0]
    S2 = c["k"].shape[1]
    n = min(48, S2 - 24 + s + 1)
    hit = np.zeros(S2, bool)
    hit[np.clip(c["si"][0, s, 0, :n], 0, S2 - 1)] = True
    assert np.isnan(dki[hit]).all(), "tokens attended by the NaN row must be NaN"
    assert np.isfinite(dki[~hit]).all(), "tokens not attended by the NaN row must stay finite"
    np.testing.assert_array_equal(dki[~hit], dki0[~hit])


def test_kl_guards():
    import dsa_triton_ascend_amd as dsa
    z = lambda *s: torch.zeros(*s, dtype=torch.bfloat16, device="cuda")  # noqa: E731
    q, k, qi, ki = z(1, 2, 4, 128), z(1, 8, 1, 128), z(1, 2, 4, 128), z(1, 8, 1, 128)
    w = torch.zeros(1, 2, 4, device="cuda")
    si = torch.zeros(1, 2, 1, 4, dtype=torch.int32, device="cuda")
    st = torch.zeros(1, 1, 2, 4, device="cuda")
    with pytest.raises(ValueError):
        dsa.sparse_lightning_indexer_grad_kl_loss_triton(q, k, qi, ki, w, si, st, st, layout="BNSD")
    with pytest.raises(ValueError):  # TND needs cumulative lengths
        dsa.sparse_lightning_indexer_grad_kl_loss_triton(q[0], k[0], qi[0], ki[0], w[0], si[0], st, st,
                                                         layout="TND")
    with pytest.raises(ValueError):
        dsa.sparse_lightning_indexer_grad_kl_loss_triton(q, k, qi, ki, w, si, st, st, sparse_mode=0)
    with pytest.raises(AssertionError):
        dsa.sparse_lightning_indexer_grad_kl_loss_triton(q, k, qi, ki, w, si.reshape(1, 1, 2, 4), st, st)


# ---------------------------------------------------------------------------
# packed (TND) rows and a paged key cache: extensions over the reference's
# BSND-only API (sparse_lightning_indexer_grad_kl_loss_triton.py:534-535)
# ---------------------------------------------------------------------------
def _dev(x, dt):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device="cuda", dtype=dt)


def _tnd_case(lq, lk, N1, D, Ni, topK, dtype, seed=7):
    """Per-batch BSND problems (B = 1, S1 = lq[b], S2 = lk[b]) packed along
    the token axis.  Indices of batch b are drawn from [0, lk[b]) and a few
    are pushed past lk[b] (clamped to the batch's last key)."""
    parts = []
    for b, (nq, nk) in enumerate(zip(lq, lk)):
        c = _case(1, nq, max(nk, 1), N1, D, Ni, topK, dtype, "causal_random", seed=seed + b)
        if nk == 0:
            c["k"], c["kr"], c["ki"] = (x[:, :0] for x in (c["k"], c["kr"], c["ki"]))
        c["si"][0, :, 0, -1] = nk + 5  # out of the batch's range: clamped
        parts.append(c)
    cat = lambda key: np.concatenate([p[key][0] for p in parts], 0)  # noqa: E731
    return dict(q=cat("q"), k=cat("k"), qr=cat("qr"), kr=cat("kr"), qi=cat("qi"), ki=cat("ki"), w=cat("w"),
                si=cat("si"), smax=np.concatenate([p["smax"][0, 0] for p in parts], 0)[None],
                ssum=np.concatenate([p["ssum"][0, 0] for p in parts], 0)[None], scale=parts[0]["scale"],
                dtype=dtype, cu_q=np.cumsum(lq).astype(np.int32), cu_k=np.cumsum(lk).astype(np.int32))


def _run_tnd(t):
    import dsa_triton_ascend_amd as dsa
    dt = t["dtype"]
    res = dsa.sparse_lightning_indexer_grad_kl_loss_triton(
        _dev(t["q"], dt), _dev(t["k"], dt), _dev(t["qi"], dt), _dev(t["ki"], dt), _dev(t["w"], torch.float32),
        _dev(t["si"], torch.int32), _dev(t["smax"], torch.float32), _dev(t["ssum"], torch.float32),
        query_rope=_dev(t["qr"], dt), key_rope=_dev(t["kr"], dt), actual_seq_qlen=t["cu_q"].tolist(),
        actual_seq_klen=t["cu_k"].tolist(), scale_value=t["scale"], layout="TND")
    torch.cuda.synchronize()
    return [r.float().cpu().numpy() for r in res]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_kl_tnd_matches_oracle(dtype):
    """Ragged packed batches (one with no query rows, one with fewer keys
    than queries) against the TND oracle."""
    lq, lk = [5, 0, 9, 3], [40, 12, 64, 2]
    print(f"[kl_bwd] TND lq={lq} lk={lk} {dtype}", flush=True)
    t = _tnd_case(lq, lk, 32, 256, 16, 48, dtype)
    got = _run_tnd(t)
    exp = kl_loss_bwd_tnd(t["q"], t["k"], t["qr"], t["kr"], t["qi"], t["ki"], t["w"], t["si"], t["smax"],
                          t["ssum"], t["scale"], t["cu_q"], t["cu_k"], compute_dtype=np.float64)
    assert got[0].shape == t["qi"].shape and got[1].shape == t["ki"].shape and got[2].shape == t["w"].shape
    _check(got, exp, "TND")


def test_kl_tnd_equal_lengths_bit_exact_to_bsnd():
    """TND with equal per-batch lengths is the BSND problem with its batch
    axis flattened: every output is bit-identical to the BSND call."""
    print("[kl_bwd] TND == BSND bit-exact", flush=True)
    B, S1, S2 = 3, 6, 50
    c = _case(B, S1, S2, 16, 128, 8, 32, torch.bfloat16, "causal_random")
    bsnd = _run_gpu(c)
    t = dict(q=c["q"].reshape(B * S1, *c["q"].shape[2:]), k=c["k"].reshape(B * S2, 1, -1),
             qr=c["qr"].reshape(B * S1, *c["qr"].shape[2:]), kr=c["kr"].reshape(B * S2, 1, -1),
             qi=c["qi"].reshape(B * S1, *c["qi"].shape[2:]), ki=c["ki"].reshape(B * S2, 1, -1),
             w=c["w"].reshape(B * S1, -1), si=c["si"].reshape(B * S1, 1, -1), smax=c["smax"], ssum=c["ssum"],
             scale=c["scale"], dtype=torch.bfloat16, cu_q=np.cumsum([S1] * B).astype(np.int32),
             cu_k=np.cumsum([S2] * B).astype(np.int32))
    tnd = _run_tnd(t)
    for a, b, nm in zip(bsnd, tnd, ("dQueryIndex", "dKeyIndex", "dW", "loss")):
        assert np.array_equal(a.reshape(-1), b.reshape(-1)), nm


def _paged_case(B, S1, N1, D, Ni, topK, page, max_blocks, nblk, table, act_k, dtype, seed=11):
    rng = np.random.RandomState(seed)
    f = lambda *s: to_dtype_np(rng.randn(*s).astype(np.float16).astype(np.float32), dtype)  # noqa: E731
    q, qr, qi = f(B, S1, N1, D), f(B, S1, N1, 64), f(B, S1, Ni, 128)
    kc, krc, kic = f(nblk, page, 1, D), f(nblk, page, 1, 64), f(nblk, page, 1, 128)
    w = np.abs(rng.randn(B, S1, Ni)).astype(np.float32)
    S2 = max_blocks * page
    si = np.zeros((B, S1, 1, topK), np.int32)
    for b in range(B):
        for s1 in range(S1):
            vis = max(act_k[b] - S1 + s1 + 1, 1)
            n = min(topK, vis)
            si[b, s1, 0, :n] = rng.choice(vis, size=n, replace=False)
    scale = 1.0 / math.sqrt(D + 64)
    kd, krd = pa_to_bsnd(kc, table, S2), pa_to_bsnd(krc, table, S2)
    smax, ssum = _dense_stats(q, kd, qr, krd, scale, [S1] * B, act_k)
    return dict(q=q, qr=qr, qi=qi, kc=kc, krc=krc, kic=kic, w=w, si=si, smax=smax, ssum=ssum, scale=scale,
                table=np.asarray(table, np.int32), act_k=list(act_k), dtype=dtype, S2=S2)


def _run_paged(c):
    import dsa_triton_ascend_amd as dsa
    dt = c["dtype"]
    res = dsa.sparse_lightning_indexer_grad_kl_loss_triton(
        _dev(c["q"], dt), _dev(c["kc"], dt), _dev(c["qi"], dt), _dev(c["kic"], dt), _dev(c["w"], torch.float32),
        _dev(c["si"], torch.int32), _dev(c["smax"], torch.float32), _dev(c["ssum"], torch.float32),
        query_rope=_dev(c["qr"], dt), key_rope=_dev(c["krc"], dt), actual_seq_klen=c["act_k"],
        scale_value=c["scale"], block_table=_dev(c["table"], torch.int32))
    torch.cuda.synchronize()
    return [r.float().cpu().numpy() for r in res]


def _paged_oracle(c):
    return kl_loss_bwd_paged(c["q"], c["kc"], c["qr"], c["krc"], c["qi"], c["kic"], c["w"], c["si"],
                             c["smax"], c["ssum"], c["scale"], c["table"], c["act_k"], compute_dtype=np.float64)


def test_kl_paged_matches_oracle_and_bsnd():
    """Disjoint pages in shuffled order, a -1 page inside a batch's visible
    range (zero key rows, no gradient) and unused cache pages (zero
    gradient).  Against the oracle, and bit-exact against the BSND kernel on
    the de-paged cache (dKi gathered back to the pages)."""
    print("[kl_bwd] paged", flush=True)
    page, max_blocks, nblk = 16, 5, 12
    table = [[7, 2, 10, -1, 4], [3, 11, 0, 5, 9]]
    act_k = [80, 70]
    c = _paged_case(2, 6, 16, 128, 8, 40, page, max_blocks, nblk, table, act_k, torch.bfloat16)
    got = _run_paged(c)
    assert got[1].shape == c["kic"].shape
    _check(got, _paged_oracle(c), "paged")
    # the same problem de-paged, through the BSND kernel
    S2 = c["S2"]
    bc = dict(q=c["q"], k=pa_to_bsnd(c["kc"], table, S2), qr=c["qr"], kr=pa_to_bsnd(c["krc"], table, S2),
              qi=c["qi"], ki=pa_to_bsnd(c["kic"], table, S2), w=c["w"], si=c["si"], smax=c["smax"],
              ssum=c["ssum"], scale=c["scale"], aq=[6, 6], ak=act_k, dtype=torch.bfloat16,
              w_dtype=torch.float32, explicit_len=True)
    ref = _run_gpu(bc)
    for i, nm in ((0, "dQueryIndex"), (2, "dW"), (3, "loss")):
        assert np.array_equal(got[i], ref[i]), nm
    used = set()
    for b in range(2):
        for i, blk in enumerate(table[b]):
            if blk >= 0:
                assert np.array_equal(got[1][blk], ref[1][b, i * page:(i + 1) * page]), f"page {blk}"
                used.add(blk)
    for blk in range(nblk):
        if blk not in used:
            assert np.all(got[1][blk] == 0), f"unused page {blk}"


def test_kl_paged_shared_prefix_page():
    """Two batches share their first page (a common prefix): its gradient
    is the sum over both batches' slots."""
    print("[kl_bwd] paged shared page", flush=True)
    table = [[4, 1, 6], [4, 0, 2]]
    c = _paged_case(2, 5, 8, 128, 8, 24, 16, 3, 8, table, [48, 40], torch.float16, seed=3)
    _check(_run_paged(c), _paged_oracle(c), "paged shared")
