"""GPU parity of the dense warm-up stage (dense indexer softmax LSE and dense
KL-loss backward) against the oracle.

Inputs follow the reference test (test_dense_loss_backward_triton.py:141-190):
RandomState(42) randn in fp16 (then the I/O dtype), |randn| weights, the
attention statistics of the full causal forward with fp16-rounded scores in
[B, N2, S1, G].  Shapes: the reference's grid (B=1, S1=2, S2=64, N1=N2=32,
D x Nidx1 x D_idx over {128,256,512} x {32,64,128} x {128,256,512}) and its
two extra configs (lines 18-36), plus the DeepSeek-V3.2 MQA shape (N2=1,
N1=128, D=512+64, Nidx1=64, D_idx=128) with short actual lengths.

Expected values: ``oracle.dense_kl`` in fp64.  Tolerances: the LSE at the
reference test's atol 1e-2 / rtol 1e-4 (lines 11-12) and rtol 1e-5 on the
max; dQi / dKi (rounded to the I/O dtype) at rtol 1e-2 with atol 1e-3 of
the tensor's largest magnitude; dW at rtol 1e-3 (fp32 weights) or 1e-2
(stored in fp16 / bf16); the loss at rtol 1e-3.
"""
import math

import numpy as np
import pytest
import torch

from oracle.dense_kl import dense_index_lse, dense_kl_bwd
from tests.helpers import assert_close, to_dtype_np

pytestmark = pytest.mark.gpu

DROPE = 64
GRID = [(1, 2, 64, 32, 32, d, ni, di) for d in (128, 256, 512) for ni in (32, 64, 128) for di in (128, 256, 512)]
EXTRA = [(1, 3, 96, 32, 32, 128, 32, 128), (1, 4, 128, 32, 32, 128, 32, 128)]


def _ids(cases):
    return [f"b{c[0]}s{c[1]}k{c[2]}n{c[3]}g{c[4]}d{c[5]}i{c[6]}di{c[7]}" for c in cases]


def _inputs(B, S1, S2, N1, N2, D, Ni, Di, dtype, w_dtype=None, seed=42):
    rng = np.random.RandomState(seed)
    f = lambda *s: to_dtype_np(rng.randn(*s).astype(np.float16).astype(np.float32), dtype)  # noqa: E731
    q, k = f(B, S1, N1, D), f(B, S2, N2, D)
    qr, kr = f(B, S1, N1, DROPE), f(B, S2, N2, DROPE)
    qi, ki = f(B, S1, Ni, Di), f(B, S2, 1, Di)
    w = to_dtype_np(np.abs(rng.randn(B, S1, Ni)).astype(np.float16).astype(np.float32), w_dtype or dtype)
    return q, k, qr, kr, qi, ki, w


def _stats(q, k, qr, kr, scale, act_q=None, act_k=None, fp16_scores=True):
    """Full causal attention stats [B, N2, S1, G] (test lines 141-173)."""
    B, S1, N1, _ = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    aq = [S1] * B if act_q is None else act_q
    ak = [S2] * B if act_k is None else act_k
    smax = np.full((B, N2, S1, G), -np.inf, np.float32)
    ssum = np.zeros((B, N2, S1, G), np.float32)
    for b in range(B):
        for s1 in range(min(S1, aq[b])):
            L = min(max(ak[b] - aq[b] + s1 + 1, 0), S2)
            if L <= 0:
                continue
            kk = np.concatenate([k[b, :L], kr[b, :L]], -1).astype(np.float64)      # [L, N2, D+Dr]
            qq = np.concatenate([q[b, s1], qr[b, s1]], -1).astype(np.float64)      # [N1, D+Dr]
            s = np.einsum("hd,thd->ht", qq, kk[:, np.arange(N1) // G, :]) * scale
            if fp16_scores:
                s = s.astype(np.float16).astype(np.float64)
            m = s.max(1)
            smax[b, np.arange(N1) // G, s1, np.arange(N1) % G] = m
            ssum[b, np.arange(N1) // G, s1, np.arange(N1) % G] = np.exp(s - m[:, None]).sum(1)
    return smax, ssum


def _dev(x, dt):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device="cuda", dtype=dt)


def _np(t):
    return t.float().cpu().numpy()


def _check(got, exp, what, w_dtype):
    dqi, dki, dw, loss = got
    assert np.isfinite(dqi).all() and np.isfinite(dki).all() and np.isfinite(dw).all()
    for g, e, nm in ((dqi, exp["dQueryIndex"], "dQueryIndex"), (dki, exp["dKeyIndex"], "dKeyIndex")):
        assert_close(g, e, 1e-2, 1e-3 * float(np.abs(e).max()) + 1e-6, f"{what} {nm}")
    rt_w = 1e-3 if w_dtype == torch.float32 else 1e-2
    assert_close(dw, exp["dW"], rt_w, 1e-5 * float(np.abs(exp["dW"]).max()) + 1e-5, f"{what} dW")
    assert_close(loss, exp["loss"], 1e-3, 1e-6, f"{what} loss")


@pytest.mark.parametrize("case", GRID[::3] + EXTRA, ids=_ids(GRID[::3] + EXTRA))
def test_dense_softmax_lse(case):
    """The LSE depends on (Nidx1, D_idx): every pair of the grid, fp16 as the
    reference test."""
    B, S1, S2, N1, N2, D, Ni, Di = case
    print(f"[dense] lse {case}", flush=True)
    import dsa_triton_ascend_amd as dsa
    _, _, _, _, qi, ki, w = _inputs(B, S1, S2, N1, N2, D, Ni, Di, torch.float16)
    cell = dsa.DenseLightningIndexerSoftmaxLseTriton(layout="BSND", sparse_mode=3)
    mx, sm = cell(_dev(qi, torch.float16), _dev(ki, torch.float16), _dev(w, torch.float16))
    torch.cuda.synchronize()
    assert tuple(mx.shape) == (B, 1, S1) and mx.dtype == torch.float32
    em, es = dense_index_lse(qi, ki, w)
    np.testing.assert_allclose(_np(mx), em, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(_np(sm), es, rtol=1e-4, atol=1e-2)


def _run(c, dtype, w_dtype, given_lse, act_q=None, act_k=None):
    import dsa_triton_ascend_amd as dsa
    q, k, qr, kr, qi, ki, w, smax, ssum, scale = c
    dq = lambda x: _dev(x, dtype)  # noqa: E731
    args = (dq(q), dq(k), dq(qi), dq(ki), _dev(w, w_dtype), _dev(smax, torch.float32), _dev(ssum, torch.float32))
    kw = dict(query_rope=dq(qr), key_rope=dq(kr), actual_seq_qlen=act_q, actual_seq_klen=act_k)
    if given_lse:
        mx, sm = dsa.npu_dense_lightning_indexer_softmax_lse_triton(args[2], args[3], args[4], act_q, act_k)
        cell = dsa.DenseLightningIndexerGradKLLossTriton(scale_value=scale, layout="BSND", sparse_mode=3)
        res = cell(*args, mx, sm, **kw)
    else:
        res = dsa.dense_loss_backward_triton(*args, scale_value=scale, layout="BSND", sparse_mode=3, **kw)
    torch.cuda.synchronize()
    for r, ref in zip(res[:3], (qi, ki, w)):
        assert tuple(r.shape) == ref.shape
    assert res[0].dtype == dtype and res[1].dtype == dtype and res[2].dtype == w_dtype
    assert tuple(res[3].shape) == (1,) and res[3].dtype == torch.float32
    return [_np(r) for r in res]


def _case(B, S1, S2, N1, N2, D, Ni, Di, dtype, w_dtype, act_q=None, act_k=None):
    q, k, qr, kr, qi, ki, w = _inputs(B, S1, S2, N1, N2, D, Ni, Di, dtype, w_dtype)
    scale = 1.0 / math.sqrt(D + DROPE)
    smax, ssum = _stats(q, k, qr, kr, scale, act_q, act_k)
    return q, k, qr, kr, qi, ki, w, smax, ssum, scale


@pytest.mark.parametrize("case", GRID + EXTRA, ids=_ids(GRID + EXTRA))
def test_dense_grad_kl_loss(case):
    """The reference's supported-shape grid (test lines 193-251), GQA with
    N2 = N1 = 32, fp16, through the two-stage path (given LSE)."""
    B, S1, S2, N1, N2, D, Ni, Di = case
    print(f"[dense] grad {case}", flush=True)
    c = _case(B, S1, S2, N1, N2, D, Ni, Di, torch.float16, torch.float16)
    got = _run(c, torch.float16, torch.float16, given_lse=True)
    q, k, qr, kr, qi, ki, w, smax, ssum, scale = c
    _check(got, dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale), f"{case}", torch.float16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_dense_compat_path_matches_two_stage(dtype):
    """Without the index statistics the backward computes them with the same
    kernel: bit-identical to passing the LSE op's output (test lines 240-251)."""
    print(f"[dense] compat path {dtype}", flush=True)
    c = _case(1, 4, 128, 32, 32, 128, 32, 128, dtype, torch.float32)
    a = _run(c, dtype, torch.float32, given_lse=True)
    b = _run(c, dtype, torch.float32, given_lse=False)
    for x, y, nm in zip(a, b, ("dQueryIndex", "dKeyIndex", "dW", "loss")):
        assert np.array_equal(x, y), nm
    q, k, qr, kr, qi, ki, w, smax, ssum, scale = c
    _check(a, dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale), f"compat {dtype}", torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_dense_mqa_dsa_shape_with_lengths(dtype):
    """The DeepSeek-V3.2 shape (MQA: N2 = 1, N1 = 128, D = 512 + 64, Nidx1 =
    64, D_idx = 128), two batches with shorter actual lengths: inactive rows
    and a row block with fewer keys than queries."""
    B, S1, S2 = 2, 96, 160
    aq, ak = [96, 40], [160, 30]
    print(f"[dense] MQA DSA shape {dtype}", flush=True)
    c = _case(B, S1, S2, 128, 1, 512, 64, 128, dtype, torch.float32, aq, ak)
    got = _run(c, dtype, torch.float32, given_lse=False, act_q=aq, act_k=ak)
    q, k, qr, kr, qi, ki, w, smax, ssum, scale = c
    exp = dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale, act_q=aq, act_k=ak)
    _check(got, exp, f"MQA {dtype}", torch.float32)
    # rows s1 >= act_q, and keys no valid row sees, get zero gradients
    assert np.all(got[0][1, 40:] == 0) and np.all(got[2][1, 40:] == 0)
    assert np.all(got[1][1, 30:] == 0)


def test_dense_deterministic():
    print("[dense] determinism", flush=True)
    c = _case(1, 64, 256, 64, 1, 256, 64, 128, torch.bfloat16, torch.float32)
    a = _run(c, torch.bfloat16, torch.float32, given_lse=False)
    b = _run(c, torch.bfloat16, torch.float32, given_lse=False)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_dense_guards():
    import dsa_triton_ascend_amd as dsa
    z = lambda *s, dt=torch.bfloat16: torch.zeros(*s, dtype=dt, device="cuda")  # noqa: E731
    q, k, qi, ki = z(1, 2, 4, 128), z(1, 8, 4, 128), z(1, 2, 32, 128), z(1, 8, 1, 128)
    w = z(1, 2, 32, dt=torch.float32)
    st = z(1, 4, 2, 1, dt=torch.float32)
    f = dsa.dense_loss_backward_triton
    with pytest.raises(ValueError):
        f(q, k, qi, ki, w, st, st, layout="TND")
    with pytest.raises(ValueError):
        f(q, k, qi, ki, w, st, st, sparse_mode=0)
    with pytest.raises(ValueError):
        f(q, k, qi, ki, w, st, st, pre_tokens=5)
    with pytest.raises(ValueError):  # Nidx1 outside (32, 64, 128)
        f(q, k, qi[:, :, :16], ki, w[:, :, :16], st, st)
    with pytest.raises(TypeError):
        f(q.float(), k, qi, ki, w, st, st)
    with pytest.raises(ValueError):  # softmax stats not [B, N2, S1, G]
        f(q, k, qi, ki, w, st.reshape(1, 1, 2, 4), st.reshape(1, 1, 2, 4))
    with pytest.raises(ValueError):
        f(q, k, qi, ki, w, st, st, softmax_max_index=z(1, 2, dt=torch.float32))
    with pytest.raises(ValueError):  # index statistics not [B, S1] (or an accepted reshape of it)
        f(q, k, qi, ki, w, st, st, softmax_max_index=z(1, 3, dt=torch.float32),
          softmax_sum_index=z(1, 3, dt=torch.float32))
    with pytest.raises(TypeError):
        f(q, k, qi, ki, w, st, st, softmax_max_index=z(1, 2), softmax_sum_index=z(1, 2))
    with pytest.raises(ValueError):
        dsa.dense_lightning_indexer_softmax_lse_triton(qi, ki, w, layout="TND")
