"""GPU parity of the pre_tokens / next_tokens band mask against the oracle.

The reference rejects any pre_tokens / next_tokens other than INT64_MAX
(sparse_flash_attention_triton.py:531-532, sparse_flash_attention_grad_triton.py:
428-429).  This build honours them as the band of the Ascend FlashAttention
operators: token t of query row s1 is visible iff
diag - pre_tokens <= t <= diag + next_tokens, diag = s1 (sparse_mode 0) or
act_kv - act_q + s1 (sparse_mode 3).  The oracle's band (``oracle.common.
band_bounds``) is pinned on the CPU by an fp64 brute force; here the kernels
are compared with it.

Tolerances as the forward / backward suites: north star rtol 2e-2 / atol
2e-3 against the fp32 oracle (atol scaled by the largest magnitude for the
scatter-added key gradients).  Open sides (INT64_MAX, or any value beyond
every token) are bit-identical to the call without a band.
"""
import numpy as np
import pytest
import torch

from oracle.sfa import sfa_fwd_bsnd, sparse_flash_attention
from oracle.sfa_grad import sfa_bwd_bsnd
from tests.helpers import assert_close, dev, sfa_inputs, sparse_indices, to_dtype_np

pytestmark = pytest.mark.gpu

INT64_MAX = 9223372036854775807
RTOL, ATOL = 2e-2, 2e-3
BF = torch.bfloat16
NAMES = ("dq", "dk", "dv", "dqr", "dkr")


def _fwd(q, k, qr, kr, si, scale, mode, pre, nxt, bs=1, act_q=None, act_k=None, dtype=BF):
    import dsa_triton_ascend_amd as dsa
    out, smax, ssum = dsa.sparse_flash_attention_triton(
        dev(q, dtype), dev(k, dtype), None, dev(si, torch.int32), scale_value=scale,
        actual_seq_lengths_query=act_q, actual_seq_lengths_kv=act_k, query_rope=dev(qr, dtype),
        key_rope=dev(kr, dtype), sparse_block_size=bs, sparse_mode=mode, pre_tokens=pre, next_tokens=nxt,
        return_softmax_lse=True)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), smax.cpu().numpy(), ssum.cpu().numpy()


def _check_fwd(got, ref, what):
    for name, g, e in zip(("out", "softmax_max", "softmax_sum"), got, ref):
        assert_close(g, e, RTOL, ATOL, f"{what} {name}")


BANDS = [(0, 0), (5, 3), (40, INT64_MAX), (INT64_MAX, 7), (3, -2), (-4, 30), (100, 0)]


@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("pre,nxt", BANDS, ids=[f"p{p if p < 10**6 else 'max'}_n{n if n < 10**6 else 'max'}"
                                                for p, n in BANDS])
def test_band_fwd_bsnd(mode, pre, nxt):
    print(f"[band] fwd BSND mode={mode} pre={pre} next={nxt}", flush=True)
    B, S1, S2, N1, D, K = 2, 12, 160, 16, 512, 96
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=3 + mode)
    act_q, act_k = [S1, 9], [S2, 130]
    si = sparse_indices(B, S1, S2, K, 1, mode, act_q=act_q, act_k=act_k, seed=4)
    scale = 1.0 / np.sqrt(D + 64)
    got = _fwd(q, k, qr, kr, si, scale, mode, pre, nxt, act_q=act_q, act_k=act_k)
    ref = sfa_fwd_bsnd(q, k, si, qr, kr, scale, act_q, act_k, 1, mode, True, "float32", positions="kernel",
                       pre_tokens=pre, next_tokens=nxt)
    _check_fwd(got, ref, f"mode {mode} band ({pre},{nxt})")


@pytest.mark.parametrize("mode", [0, 3])
def test_band_open_sides_bit_identical(mode):
    print(f"[band] open sides mode={mode}", flush=True)
    B, S1, S2, N1, D, K = 2, 6, 200, 32, 256, 64
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=9)
    si = sparse_indices(B, S1, S2, K, 1, mode, seed=10)
    base = _fwd(q, k, qr, kr, si, 0.06, mode, INT64_MAX, INT64_MAX)
    for pre, nxt in ((1 << 62, INT64_MAX), (INT64_MAX, 1 << 50), (10**6, 10**6), (S2, S2)):
        got = _fwd(q, k, qr, kr, si, 0.06, mode, pre, nxt)
        for a, b in zip(base, got):
            np.testing.assert_array_equal(a, b)


def test_band_fwd_empty_band_rows_are_zero():
    print("[band] empty band", flush=True)
    B, S1, S2, N1, D, K = 1, 4, 64, 16, 128, 32
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=12)
    si = sparse_indices(B, S1, S2, K, 1, 0, seed=13)
    for pre, nxt in ((-1 << 62, INT64_MAX), (INT64_MAX, -(S2 + 5)), (-3, -4)):
        out, smax, ssum = _fwd(q, k, qr, kr, si, 0.1, 0, pre, nxt)
        assert not out.any() and not smax.any() and not ssum.any(), (pre, nxt)


def test_band_fwd_blockwise():
    print("[band] block-wise ids", flush=True)
    B, S1, S2, N1, D, K, bs = 1, 10, 256, 32, 512, 24, 4
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=14)
    si = sparse_indices(B, S1, S2, K, bs, 3, seed=15)
    scale = 1.0 / np.sqrt(D + 64)
    got = _fwd(q, k, qr, kr, si, scale, 3, 37, 0, bs=bs)
    ref = sparse_flash_attention(q, k, si, scale, qr, kr, sparse_block_size=bs, sparse_mode=3,
                                 return_softmax_lse=True, dtype="float32", pre_tokens=37, next_tokens=0)
    _check_fwd(got, ref, "block-wise")


def test_band_fwd_tnd():
    print("[band] TND", flush=True)
    import dsa_triton_ascend_amd as dsa
    lens = [7, 20, 11]
    N1, D, K = 16, 512, 16
    qs, ks, qrs, krs, sis = [], [], [], [], []
    for i, n in enumerate(lens):
        q, k, qr, kr = sfa_inputs(1, n, n, N1, D, BF, seed=50 + i)
        qs.append(q[0]); ks.append(k[0]); qrs.append(qr[0]); krs.append(kr[0])
        sis.append(sparse_indices(1, n, n, K, 1, 3, seed=60 + i)[0])
    cum = np.cumsum(lens).tolist()
    Q, Kt, QR, KR, SI = (np.concatenate(x) for x in (qs, ks, qrs, krs, sis))
    out, smax, ssum = dsa.sparse_flash_attention_triton(
        dev(Q, BF), dev(Kt, BF), None, dev(SI, torch.int32), scale_value=0.05,
        actual_seq_lengths_query=cum, actual_seq_lengths_kv=cum, query_rope=dev(QR, BF),
        key_rope=dev(KR, BF), layout_query="TND", layout_kv="TND", sparse_mode=3, pre_tokens=6,
        return_softmax_lse=True)
    ref = sparse_flash_attention(Q, Kt, SI, 0.05, QR, KR, actual_seq_lengths_query=cum,
                                 actual_seq_lengths_kv=cum, layout_query="TND", layout_kv="TND",
                                 sparse_mode=3, return_softmax_lse=True, dtype="float32", pre_tokens=6)
    _check_fwd((out.float().cpu().numpy(), smax.cpu().numpy(), ssum.cpu().numpy()), ref, "TND")


@pytest.mark.parametrize("B,N1,K,ctx,page,window", [(2, 128, 2048, 4096, 64, 1500), (4, 64, 512, 1024, 32, 200)])
def test_band_paged_decode_sliding_window(B, N1, K, ctx, page, window):
    """Decode over a paged cache with a sliding window (sparse_mode 3,
    pre_tokens = window): few rows, so the token-split path runs."""
    print(f"[band] paged decode B={B} N1={N1} K={K} ctx={ctx} window={window}", flush=True)
    import dsa_triton_ascend_amd as dsa
    D = 512
    rng = np.random.RandomState(70)
    f = lambda *s: to_dtype_np(rng.randn(*s).astype(np.float32), BF)  # noqa: E731
    nb = ctx // page
    nblk = B * nb + 3
    q, qr = f(B, 1, N1, D), f(B, 1, N1, 64)
    cache, cache_r = f(nblk, page, 1, D), f(nblk, page, 1, 64)
    bt = rng.permutation(nblk)[:B * nb].reshape(B, nb).astype(np.int32)
    act_k = [ctx] + [ctx - 37 * (i + 1) for i in range(B - 1)]
    si = np.stack([np.sort(rng.permutation(act_k[b])[:K]) for b in range(B)]).astype(np.int32).reshape(B, 1, 1, K)
    scale = 1.0 / np.sqrt(D + 64)
    out, smax, ssum = dsa.sparse_flash_attention_triton(
        dev(q, BF), dev(cache, BF), None, dev(si, torch.int32), scale_value=scale,
        block_table=dev(bt, torch.int32), actual_seq_lengths_kv=act_k, query_rope=dev(qr, BF),
        key_rope=dev(cache_r, BF), layout_kv="PA_BSND", sparse_mode=3, pre_tokens=window,
        return_softmax_lse=True, block_size=page)
    torch.cuda.synchronize()
    ref = sparse_flash_attention(q, cache, si, scale, qr, cache_r, block_table=bt, actual_seq_lengths_kv=act_k,
                                 layout_kv="PA_BSND", sparse_mode=3, return_softmax_lse=True, dtype="float32",
                                 pre_tokens=window)
    _check_fwd((out.float().cpu().numpy(), smax.cpu().numpy(), ssum.cpu().numpy()), ref, "paged window")


def _bwd_case(mode, pre, nxt, seed):
    B, S1, S2, N1, D, K = 2, 10, 192, 32, 512, 80
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=seed)
    rng = np.random.RandomState(seed + 1)
    do = to_dtype_np(rng.randn(B, S1, N1, D).astype(np.float32), BF)
    si = sparse_indices(B, S1, S2, K, 1, mode, seed=seed + 2)
    scale = 1.0 / np.sqrt(D + 64)
    act = ([S1] * B, [S2] * B)
    out, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, *act, 1, mode, True, "float32", positions="kernel",
                                   pre_tokens=pre, next_tokens=nxt)
    return q, k, qr, kr, si, do, to_dtype_np(out, BF), smax, ssum, scale, act


@pytest.mark.parametrize("mode,pre,nxt", [(0, 20, 5), (3, 30, INT64_MAX), (3, 8, -2), (0, INT64_MAX, 0)])
@pytest.mark.parametrize("merge", [False, True], ids=["dk_dv", "merged"])
def test_band_bwd(mode, pre, nxt, merge):
    print(f"[band] bwd mode={mode} pre={pre} next={nxt} merge={merge}", flush=True)
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import _sfa_grad
    q, k, qr, kr, si, do, out, smax, ssum, scale, act = _bwd_case(mode, pre, nxt, seed=80 + mode)
    res = _sfa_grad(dev(q, BF), dev(k, BF), dev(k, BF), dev(si, torch.int32), dev(do, BF), dev(out, BF),
                    dev(smax, torch.float32), dev(ssum, torch.float32), scale, dev(qr, BF), dev(kr, BF),
                    None, None, 1, "BSND", mode, pre, nxt, False, merge_kv=merge)
    torch.cuda.synchronize()
    got = [None if r is None else r.float().cpu().numpy() for r in res]
    exp = sfa_bwd_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, *act, 1, mode, "float32",
                       positions="kernel", guard_sum=True, pre_tokens=pre, next_tokens=nxt)
    if merge:
        exp = (exp[0], exp[1] + exp[2], None, exp[3], exp[4])
    for name, g, e in zip(NAMES, got, exp):
        if g is None:
            continue
        tol = ATOL if name in ("dq", "dqr") else ATOL * max(1.0, float(np.abs(e).max()))
        assert_close(g, e, RTOL, tol, f"band bwd {name}")


def test_band_autograd_train():
    """sparse_flash_attention_train with a band: forward and the merged key
    gradient (dk + dv) against the oracle."""
    print("[band] autograd", flush=True)
    import dsa_triton_ascend_amd as dsa
    mode, pre, nxt = 3, 25, INT64_MAX
    q, k, qr, kr, si, do, out_ref, smax, ssum, scale, act = _bwd_case(mode, pre, nxt, seed=90)
    tq, tk, tqr, tkr = (dev(x, BF).requires_grad_(True) for x in (q, k, qr, kr))
    out, _, _ = dsa.sparse_flash_attention_train(tq, tk, dev(si, torch.int32), scale_value=scale, query_rope=tqr,
                                                 key_rope=tkr, sparse_mode=mode, pre_tokens=pre, next_tokens=nxt)
    out.backward(dev(do, BF))
    torch.cuda.synchronize()
    ref = sfa_fwd_bsnd(q, k, si, qr, kr, scale, *act, 1, mode, True, "float32", positions="kernel",
                       pre_tokens=pre, next_tokens=nxt)
    assert_close(out.detach().float().cpu().numpy(), ref[0], RTOL, ATOL, "out")
    exp = sfa_bwd_bsnd(q, k, si, do, out.detach().float().cpu().numpy(), ref[1], ref[2], qr, kr, scale, *act, 1,
                       mode, "float32", positions="kernel", guard_sum=True, pre_tokens=pre, next_tokens=nxt)
    for name, g, e in (("dq", tq.grad, exp[0]), ("dkey", tk.grad, exp[1] + exp[2]), ("dqr", tqr.grad, exp[3]),
                       ("dkr", tkr.grad, exp[4])):
        g = g.float().cpu().numpy()
        tol = ATOL if name in ("dq", "dqr") else ATOL * max(1.0, float(np.abs(e).max()))
        assert_close(g, e, RTOL, tol, f"autograd {name}")
