"""GPU parity of the HIP sparse flash attention backward against the oracle.

Tolerances:
* north star: rtol 2e-2 / atol 2e-3 against the fp32 golden (the oracle's
  backward evaluated without any rounding of the gradients), for dq / dq_rope
  (one row each) and, with atol scaled by the gradient's magnitude, for the
  scatter-added dk / dk_rope / dv: those sum contributions of many query rows
  (the reference scales its own atol the same way, test_sfa_grad_triton.py:
  85-93, 145), so their absolute error grows with the number of rows that
  hit a key; the scale used is max|ref| of the tensor, i.e. atol is 2e-3 of
  the largest gradient entry;
* against the reference golden's dtype-rounded fixtures
  (sparse_flash_attention_grad_numpy.py) the reference's backward tolerance,
  rtol 6e-2 / atol 5e-2 (bf16) and 3e-2 / 2e-2 (fp16)
  (test_sfa_grad_triton.py:85-93).
Inputs out / softmax_max / softmax_sum come from the oracle's fp32 forward
on the same data (rounded to the I/O dtype for out), as the reference tests
derive them (test_sfa_grad_triton.py:104-140).
"""
import glob
import os

import numpy as np
import pytest
import torch

from oracle.sfa import sfa_fwd_bsnd
from oracle.sfa_grad import sfa_bwd_bsnd
from tests.conftest import GOLDEN_DIR
from tests.helpers import assert_close, dev, np_dtype_name, sfa_inputs, sparse_indices, to_dtype_np

pytestmark = pytest.mark.gpu

FIXTURES = sorted(glob.glob(os.path.join(GOLDEN_DIR, "sfa_*.npz")))
REF_TOL = {torch.bfloat16: (6e-2, 5e-2), torch.float16: (3e-2, 2e-2)}
NAMES = ("dq", "dk", "dv", "dqr", "dkr")


def _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, mode, bs=1, act_q=None, act_k=None,
             layout="BSND"):
    import dsa_triton_ascend_amd as dsa
    res = dsa.sparse_flash_attention_grad_triton(
        dev(q, dtype), dev(k, dtype), dev(k, dtype), dev(si, torch.int32), dev(do, dtype), dev(out, dtype),
        dev(smax, torch.float32), dev(ssum, torch.float32), scale_value=scale, query_rope=dev(qr, dtype),
        key_rope=dev(kr, dtype), actual_seq_lengths_query=act_q, actual_seq_lengths_kv=act_k,
        sparse_block_size=bs, layout=layout, sparse_mode=mode)
    torch.cuda.synchronize()
    return [r.float().cpu().numpy() for r in res]


def _check_vs_fp32(got, exp, what):
    for name, g, e in zip(NAMES, got, exp):
        if name in ("dq", "dqr"):
            assert_close(g, e, 2e-2, 2e-3, f"{what} {name}")
        else:
            scale = max(1.0, float(np.abs(e).max()))
            assert_close(g, e, 2e-2, 2e-3 * scale, f"{what} {name}")


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[4:-4] for p in FIXTURES])
def test_bwd_matches_reference_golden_fixture(path):
    f = dict(np.load(path, allow_pickle=False))
    dtype = torch.bfloat16 if str(f["dtype"]) == "bfloat16" else torch.float16
    print(f"[sfa_bwd fixture] {os.path.basename(path)}", flush=True)
    act_q = [int(x) for x in f["act_q"]]
    act_k = [int(x) for x in f["act_k"]]
    got = _bwd_gpu(f["q"], f["k"], f["qr"], f["kr"], f["sparse_indices"], f["d_out"], f["out"],
                   f["softmax_max"], f["softmax_sum"], dtype, float(f["scale"]), int(f["sparse_mode"]),
                   int(f["sparse_block_size"]), act_q, act_k)
    positions = "kernel" if "mid_minus1" in path else "golden"
    exp32 = sfa_bwd_bsnd(f["q"], f["k"], f["sparse_indices"], f["d_out"], f["out"], f["softmax_max"],
                         f["softmax_sum"], f["qr"], f["kr"], float(f["scale"]), f["act_q"], f["act_k"],
                         int(f["sparse_block_size"]), int(f["sparse_mode"]), "float32",
                         positions=positions, guard_sum=True)
    _check_vs_fp32(got, exp32, os.path.basename(path))
    if "mid_minus1" not in path:
        rtol, atol = REF_TOL[dtype]
        S1 = f["q"].shape[1]
        for name, g in zip(NAMES, got):
            scale = S1 if name in ("dk", "dv", "dkr") else 1.0
            assert_close(g, f[name], rtol, atol * scale, f"{name} vs reference golden")


CASES = [
    # B, S1, S2, N1, D, K, bs, mode
    (1, 4, 256, 8, 128, 64, 1, 0),
    (2, 9, 300, 16, 128, 96, 1, 3),
    (1, 6, 512, 128, 512, 128, 1, 3),
    (1, 5, 200, 64, 256, 48, 2, 3),
    (2, 3, 160, 1, 512, 40, 4, 0),
    (1, 40, 64, 32, 128, 64, 1, 3),      # many rows hitting the same keys
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}s{c[1]}k{c[2]}n{c[3]}d{c[4]}K{c[5]}bs{c[6]}m{c[7]}"
                                             for c in CASES])
def test_bwd_random(case, dtype):
    B, S1, S2, N1, D, K, bs, mode = case
    print(f"[sfa_bwd] {case} {dtype}", flush=True)
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, dtype)
    rng = np.random.RandomState(43)
    do = to_dtype_np(rng.randn(B, S1, N1, D).astype(np.float32), dtype)
    act_q = [S1] * B
    act_k = [S2] * B
    if B > 1:
        act_q[1] = max(1, S1 - 2)
        act_k[1] = S2 - 17
    si = sparse_indices(B, S1, S2, K, bs, mode, act_q, act_k)
    scale = 1.0 / np.sqrt(D + 64)
    out, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, act_q, act_k, bs, mode, True, "float32",
                                   positions="kernel")
    out = to_dtype_np(out, dtype)
    got = _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, mode, bs, act_q, act_k)
    exp = sfa_bwd_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, act_q, act_k, bs, mode, "float32",
                       positions="kernel", guard_sum=True)
    _check_vs_fp32(got, exp, f"case {case}")


def test_bwd_tnd_matches_bsnd():
    """TND packing gives the per-sequence BSND gradients."""
    dtype = torch.bfloat16
    N1, D, K = 16, 128, 32
    lens_q, lens_k = [5, 3], [70, 90]
    rng = np.random.RandomState(9)
    parts = []
    for b in range(2):
        q, k, qr, kr = sfa_inputs(1, lens_q[b], lens_k[b], N1, D, dtype, seed=50 + b)
        do = to_dtype_np(rng.randn(1, lens_q[b], N1, D).astype(np.float32), dtype)
        si = sparse_indices(1, lens_q[b], lens_k[b], K, 1, 3)
        scale = 1.0 / np.sqrt(D + 64)
        out, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [lens_q[b]], [lens_k[b]], 1, 3, True,
                                       "float32", positions="kernel")
        out = to_dtype_np(out, dtype)
        ref = _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, 3)
        parts.append((q, k, qr, kr, si, do, out, smax, ssum, ref))
    cat = lambda i, ax=1: np.concatenate([p[i] for p in parts], axis=ax)[0]  # noqa: E731
    q, k, qr, kr, si, do, out = (cat(i) for i in range(7))
    smax = np.concatenate([p[7][0, 0] for p in parts])[None]      # (1, T1, N1)
    ssum = np.concatenate([p[8][0, 0] for p in parts])[None]
    cq, ck = list(np.cumsum(lens_q)), list(np.cumsum(lens_k))
    got = _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, 1.0 / np.sqrt(D + 64), 3,
                   act_q=cq, act_k=ck, layout="TND")
    for i, name in enumerate(NAMES):
        ax = 0
        exp = np.concatenate([p[9][i][0] for p in parts], axis=ax)
        # the same sums in the same fixed-point arithmetic: bit-identical
        np.testing.assert_array_equal(got[i], exp, err_msg=f"TND {name}")


def test_bwd_guards():
    import dsa_triton_ascend_amd as dsa
    z = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16, device="cuda")
    kz = torch.zeros(1, 16, 1, 128, dtype=torch.bfloat16, device="cuda")
    r = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16, device="cuda")
    kr = torch.zeros(1, 16, 1, 64, dtype=torch.bfloat16, device="cuda")
    si = torch.zeros(1, 2, 1, 4, dtype=torch.int32, device="cuda")
    st = torch.zeros(1, 1, 2, 8, device="cuda")
    with pytest.raises(ValueError):
        dsa.sparse_flash_attention_grad_triton(z, kz, kz, si, z, z, st, st, query_rope=r, key_rope=kr,
                                               deterministic=True)
    with pytest.raises(ValueError):
        dsa.sparse_flash_attention_grad_triton(z, kz, kz, si, z, z, st, st, query_rope=r, key_rope=kr,
                                               sparse_mode=1)


def _random_case(case, dtype, seed=0):
    B, S1, S2, N1, D, K, bs, mode = case
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, dtype, seed=42 + seed)
    rng = np.random.RandomState(43 + seed)
    do = to_dtype_np(rng.randn(B, S1, N1, D).astype(np.float32), dtype)
    si = sparse_indices(B, S1, S2, K, bs, mode, seed=7 + seed)
    scale = 1.0 / np.sqrt(D + 64)
    out, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [S1] * B, [S2] * B, bs, mode, True, "float32",
                                   positions="kernel")
    return q, k, qr, kr, si, do, to_dtype_np(out, dtype), smax, ssum, scale, mode, bs


@pytest.mark.parametrize("case", [CASES[1], CASES[2], CASES[5]], ids=["b2s9", "n128d512", "s40"])
def test_bwd_bitwise_repeatable(case):
    """Two calls give bit-identical gradients (no floating-point atomics)."""
    print(f"[sfa_bwd] determinism {case}", flush=True)
    dtype = torch.bfloat16
    q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs = _random_case(case, dtype)
    a = _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, mode, bs)
    b = _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, mode, bs)
    for name, x, y in zip(NAMES, a, b):
        np.testing.assert_array_equal(x, y, err_msg=name)


def _with_flags(flags, fn):
    from dsa_triton_ascend_amd import _lib
    lib = _lib.load()
    lib.dsa_set_test_flags(flags)
    try:
        return fn()
    finally:
        lib.dsa_set_test_flags(0)


@pytest.mark.parametrize("merge", [False, True], ids=["dk_dv", "merged"])
def test_bwd_nan_in_one_row_reaches_exactly_its_tokens(merge):
    """A NaN in one query row's d_out (one head, one column) makes that
    row's dS NaN for the head, so the key gradients of exactly the tokens
    the row attends carry NaN: all dK / dK_rope columns (as in the
    reference), and at least the d_out column in dV.  The records are summed
    in fixed point, which has no NaN: a record slice holding a non-finite
    value is flagged and its token's slice is written as NaN.  Every other
    token's gradients stay finite and equal to a clean run's."""
    from dsa_triton_ascend_amd.sparse_flash_attention import INT64_MAX
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import _sfa_grad
    print(f"[sfa_bwd] NaN row merge={merge}", flush=True)
    dtype = torch.bfloat16
    q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs = _random_case(CASES[5], dtype, seed=5)

    def run(d_out):
        res = _sfa_grad(dev(q, dtype), dev(k, dtype), dev(k, dtype), dev(si, torch.int32), dev(d_out, dtype),
                        dev(out, dtype), dev(smax, torch.float32), dev(ssum, torch.float32), scale, dev(qr, dtype),
                        dev(kr, dtype), None, None, bs, "BSND", mode, INT64_MAX, INT64_MAX, False, merge_kv=merge)
        torch.cuda.synchronize()
        return [None if r is None else r.float().cpu().numpy() for r in res]
    clean = run(do)
    s, h = 30, 3
    bad = do.copy()
    bad[0, s, h, 0] = np.nan
    got = run(bad)
    S2 = k.shape[1]
    n = min(si.shape[-1], S2 - q.shape[1] + s + 1)   # mode 3: the row's visible slots
    toks = si[0, s, 0, :n]
    hit = np.zeros(S2, bool)
    hit[toks[(toks >= 0) & (toks < S2)]] = True
    dk, dk0 = got[1][0, :, 0], clean[1][0, :, 0]
    assert np.isnan(dk[hit]).all(), "dK of the tokens the NaN row attends"
    assert np.isfinite(dk[~hit]).all()
    np.testing.assert_array_equal(dk[~hit], dk0[~hit])
    dkr = got[4][0, :, 0]
    assert np.isnan(dkr[hit]).all() and np.isfinite(dkr[~hit]).all()
    np.testing.assert_array_equal(dkr[~hit], clean[4][0, :, 0][~hit])
    if not merge:
        dv = got[2][0, :, 0]
        assert np.isnan(dv[hit, 0]).all(), "dV's d_out column of the tokens the NaN row attends"
        assert np.isfinite(dv[~hit]).all()
        np.testing.assert_array_equal(dv[~hit], clean[2][0, :, 0][~hit])
    dq = got[0][0]
    assert np.isnan(dq[s, h]).all()
    rows = np.arange(q.shape[1]) != s
    np.testing.assert_array_equal(dq[rows], clean[0][0][rows])


@pytest.mark.parametrize("case", [CASES[1], CASES[3], CASES[5]], ids=["b2s9", "d256bs2", "s40"])
@pytest.mark.parametrize("merge", [False, True], ids=["dk_dv", "merged"])
def test_bwd_row_chunks_match_one_chunk(case, merge):
    """Rows processed in several chunks (a forced small workspace budget; the
    chunks' sums are added in fp32 in chunk order) give the gradients of one
    chunk to fp32 rounding, and match the oracle."""
    from dsa_triton_ascend_amd import _lib
    from dsa_triton_ascend_amd.sparse_flash_attention import INT64_MAX
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import _sfa_grad
    print(f"[sfa_bwd] row chunks {case} merge={merge}", flush=True)
    dtype = torch.bfloat16
    q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs = _random_case(case, dtype, seed=3)

    def run():
        res = _sfa_grad(dev(q, dtype), dev(k, dtype), dev(k, dtype), dev(si, torch.int32), dev(do, dtype),
                        dev(out, dtype), dev(smax, torch.float32), dev(ssum, torch.float32), scale, dev(qr, dtype),
                        dev(kr, dtype), None, None, bs, "BSND", mode, INT64_MAX, INT64_MAX, False, merge_kv=merge)
        torch.cuda.synchronize()
        return [None if r is None else r.float().cpu().numpy() for r in res]
    one = run()
    many = _with_flags(_lib.TEST_SMALL_BWD_CHUNKS, run)
    B, S1 = q.shape[0], q.shape[1]
    exp = sfa_bwd_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, [S1] * B, [k.shape[1]] * B, bs, mode,
                       "float32", positions="kernel", guard_sum=True)
    if merge:
        exp = (exp[0], exp[1] + exp[2], None, exp[3], exp[4])
    for name, a, b, e in zip(NAMES, one, many, exp):
        if a is None:
            continue
        if name in ("dq", "dqr"):
            np.testing.assert_array_equal(a, b, err_msg=name)   # row-local: no chunk sums
        else:
            assert_close(b, a, 1e-2, 1e-3 * max(1.0, float(np.abs(a).max())), f"{name} chunks vs one")
        tol = 2e-3 if name in ("dq", "dqr") else 2e-3 * max(1.0, float(np.abs(e).max()))
        assert_close(b, e, 2e-2, tol, f"{name} chunked vs oracle")


@pytest.mark.parametrize("case", [CASES[0], CASES[2]], ids=["d128", "n128d512"])
def test_bwd_global_address_gather(case):
    """The key gather of key tensors of 2 GiB or more (64-bit addresses)
    forced at small shapes: bit-identical to the buffer-offset gather."""
    from dsa_triton_ascend_amd import _lib
    print(f"[sfa_bwd] global gather {case}", flush=True)
    dtype = torch.bfloat16
    q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs = _random_case(case, dtype, seed=5)
    a = _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, mode, bs)
    b = _with_flags(_lib.TEST_FORCE_GLOBAL_GATHER,
                    lambda: _bwd_gpu(q, k, qr, kr, si, do, out, smax, ssum, dtype, scale, mode, bs))
    for name, x, y in zip(NAMES, a, b):
        np.testing.assert_array_equal(x, y, err_msg=name)


def _grads_both_paths(q, k, qr, kr, si, d_out, out, smax, ssum, scale, mode, bs, dtype, merge):
    from dsa_triton_ascend_amd.sparse_flash_attention import INT64_MAX
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import _sfa_grad
    res = _sfa_grad(dev(q, dtype), dev(k, dtype), dev(k, dtype), dev(si, torch.int32), dev(d_out, dtype),
                    dev(out, dtype), dev(smax, torch.float32), dev(ssum, torch.float32), scale, dev(qr, dtype),
                    dev(kr, dtype), None, None, bs, "BSND", mode, INT64_MAX, INT64_MAX, False, merge_kv=merge)
    torch.cuda.synchronize()
    return [None if r is None else r.float().cpu().numpy() for r in res]


@pytest.mark.parametrize("merge", [False, True], ids=["dk_dv", "merged"])
def test_bwd_underflowing_records_stay_finite(merge):
    """bf16 rows whose d_out is ~2^-130 (bf16 subnormals): every record of
    such a row has a largest magnitude far below 2^-128, where the record's
    scale 2^-e would overflow fp32 unless the exponent is clamped.  The
    tokens that only these rows attend get all-tiny sums.  dK / dV stay
    finite and match the fp32 oracle at the tensor-relative tolerance."""
    print(f"[sfa_bwd] underflowing records merge={merge}", flush=True)
    dtype = torch.bfloat16
    q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs = _random_case(CASES[5], dtype, seed=9)
    S1 = q.shape[1]
    do = do.copy()
    do[0, S1 // 2:] = to_dtype_np(do[0, S1 // 2:] * np.float32(2.0 ** -130), dtype)
    got = _grads_both_paths(q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs, dtype, merge)
    exp = sfa_bwd_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, [S1], [k.shape[1]], bs, mode, "float32",
                       positions="kernel", guard_sum=True)
    if merge:
        got = [got[0], got[1], None, got[3], got[4]]
        exp = [exp[0], exp[1] + exp[2], None, exp[3], exp[4]]
    for name, g, e in zip(NAMES, got, exp):
        if g is None:
            continue
        assert np.isfinite(g).all(), f"{name}: non-finite values"
        assert_close(g, e, 2e-2, 2e-3 * max(1.0, float(np.abs(e).max())), f"underflow {name}")


@pytest.mark.parametrize("merge", [False, True], ids=["dk_dv", "merged"])
def test_bwd_zero_rows_keep_small_gradients_resolved(merge):
    """Half the rows have d_out = 0 (all-zero records) and the other half
    d_out ~ 2^-60: the key gradients are ~2^-63.  An all-zero record slice
    carries the smallest exponent, so it cannot raise the token's largest
    exponent and coarsen the fixed-point sum (with exponent 0 its resolution
    would be about 2^-55, above every value here).  All five gradients match
    the fp32 oracle at 2e-3 of each tensor's own largest entry."""
    print(f"[sfa_bwd] zero rows + tiny gradients merge={merge}", flush=True)
    dtype = torch.bfloat16
    q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs = _random_case(CASES[5], dtype, seed=10)
    S1 = q.shape[1]
    do = to_dtype_np(do * np.float32(2.0 ** -60), dtype)
    do[0, ::2] = 0.0
    got = _grads_both_paths(q, k, qr, kr, si, do, out, smax, ssum, scale, mode, bs, dtype, merge)
    exp = sfa_bwd_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, [S1], [k.shape[1]], bs, mode, "float32",
                       positions="kernel", guard_sum=True)
    if merge:
        got = [got[0], got[1], None, got[3], got[4]]
        exp = [exp[0], exp[1] + exp[2], None, exp[3], exp[4]]
    for name, g, e in zip(NAMES, got, exp):
        if g is None:
            continue
        m = float(np.abs(e).max())
        assert m > 0.0 and m < 2.0 ** -50
        assert_close(g, e, 2e-2, 2e-3 * m, f"tiny gradients {name}")
