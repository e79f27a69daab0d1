"""Pins for the SFA forward/backward oracle (CPU only).

What pins what:
* ``round_bf16``: torch's own fp32->bf16 cast (a library routine).
* ``sfa_fwd_bsnd`` / ``sfa_bwd_bsnd``: the committed fixtures written by the
  reference's numpy goldens (tests/golden/make_fixtures.py), an independent
  fp64 brute force with scalar loops, closed forms, permutation invariance,
  central finite differences of the fp64 forward (as verify_grad_algo.py:42-88
  does for the golden), and the delta identity dO.O = sum_p P.dP.
* layout helpers: PA == de-paged BSND, TND == per-sequence BSND,
  block-wise == expanded token-wise.
* band mask (pre_tokens / next_tokens, which the reference rejects): an fp64
  brute force that tests each key position's offset from the diagonal, open
  sides == no band, the diagonal-only closed form, empty bands, and finite
  differences of the banded forward for the banded backward.
"""
import glob
import math
import os

import numpy as np
import pytest

from oracle.common import (round_bf16, gather_positions, kernel_positions,
                           expand_block_indices, pa_to_bsnd, tnd_to_bsnd)
from oracle.sfa import sfa_fwd_bsnd, sparse_flash_attention
from oracle.sfa_grad import sfa_bwd_bsnd
from tests.conftest import GOLDEN_DIR

FIXTURES = sorted(glob.glob(os.path.join(GOLDEN_DIR, "sfa_*.npz")))


def _bf16_ulps(a, b):
    """Distance in bf16 units of the larger magnitude (for bf16-rounded outputs)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    mag = np.maximum(np.abs(a), np.abs(b))
    ulp = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7), 1e-30)
    return np.abs(a - b) / ulp


def test_round_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.RandomState(0)
    x = np.concatenate([rng.randn(100000).astype(np.float32) * 10.0 ** rng.randint(-6, 6, 100000),
                        np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 3.0e38, 1e-40], np.float32)])
    # include exact ties (low 16 bits == 0x8000) in both parity cases
    ties = (np.arange(1000, dtype=np.uint32) << 16) | np.uint32(0x3F808000)
    x = np.concatenate([x.astype(np.float32), ties.view(np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_bf16(x).view(np.uint32), ref.view(np.uint32))


def _load(path):
    z = np.load(path, allow_pickle=False)
    return {k: z[k] for k in z.files}


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[4:-4] for p in FIXTURES])
def test_fwd_oracle_matches_reference_golden_fixture(path):
    f = _load(path)
    out, smax, ssum = sfa_fwd_bsnd(
        f["q"], f["k"], f["sparse_indices"], f["qr"], f["kr"], float(f["scale"]),
        f["act_q"], f["act_k"], sparse_block_size=int(f["sparse_block_size"]),
        sparse_mode=int(f["sparse_mode"]), return_lse=True, dtype=str(f["dtype"]),
        positions="golden")
    np.testing.assert_allclose(smax, f["softmax_max"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(ssum, f["softmax_sum"], rtol=1e-5, atol=1e-6)
    # the oracle evaluates heads as one matrix product; fp32 summation order
    # may move a rounded probability or output across a rounding boundary:
    # allow one unit of the I/O dtype at the row's magnitude, on under 1% of
    # the elements
    ref = f["out"]
    unit = 2.0 ** -8 if str(f["dtype"]) == "bfloat16" else 2.0 ** -11
    row_mag = np.abs(ref).max(axis=-1, keepdims=True)
    err = np.abs(out - ref)
    assert np.all(err <= unit * row_mag + 1e-7)
    assert (err > 0).mean() < 0.01


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[4:-4] for p in FIXTURES])
def test_bwd_oracle_matches_reference_golden_fixture(path):
    f = _load(path)
    g = sfa_bwd_bsnd(
        f["q"], f["k"], f["sparse_indices"], f["d_out"], f["out"], f["softmax_max"],
        f["softmax_sum"], f["qr"], f["kr"], float(f["scale"]), f["act_q"], f["act_k"],
        sparse_block_size=int(f["sparse_block_size"]), sparse_mode=int(f["sparse_mode"]),
        dtype=str(f["dtype"]), positions="golden")
    for name, mine in zip(("dq", "dk", "dv", "dqr", "dkr"), g):
        ref = f[name]
        tol = 2.0 ** -7 if str(f["dtype"]) == "bfloat16" else 2.0 ** -10
        err = np.abs(mine - ref)
        bound = np.maximum(np.abs(ref), np.abs(mine)) * tol * 1.01 + 1e-6
        assert np.all(err <= bound), name


def test_kernel_masking_agrees_with_golden_scan_on_front_valid_rows():
    """All fixtures except the mid -1 one are front-valid: both rules agree."""
    for path in FIXTURES:
        f = _load(path)
        si = f["sparse_indices"]
        bs = int(f["sparse_block_size"])
        mode = int(f["sparse_mode"])
        B, S1 = si.shape[0], si.shape[1]
        same = True
        for b in range(B):
            aq, ak = int(f["act_q"][b]), int(f["act_k"][b])
            for s1 in range(min(S1, aq)):
                thr = ak if mode == 0 else ak - aq + s1 + 1
                if thr <= 0:
                    continue
                g = gather_positions(si[b, s1, 0], bs, thr, ak)
                kk = kernel_positions(si[b, s1, 0], bs, thr, ak)
                same &= g == kk
        if "mid_minus1" in path:
            assert not same
        else:
            assert same, path


# ---------------------------------------------------------------------------
# independent fp64 brute force (scalar loops, math.exp)
# ---------------------------------------------------------------------------
def _brute_fwd(q, k, qr, kr, si, scale, aq, ak, mode):
    B, S1, N1, D = q.shape
    out = np.zeros((B, S1, N1, D))
    mx = np.zeros((B, 1, S1, N1))
    sm = np.zeros((B, 1, S1, N1))
    for b in range(B):
        for s1 in range(aq[b]):
            thr = ak[b] if mode == 0 else ak[b] - aq[b] + s1 + 1
            toks = [int(t) for t in si[b, s1, 0] if t != -1 and t < thr and t < ak[b]]
            if thr <= 0 or not toks:
                continue
            for h in range(N1):
                sc = []
                for t in toks:
                    acc = 0.0
                    for d in range(D):
                        acc += float(q[b, s1, h, d]) * float(k[b, t, 0, d])
                    for d in range(qr.shape[-1]):
                        acc += float(qr[b, s1, h, d]) * float(kr[b, t, 0, d])
                    sc.append(acc * scale)
                m = max(sc)
                ex = [math.exp(s - m) for s in sc]
                z = sum(ex)
                mx[b, 0, s1, h] = m
                sm[b, 0, s1, h] = z
                for d in range(D):
                    out[b, s1, h, d] = sum(e / z * float(k[b, t, 0, d]) for e, t in zip(ex, toks))
    return out, mx, sm


@pytest.mark.parametrize("mode", [0, 3])
def test_fwd_oracle_fp64_matches_brute_force(mode):
    rng = np.random.RandomState(3)
    B, S1, S2, N1, D, Dr, K = 2, 3, 12, 2, 8, 4, 5
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    si = np.full((B, S1, 1, K), -1, np.int32)
    for b in range(B):
        for s in range(S1):
            si[b, s, 0, :4] = np.sort(rng.choice(S2 if mode == 0 else S2 - S1 + s + 1, 4, replace=False))
    aq, ak = [S1, S1 - 1], [S2, S2 - 2]
    out, mx, sm = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, aq, ak, sparse_mode=mode,
                               positions="kernel", compute_dtype=np.float64)
    bo, bm, bs = _brute_fwd(q, k, qr, kr, si, 0.3, aq, ak, mode)
    np.testing.assert_allclose(out, bo, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mx, bm, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sm, bs, rtol=1e-12, atol=1e-12)


def test_fwd_closed_forms():
    rng = np.random.RandomState(5)
    B, S1, S2, N1, D, Dr = 1, 3, 16, 4, 8, 4
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    aq, ak = [S1], [S2]
    # (i) one valid index: out = v_idx, max = score, sum = 1
    si = np.full((B, S1, 1, 4), -1, np.int32); si[0, :, 0, 0] = [3, 7, 11]
    out, mx, sm = sfa_fwd_bsnd(q, k, si, qr, kr, 0.5, aq, ak, sparse_mode=0, compute_dtype=np.float64)
    for s1, t in enumerate([3, 7, 11]):
        np.testing.assert_allclose(out[0, s1], np.broadcast_to(k[0, t, 0], (N1, D)), rtol=1e-13)
        np.testing.assert_allclose(sm[0, 0, s1], 1.0)
        np.testing.assert_allclose(mx[0, 0, s1], 0.5 * (q[0, s1] @ k[0, t, 0] + qr[0, s1] @ kr[0, t, 0]))
    # (ii) identical K rows: out = that row for any q
    k2 = np.broadcast_to(k[:, :1], k.shape).copy(); kr2 = np.broadcast_to(kr[:, :1], kr.shape).copy()
    si = np.tile(np.arange(6, dtype=np.int32), (B, S1, 1, 1))
    out, _, sm = sfa_fwd_bsnd(q, k2, si, qr, kr2, 0.5, aq, ak, sparse_mode=0, compute_dtype=np.float64)
    np.testing.assert_allclose(out[0], np.broadcast_to(k2[0, 0, 0], (S1, N1, D)), rtol=1e-13)
    np.testing.assert_allclose(sm, 6.0)
    # (iii) q = 0: out = mean of gathered v, max 0, sum n
    out, mx, sm = sfa_fwd_bsnd(np.zeros_like(q), k, si, np.zeros_like(qr), kr, 0.5, aq, ak,
                               sparse_mode=0, compute_dtype=np.float64)
    np.testing.assert_allclose(out[0, 0, 0], k[0, :6, 0].mean(axis=0), rtol=1e-13)
    np.testing.assert_allclose(mx, 0.0); np.testing.assert_allclose(sm, 6.0)


def test_fwd_duplicates_count_twice_and_order_invariant():
    rng = np.random.RandomState(6)
    B, S1, S2, N1, D, Dr = 1, 1, 10, 3, 8, 4
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    a = np.array([[[[1, 4, 4, 9]]]], np.int32)
    b = np.array([[[[9, 4, 1, 4]]]], np.int32)
    oa, ma, sa = sfa_fwd_bsnd(q, k, a, qr, kr, 0.4, [1], [S2], sparse_mode=0, positions="kernel", compute_dtype=np.float64)
    ob, mb, sb = sfa_fwd_bsnd(q, k, b, qr, kr, 0.4, [1], [S2], sparse_mode=0, positions="kernel", compute_dtype=np.float64)
    np.testing.assert_allclose(oa, ob, rtol=1e-13); np.testing.assert_allclose(sa, sb, rtol=1e-13)
    # weight of token 4 is doubled relative to a single occurrence
    s = 0.4 * (q[0, 0] @ k[0, :, 0].T + qr[0, 0] @ kr[0, :, 0].T)
    w = np.exp(s[:, [1, 4, 4, 9]] - ma[0, 0, 0][:, None])
    np.testing.assert_allclose(sa[0, 0, 0], w.sum(axis=1), rtol=1e-13)


def test_fwd_mode3_hidden_rows_are_zero():
    rng = np.random.RandomState(8)
    B, S1, S2, N1, D, Dr = 1, 6, 3, 2, 8, 4
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    si = np.tile(np.arange(3, dtype=np.int32), (B, S1, 1, 1))
    out, mx, sm = sfa_fwd_bsnd(q, k, si, qr, kr, 0.4, [S1], [S2], sparse_mode=3)
    # rows s1 < act_q - act_k = 3 see nothing
    assert np.all(out[0, :3] == 0) and np.all(mx[0, 0, :3] == 0) and np.all(sm[0, 0, :3] == 0)
    assert np.all(sm[0, 0, 3:] > 0)


# ---------------------------------------------------------------------------
# layout equivalences
# ---------------------------------------------------------------------------
def _rand_case(rng, B, S1, S2, N1, D, K, mode):
    q = round_bf16(rng.randn(B, S1, N1, D).astype(np.float32))
    k = round_bf16(rng.randn(B, S2, 1, D).astype(np.float32))
    qr = round_bf16(rng.randn(B, S1, N1, 64).astype(np.float32))
    kr = round_bf16(rng.randn(B, S2, 1, 64).astype(np.float32))
    si = np.full((B, S1, 1, K), -1, np.int32)
    for b in range(B):
        for s in range(S1):
            thr = S2 if mode == 0 else S2 - S1 + s + 1
            if thr > 0:
                n = min(K, thr)
                si[b, s, 0, :n] = np.sort(rng.permutation(thr)[:n])
    return q, k, qr, kr, si


def test_pa_equals_bsnd():
    rng = np.random.RandomState(11)
    B, S1, S2, N1, D, K, bs = 2, 2, 32, 4, 128, 8, 8
    q, k, qr, kr, si = _rand_case(rng, B, S1, S2, N1, D, K, 0)
    nblk = B * S2 // bs
    perm = rng.permutation(nblk + 3)[:nblk]
    cache = np.zeros((nblk + 3, bs, 1, D), np.float32)
    cache_r = np.zeros((nblk + 3, bs, 1, 64), np.float32)
    bt = perm.reshape(B, S2 // bs).astype(np.int32)
    for b in range(B):
        for i in range(S2 // bs):
            cache[bt[b, i]] = k[b, i * bs:(i + 1) * bs]
            cache_r[bt[b, i]] = kr[b, i * bs:(i + 1) * bs]
    np.testing.assert_array_equal(pa_to_bsnd(cache, bt, S2), k)
    a = sparse_flash_attention(q, k, si, 0.1, qr, kr, return_softmax_lse=True)
    p = sparse_flash_attention(q, cache, si, 0.1, qr, cache_r, block_table=bt,
                               actual_seq_lengths_kv=[S2] * B, layout_kv="PA_BSND",
                               return_softmax_lse=True)
    for x, y in zip(a, p):
        np.testing.assert_array_equal(x, y)


def test_pa_minus1_block_reads_zero_rows():
    cache = np.ones((2, 4, 1, 3), np.float32)
    bt = np.array([[1, -1, 0]], np.int32)
    d = pa_to_bsnd(cache, bt, 12)
    assert np.all(d[0, :4] == 1) and np.all(d[0, 4:8] == 0) and np.all(d[0, 8:] == 1)


def test_tnd_equals_per_sequence_bsnd():
    rng = np.random.RandomState(12)
    lens = [5, 9, 3]
    N1, D, K = 4, 128, 8
    qs, ks, qrs, krs, sis = [], [], [], [], []
    for n in lens:
        q, k, qr, kr, si = _rand_case(rng, 1, n, n, N1, D, K, 3)
        qs.append(q[0]); ks.append(k[0]); qrs.append(qr[0]); krs.append(kr[0]); sis.append(si[0])
    cum = np.cumsum(lens)
    out, mx, sm = sparse_flash_attention(
        np.concatenate(qs), np.concatenate(ks), np.concatenate(sis), 0.2,
        np.concatenate(qrs), np.concatenate(krs), actual_seq_lengths_query=cum,
        actual_seq_lengths_kv=cum, layout_query="TND", layout_kv="TND", sparse_mode=3,
        return_softmax_lse=True)
    assert out.shape == (sum(lens), N1, D) and mx.shape == (1, sum(lens), N1)
    start = 0
    for i, n in enumerate(lens):
        o1, m1, s1_ = sparse_flash_attention(qs[i][None], ks[i][None], sis[i][None], 0.2,
                                             qrs[i][None], krs[i][None], sparse_mode=3,
                                             return_softmax_lse=True)
        np.testing.assert_array_equal(out[start:start + n], o1[0])
        np.testing.assert_array_equal(mx[0, start:start + n], m1[0, 0])
        np.testing.assert_array_equal(sm[0, start:start + n], s1_[0, 0])
        start += n


def test_blockwise_equals_expanded_tokenwise():
    rng = np.random.RandomState(13)
    B, S1, S2, N1, D, bs = 1, 4, 64, 2, 128, 4
    q, k, qr, kr, _ = _rand_case(rng, B, S1, S2, N1, D, 4, 3)
    si = np.full((B, S1, 1, 6), -1, np.int32)
    for s in range(S1):
        nb = -(-(S2 - S1 + s + 1) // bs)
        si[0, s, 0, :5] = np.sort(rng.permutation(nb)[:5])
    tok = expand_block_indices(si, bs)
    assert tok.shape[-1] == 24 and np.all(tok[si.repeat(bs, -1) == -1] == -1)
    a = sparse_flash_attention(q, k, si, 0.1, qr, kr, sparse_block_size=bs, sparse_mode=3,
                               return_softmax_lse=True)
    b = sparse_flash_attention(q, k, tok, 0.1, qr, kr, sparse_block_size=1, sparse_mode=3,
                               return_softmax_lse=True)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    g = sfa_fwd_bsnd(q, k, si, qr, kr, 0.1, [S1], [S2], sparse_block_size=bs, sparse_mode=3,
                     positions="golden")
    for x, y in zip(a, g):
        np.testing.assert_array_equal(x, y)


def test_tnd_pack_roundtrip():
    x = np.arange(10 * 3).reshape(10, 3)
    d = tnd_to_bsnd(x, [4, 0, 6])
    assert d.shape == (3, 6, 3) and np.all(d[1] == 0)
    from oracle.common import bsnd_to_tnd
    np.testing.assert_array_equal(bsnd_to_tnd(d, [4, 0, 6]), x)


# ---------------------------------------------------------------------------
# backward pins
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("mode", [0, 3])
def test_bwd_oracle_matches_finite_differences(mode):
    """Central differences of the fp64 forward, d(k_nope) = dk + dv (value = key)."""
    rng = np.random.RandomState(0)
    B, S1, S2, N1, D, Dr, K = 1, 4, 8, 2, 16, 8, 4
    qn = rng.randn(B, S1, N1, D) * 0.3; kn = rng.randn(B, S2, 1, D) * 0.3
    qr = rng.randn(B, S1, N1, Dr) * 0.3; kr = rng.randn(B, S2, 1, Dr) * 0.3
    do = rng.randn(B, S1, N1, D)
    si = np.full((B, S1, 1, K), -1, np.int32)
    for s in range(S1):
        thr = S2 if mode == 0 else S2 - S1 + s + 1
        n = min(K, thr)
        si[0, s, 0, :n] = np.sort(rng.permutation(thr)[:n])
    sc, aq, ak = 1 / np.sqrt(D + Dr), [S1], [S2]

    def loss(qn_, kn_, qr_, kr_):
        o, _, _ = sfa_fwd_bsnd(qn_, kn_, si, qr_, kr_, sc, aq, ak, sparse_mode=mode,
                               compute_dtype=np.float64)
        return float(np.sum(o * do))

    out, mx, sm = sfa_fwd_bsnd(qn, kn, si, qr, kr, sc, aq, ak, sparse_mode=mode, compute_dtype=np.float64)
    dq, dk, dv, dqr, dkr = sfa_bwd_bsnd(qn, kn, si, do, out, mx, sm, qr, kr, sc, aq, ak,
                                        sparse_mode=mode, compute_dtype=np.float64)
    eps = 1e-6
    args = [qn, kn, qr, kr]
    grads = [dq, dk + dv, dqr, dkr]
    for ai, (arr, g) in enumerate(zip(args, grads)):
        for idx in list(np.ndindex(arr.shape))[::max(1, arr.size // 12)]:
            a = [x.copy() for x in args]
            a[ai][idx] += eps
            lp = loss(*a)
            a[ai][idx] -= 2 * eps
            lm = loss(*a)
            assert abs((lp - lm) / (2 * eps) - g[idx]) < 1e-7, (ai, idx)


def test_bwd_delta_identity():
    """delta = dO.O equals sum_p P*dP (the identity the backward relies on)."""
    rng = np.random.RandomState(2)
    B, S1, S2, N1, D, Dr = 1, 2, 10, 3, 8, 4
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    do = rng.randn(B, S1, N1, D)
    si = np.tile(np.arange(0, 10, 2, dtype=np.int32), (B, S1, 1, 1))
    out, mx, sm = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, [S1], [S2], sparse_mode=0, compute_dtype=np.float64)
    pos = np.arange(0, 10, 2)
    for s1 in range(S1):
        sc = 0.3 * (q[0, s1] @ k[0, pos, 0].T + qr[0, s1] @ kr[0, pos, 0].T)
        P = np.exp(sc - mx[0, 0, s1][:, None]) / sm[0, 0, s1][:, None]
        dP = do[0, s1] @ k[0, pos, 0].T
        np.testing.assert_allclose((P * dP).sum(1), (do[0, s1] * out[0, s1]).sum(1), rtol=1e-12)


# ---------------------------------------------------------------------------
# band mask (pre_tokens / next_tokens)
# ---------------------------------------------------------------------------
INT64_MAX = 9223372036854775807


def _brute_band_fwd(q, k, qr, kr, si, scale, aq, ak, mode, pre, nxt):
    """fp64 brute force over every key position with an explicit visibility
    test: t is kept once per index entry naming it, iff t < act_k, t is at or
    before the causal diagonal (mode 3) and its offset from the band's
    diagonal lies in [-pre, next]."""
    B, S1, N1, D = q.shape
    S2 = k.shape[1]
    out = np.zeros((B, S1, N1, D))
    mx = np.zeros((B, 1, S1, N1))
    sm = np.zeros((B, 1, S1, N1))
    for b in range(B):
        for s1 in range(aq[b]):
            diag = s1 if mode == 0 else ak[b] - aq[b] + s1
            toks = []
            for t in range(S2):
                mult = sum(1 for e in si[b, s1, 0] if int(e) == t)
                off = t - diag
                causal_ok = mode == 0 or t <= ak[b] - aq[b] + s1
                if mult and t < ak[b] and causal_ok and -pre <= off <= nxt:
                    toks.extend([t] * mult)
            if not toks:
                continue
            sc = np.array([(q[b, s1] @ k[b, t, 0] + qr[b, s1] @ kr[b, t, 0]) * scale for t in toks]).T
            m = sc.max(axis=1, keepdims=True)
            e = np.exp(sc - m)
            z = e.sum(axis=1, keepdims=True)
            out[b, s1] = (e / z) @ k[b, toks, 0]
            mx[b, 0, s1] = m[:, 0]
            sm[b, 0, s1] = z[:, 0]
    return out, mx, sm


def _band_case(seed, mode, S1=5, S2=14, K=9):
    rng = np.random.RandomState(seed)
    B, N1, D, Dr = 2, 2, 8, 4
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    si = rng.randint(-1, S2, size=(B, S1, 1, K)).astype(np.int32)
    aq, ak = [S1, S1 - 2], [S2, S2 - 3]
    return q, k, qr, kr, si, aq, ak


@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("pre,nxt", [(0, 0), (2, 1), (3, INT64_MAX), (INT64_MAX, 2), (1, -1), (-2, 4),
                                     (INT64_MAX, -3), (6, 0), (0, 9)])
def test_band_oracle_matches_brute_force(mode, pre, nxt):
    q, k, qr, kr, si, aq, ak = _band_case(11 + mode, mode)
    got = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, aq, ak, sparse_mode=mode, positions="kernel",
                       compute_dtype=np.float64, pre_tokens=pre, next_tokens=nxt)
    exp = _brute_band_fwd(q, k, qr, kr, si, 0.3, aq, ak, mode, pre, nxt)
    for g, e in zip(got, exp):
        np.testing.assert_allclose(g, e, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("mode", [0, 3])
def test_band_open_sides_equal_no_band(mode):
    q, k, qr, kr, si, aq, ak = _band_case(21, mode)
    base = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, aq, ak, sparse_mode=mode, positions="kernel",
                        compute_dtype=np.float64)
    wide = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, aq, ak, sparse_mode=mode, positions="kernel",
                        compute_dtype=np.float64, pre_tokens=10**6, next_tokens=10**6)
    for a, b in zip(base, wide):
        np.testing.assert_array_equal(a, b)
    if mode == 3:
        # bottom-right band: next_tokens >= 0 adds nothing to the causal bound
        nz = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, aq, ak, sparse_mode=3, positions="kernel",
                          compute_dtype=np.float64, next_tokens=0)
        for a, b in zip(base, nz):
            np.testing.assert_array_equal(a, b)


def test_band_diagonal_only_closed_form():
    """pre = next = 0 keeps exactly the diagonal token: out = v[diag], sum 1."""
    rng = np.random.RandomState(31)
    B, S1, S2, N1, D, Dr = 1, 4, 10, 3, 8, 4
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, 1, D)
    qr = rng.randn(B, S1, N1, Dr); kr = rng.randn(B, S2, 1, Dr)
    si = np.tile(np.arange(S2, dtype=np.int32), (B, S1, 1, 1))
    for mode, diag in ((0, lambda s: s), (3, lambda s: S2 - S1 + s)):
        out, mx, sm = sfa_fwd_bsnd(q, k, si, qr, kr, 0.5, [S1], [S2], sparse_mode=mode, positions="kernel",
                                   compute_dtype=np.float64, pre_tokens=0, next_tokens=0)
        for s1 in range(S1):
            t = diag(s1)
            np.testing.assert_allclose(out[0, s1], np.broadcast_to(k[0, t, 0], (N1, D)), rtol=1e-13)
            np.testing.assert_allclose(sm[0, 0, s1], 1.0)
            np.testing.assert_allclose(mx[0, 0, s1], 0.5 * (q[0, s1] @ k[0, t, 0] + qr[0, s1] @ kr[0, t, 0]))


def test_band_empty_rows_are_zero():
    """A band that lies wholly outside [0, act_k) leaves output and stats zero."""
    q, k, qr, kr, si, aq, ak = _band_case(41, 0)
    out, mx, sm = sfa_fwd_bsnd(q, k, si, qr, kr, 0.3, aq, ak, sparse_mode=0, positions="kernel",
                               compute_dtype=np.float64, pre_tokens=-100, next_tokens=INT64_MAX)
    assert not out.any() and not mx.any() and not sm.any()


@pytest.mark.parametrize("mode", [0, 3])
def test_band_bwd_matches_finite_differences(mode):
    rng = np.random.RandomState(51)
    B, S1, S2, N1, D, Dr, K = 1, 4, 9, 2, 8, 4, 7
    qn = rng.randn(B, S1, N1, D) * 0.3; kn = rng.randn(B, S2, 1, D) * 0.3
    qr = rng.randn(B, S1, N1, Dr) * 0.3; kr = rng.randn(B, S2, 1, Dr) * 0.3
    do = rng.randn(B, S1, N1, D)
    si = np.stack([rng.permutation(S2)[:K] for _ in range(S1)]).astype(np.int32).reshape(B, S1, 1, K)
    sc, aq, ak, pre, nxt = 1 / np.sqrt(D + Dr), [S1], [S2], 2, 1
    kw = dict(sparse_mode=mode, positions="kernel", compute_dtype=np.float64, pre_tokens=pre, next_tokens=nxt)

    def loss(qn_, kn_, qr_, kr_):
        return float(np.sum(sfa_fwd_bsnd(qn_, kn_, si, qr_, kr_, sc, aq, ak, **kw)[0] * do))

    out, mx, sm = sfa_fwd_bsnd(qn, kn, si, qr, kr, sc, aq, ak, **kw)
    dq, dk, dv, dqr, dkr = sfa_bwd_bsnd(qn, kn, si, do, out, mx, sm, qr, kr, sc, aq, ak, **kw)
    assert np.abs(dk).sum() > 0
    eps = 1e-6
    args = [qn, kn, qr, kr]
    for ai, (arr, g) in enumerate(zip(args, [dq, dk + dv, dqr, dkr])):
        for idx in list(np.ndindex(arr.shape))[::max(1, arr.size // 12)]:
            a = [x.copy() for x in args]
            a[ai][idx] += eps
            lp = loss(*a)
            a[ai][idx] -= 2 * eps
            lm = loss(*a)
            assert abs((lp - lm) / (2 * eps) - g[idx]) < 1e-7, (ai, idx)
