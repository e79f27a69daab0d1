"""Shared input builders for the GPU parity tests (seeded, reference recipes)."""
import numpy as np
import torch

from oracle.common import round_to


def to_dtype_np(x, dtype):
    """fp32 numpy -> values representable in ``dtype`` (torch cast, RNE)."""
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dtype)
    return t.float().numpy()


def dev(x, dtype, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def np_dtype_name(dtype):
    return {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[dtype]


def sparse_indices(B, S1, S2, count, bs, mode, act_q=None, act_k=None, seed=7):
    """Front-valid sorted block ids with -1 padding (test_sfa_triton.py:63-85)."""
    rng = np.random.RandomState(seed)
    si = np.full((B, S1, 1, count), -1, np.int32)
    for b in range(B):
        aq = S1 if act_q is None else act_q[b]
        ak = S2 if act_k is None else act_k[b]
        for s1 in range(S1):
            thr = ak if mode == 0 else ak - aq + s1 + 1
            if thr <= 0:
                continue
            nb = -(-thr // bs)
            n = min(count, nb)
            si[b, s1, 0, :n] = np.sort(rng.permutation(nb)[:n])
    return si


def sfa_inputs(B, S1, S2, N1, D, dtype, scale_qk=1.0, seed=42):
    """q, k, qr, kr as fp32 arrays holding ``dtype`` values (randn -> fp16 -> dtype)."""
    rng = np.random.RandomState(seed)

    def t(shape):
        x = (rng.randn(*shape) * scale_qk).astype(np.float16).astype(np.float32)
        return to_dtype_np(x, dtype)

    q = t((B, S1, N1, D))
    k = t((B, S2, 1, D))
    qr = t((B, S1, N1, 64))
    kr = t((B, S2, 1, 64))
    return q, k, qr, kr


def assert_close(actual, expected, rtol, atol, what=""):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} vs {e.shape}"
    err = np.abs(a - e)
    tol = atol + rtol * np.abs(e)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(
            f"{what}: {bad.sum()}/{bad.size} elements out of tolerance "
            f"(rtol={rtol}, atol={atol}); worst at {i}: got {a[i]:.6g} expected {e[i]:.6g}; "
            f"max abs err {err.max():.3g}")
    assert np.all(np.isfinite(a)), f"{what}: non-finite values"
