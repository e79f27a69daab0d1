"""Write the golden-vector fixtures under tests/golden/ from the reference's
own numpy goldens.

Run in the build container only (it reads /root/reference, which does not
exist on GPU boxes):

    python tests/golden/make_fixtures.py

It imports ``sparse_flash_attention_numpy`` and
``sparse_flash_attention_grad_numpy`` from the reference checkout (both
import only numpy and math), draws inputs with the reference tests' seeded
recipes (test_sfa_triton.py:47-85, test_sfa_grad_triton.py:49-82), calls the
goldens, and saves inputs plus outputs as small ``.npz`` files.  Only data is
written; no reference source is copied.  The fixtures pin the goldens'
rounding placement (probabilities rounded to the I/O dtype before P.V, the
output and gradients rounded at the end) and their index-scan rules, which
closed-form checks cannot pin.
"""
import os
import sys

import numpy as np

REF = os.environ.get("DSA_REFERENCE_DIR", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))


def _load_goldens():
    sys.path.insert(0, REF)
    import sparse_flash_attention_numpy as fwd_mod  # noqa: E402
    import sparse_flash_attention_grad_numpy as bwd_mod  # noqa: E402
    return fwd_mod, bwd_mod


def _as_dtype(x16, dtype, fwd_mod):
    """fp16 values -> values of ``dtype`` held in fp32 (test_sfa_triton.py:52-53)."""
    x = x16.astype(np.float32)
    if dtype == "bfloat16":
        return fwd_mod._round_bf16(x)
    return x


def _indices(B, S1, S2, count, bs, mode, act_q=None, act_k=None, seed=7):
    """Front-valid sorted block ids, -1 padded (test_sfa_triton.py:63-85)."""
    rng = np.random.RandomState(seed)
    si = np.full((B, S1, 1, count), -1, np.int32)
    for b in range(B):
        aq = S1 if act_q is None else act_q[b]
        ak = S2 if act_k is None else act_k[b]
        for s1 in range(S1):
            thr = ak if mode == 0 else ak - aq + s1 + 1
            if thr <= 0:
                continue
            nb = int(np.ceil(thr / bs))
            n = min(count, nb)
            si[b, s1, 0, :n] = np.sort(rng.permutation(nb)[:n]).astype(np.int32)
    return si


CASES = [
    # name, B, S1, S2, N1, D, count, bs, mode, dtype, extra
    ("cfg1_bsnd_mode0_bf16", 1, 4, 256, 8, 128, 64, 1, 0, "bfloat16", {}),
    ("mode3_bf16_b2", 2, 16, 64, 8, 128, 32, 1, 3, "bfloat16", {}),
    ("mode3_fp16_d256", 1, 4, 128, 4, 256, 64, 1, 3, "float16", {}),
    ("mode3_bf16_d512_n16", 1, 2, 96, 16, 512, 48, 1, 3, "bfloat16", {}),
    ("blockwise_bs2_mode3", 1, 8, 128, 8, 128, 32, 2, 3, "bfloat16", {}),
    ("blockwise_bs4_mode3_fp16", 1, 8, 256, 4, 128, 32, 4, 3, "float16", {}),
    ("s1_gt_s2_mode3", 1, 12, 8, 4, 128, 8, 1, 3, "bfloat16", {}),
    ("n1_1_mode3", 1, 4, 128, 1, 128, 64, 1, 3, "bfloat16", {}),
    ("n1_128_mode0", 1, 2, 64, 128, 128, 16, 1, 0, "bfloat16", {}),
    ("actlen_mode3", 2, 8, 64, 4, 128, 16, 1, 3, "bfloat16",
     {"act_q": [5, 8], "act_k": [40, 64]}),
    ("actlen_mode0", 2, 8, 64, 4, 128, 16, 1, 0, "float16",
     {"act_q": [8, 3], "act_k": [17, 64]}),
    ("mid_minus1_mode0", 1, 3, 64, 4, 128, 16, 1, 0, "bfloat16", {"mid_minus1": True}),
    ("duplicates_mode0", 1, 3, 64, 4, 128, 16, 1, 0, "bfloat16", {"duplicates": True}),
]


def make_case(fwd_mod, bwd_mod, name, B, S1, S2, N1, D, count, bs, mode, dtype, extra):
    Dr = 64
    rng = np.random.RandomState(42)
    q = _as_dtype(rng.randn(B, S1, N1, D).astype(np.float16), dtype, fwd_mod)
    k = _as_dtype(rng.randn(B, S2, 1, D).astype(np.float16), dtype, fwd_mod)
    v = _as_dtype(rng.randn(B, S2, 1, D).astype(np.float16), dtype, fwd_mod)
    qr = _as_dtype(rng.randn(B, S1, N1, Dr).astype(np.float16), dtype, fwd_mod)
    kr = _as_dtype(rng.randn(B, S2, 1, Dr).astype(np.float16), dtype, fwd_mod)
    rng_do = np.random.RandomState(43)
    do = _as_dtype((rng_do.randn(B, S1, N1, D) * 0.5).astype(np.float16), dtype, fwd_mod)
    act_q = extra.get("act_q", [S1] * B)
    act_k = extra.get("act_k", [S2] * B)
    si = _indices(B, S1, S2, count, bs, mode, act_q, act_k)
    if extra.get("mid_minus1"):
        # a -1 in the middle of row 1: the golden stops scanning there
        si[0, 1, 0, count // 2] = -1
    if extra.get("duplicates"):
        si[0, 2, 0, 1] = si[0, 2, 0, 0]
    gdt = fwd_mod.BF16 if dtype == "bfloat16" else np.float16
    scale = 1.0 / np.sqrt(D + Dr)
    out, smax, ssum = fwd_mod.sparse_flash_attention_golden_bsnd(
        q, k, v, si, qr, kr, scale, act_q, act_k, sparse_block_size=bs,
        sparse_mode=mode, return_softmax_lse=True, dtype=gdt)
    # the backward golden consumes the forward golden's own state
    # (test_sfa_grad_triton.py:121-136 does the same with the device forward)
    dq, dk, dv, dqr, dkr = bwd_mod.sparse_flash_attention_grad_golden_bsnd(
        q, k, v, si, do, out, smax, ssum, qr, kr, scale, act_q, act_k,
        sparse_block_size=bs, sparse_mode=mode, dtype=gdt)
    path = os.path.join(HERE, f"sfa_{name}.npz")
    np.savez_compressed(
        path, q=q, k=k, qr=qr, kr=kr, sparse_indices=si, d_out=do,
        act_q=np.asarray(act_q, np.int32), act_k=np.asarray(act_k, np.int32),
        scale=np.float64(scale), sparse_block_size=np.int32(bs),
        sparse_mode=np.int32(mode), dtype=np.array(dtype),
        out=out, softmax_max=smax, softmax_sum=ssum,
        dq=dq, dk=dk, dv=dv, dqr=dqr, dkr=dkr)
    return path


def main():
    fwd_mod, bwd_mod = _load_goldens()
    for case in CASES:
        p = make_case(fwd_mod, bwd_mod, *case)
        print(f"wrote {os.path.relpath(p)} ({os.path.getsize(p)} bytes)")


if __name__ == "__main__":
    main()
