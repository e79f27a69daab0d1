"""Shared oracle helpers: dtype rounding, token-position scan, layout helpers.

Test infrastructure only (see ``oracle/__init__.py``).
"""
import math

import numpy as np

BF16 = "bfloat16"
FP16 = "float16"
FP32 = "float32"

INT64_MAX = 9223372036854775807


def round_bf16(x):
    """fp32 -> bf16 -> fp32, round-to-nearest-even on the upper 16 bits.

    Restates sparse_flash_attention_numpy.py:26-32 (finite inputs).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = (u + np.uint32(0x7FFF) + lsb) & np.uint32(0xFFFF0000)
    return r.view(np.float32).reshape(np.shape(x))


def round_to(x, dtype):
    """Round an fp32 array to ``dtype`` precision and return fp32.

    ``dtype`` is one of "bfloat16", "float16", "float32" (or the numpy
    float16/float32 types), following the golden's ``_round`` helpers
    (sparse_flash_attention_numpy.py:108-115).
    """
    name = dtype_name(dtype)
    x = np.asarray(x, dtype=np.float32)
    if name == FP16:
        return x.astype(np.float16).astype(np.float32)
    if name == BF16:
        return round_bf16(x)
    return x


def dtype_name(dtype):
    if dtype in (np.float16, FP16, "fp16", "half"):
        return FP16
    if dtype in (BF16, "bf16"):
        return BF16
    if dtype in (np.float32, FP32, "fp32", "float"):
        return FP32
    raise ValueError(f"unknown dtype {dtype!r}")


def row_threshold(sparse_mode, act_q, act_k, s1):
    """Visible-token bound of query row ``s1``.

    sparse_mode 0: act_k; sparse_mode 3 (rightDownCausal): act_k - act_q + s1 + 1
    (sparse_flash_attention_triton.py:247-251).
    """
    return act_k if sparse_mode == 0 else act_k - act_q + s1 + 1


def band_bounds(sparse_mode, act_q, act_k, s1, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """(lo, threshold) of query row ``s1``: tokens lo <= t < threshold are visible.

    ``threshold`` starts from ``row_threshold``.  The reference accepts only
    the default pre_tokens = next_tokens = INT64_MAX
    (sparse_flash_attention_triton.py:531-532,
    sparse_flash_attention_grad_triton.py:428-429).  Other values are read as
    the band of the Ascend FlashAttention operators: token t is visible iff
    diag - pre_tokens <= t <= diag + next_tokens, where diag = s1 in mode 0
    (aligned at the top left) and diag = act_k - act_q + s1 in mode 3 (aligned
    at the bottom right, so next_tokens >= 0 leaves the causal bound as it
    is).  INT64_MAX on either side means that side is open.  Python integers
    make the sums exact (no saturation is needed here).
    """
    thr = row_threshold(sparse_mode, act_q, act_k, s1)
    diag = s1 if sparse_mode == 0 else act_k - act_q + s1
    lo = 0
    if pre_tokens != INT64_MAX:
        lo = max(0, diag - int(pre_tokens))
    if next_tokens != INT64_MAX:
        thr = min(thr, diag + int(next_tokens) + 1)
    return lo, thr


def gather_positions(idx_row, block_size, threshold, act_k, band_lo=0):
    """Token positions a row attends to, following the golden's scan.

    Restates sparse_flash_attention_numpy.py:38-60: only the first
    ceil(threshold / block_size) entries are scanned, a -1 entry ends the
    scan, each block id expands to [id*bs, id*bs+bs) clipped to act_k and to
    the threshold.  Duplicated ids contribute their positions twice.
    Positions below ``band_lo`` (the band's lower edge, ``band_bounds``)
    are dropped.
    """
    count = min(len(idx_row), math.ceil(threshold / block_size))
    out = []
    for i in range(count):
        blk = int(idx_row[i])
        if blk == -1:
            break
        lo = blk * block_size
        hi = min(lo + block_size, act_k)
        if lo >= threshold:
            continue
        out.extend(range(max(lo, band_lo), min(hi, threshold)))
    return out


def kernel_positions(idx_row, block_size, threshold, act_k, band_lo=0):
    """Token positions under per-entry masking (the device kernels' rule).

    Block ids are expanded to token ids first (sparse_flash_attention_triton.py
    :406-421); each token is kept iff tok != -1, tok < threshold and
    tok < act_k (sparse_flash_attention_triton.py:270-272), and tok >=
    ``band_lo`` (the band's lower edge, ``band_bounds``).  Agrees with
    ``gather_positions`` on front-valid rows.
    """
    out = []
    for blk in idx_row:
        blk = int(blk)
        if blk == -1:
            continue
        for t in range(blk * block_size, blk * block_size + block_size):
            if max(0, band_lo) <= t < threshold and t < act_k:
                out.append(t)
    return out


def expand_block_indices(indices, block_size):
    """Block ids [..., K] -> token ids [..., K*bs]; -1 stays -1.

    Restates sparse_flash_attention_triton.py:406-421.
    """
    indices = np.asarray(indices, dtype=np.int64)
    if block_size == 1:
        return indices.astype(np.int32)
    offs = np.arange(block_size, dtype=np.int64)
    tok = indices[..., None] * block_size + offs
    tok = np.where(indices[..., None] == -1, -1, tok)
    return tok.reshape(*indices.shape[:-1], indices.shape[-1] * block_size).astype(np.int32)


def cumsum_to_lengths(cum):
    """TND cumulative lengths -> per-batch lengths (sparse_flash_attention_triton.py:345-347)."""
    cum = np.asarray(cum, dtype=np.int64)
    return cum - np.concatenate([[0], cum[:-1]])


def tnd_to_bsnd(x, lengths):
    """[T, ...] -> [B, max_len, ...] zero padded (sparse_flash_attention_triton.py:350-364)."""
    lengths = [int(v) for v in lengths]
    max_len = max(lengths) if lengths else 0
    out = np.zeros((len(lengths), max_len) + x.shape[1:], dtype=x.dtype)
    start = 0
    for b, n in enumerate(lengths):
        if n > 0:
            out[b, :n] = x[start:start + n]
            start += n
    return out


def bsnd_to_tnd(x, lengths):
    """[B, S, ...] -> [T, ...]; inverse of ``tnd_to_bsnd`` (sparse_flash_attention_triton.py:367-379)."""
    lengths = [int(v) for v in lengths]
    parts = [x[b, :n] for b, n in enumerate(lengths) if n > 0]
    if not parts:
        return np.zeros((0,) + x.shape[2:], dtype=x.dtype)
    return np.concatenate(parts, axis=0)


def pa_to_bsnd(cache, block_table, max_s2):
    """Paged cache [blocks, bs, N, Dx] -> dense [B, max_s2, N, Dx].

    Restates sparse_flash_attention_triton.py:382-403: block id -1 leaves the
    span zero.
    """
    nblk, bs = cache.shape[0], cache.shape[1]
    block_table = np.asarray(block_table)
    B = block_table.shape[0]
    out = np.zeros((B, max_s2) + cache.shape[2:], dtype=cache.dtype)
    for b in range(B):
        for i in range(block_table.shape[1]):
            blk = int(block_table[b, i])
            if blk == -1:
                continue
            dst = i * bs
            if dst >= max_s2:
                break
            end = min(dst + bs, max_s2)
            out[b, dst:end] = cache[blk, :end - dst]
    return out
