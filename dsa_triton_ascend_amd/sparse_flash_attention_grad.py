"""sparse_flash_attention backward on MI355X: the reference's public API over
the HIP library.

Drop-in for ``sparse_flash_attention_grad_triton`` /
``SparseFlashAttentionGradTriton`` (sparse_flash_attention_grad_triton.py:
382-586): same argument names and defaults (``layout="BSND"``,
``sparse_mode=3``), the same guards (ValueError for sparse modes other than
0/3, missing rope, ``deterministic=True``, a block size that is not a power of two <= 128, D,
rope width, N2 != 1, N1 not a power of two <= 128) and the same return tuple
``(d_query, d_key, d_value, d_query_rope, d_key_rope)`` with the shapes and
dtypes of the corresponding inputs.  TND rows and block-wise indices are
resolved in the kernel (no host unpacking).  ``pre_tokens`` /
``next_tokens`` other than INT64_MAX, which the reference rejects (lines
428-429), select the same band as the forward: token t of query row s1 is
visible iff diag - pre_tokens <= t <= diag + next_tokens, diag = s1 in
sparse_mode 0 and act_kv - act_q + s1 in sparse_mode 3.
"""
import torch

from . import _lib
from .sparse_flash_attention import (INT64_MAX, _band_args, _check_device, _expect_numel, _expect_shape,
                                     _seq_tensor, _VALID_D, _VALID_N1)

_D_ROPE = 64


def sparse_flash_attention_grad_triton(
    query,
    key,
    value,
    sparse_indices,
    d_out,
    out,
    softmax_max,
    softmax_sum,
    scale_value=1.0,
    query_rope=None,
    key_rope=None,
    actual_seq_lengths_query=None,
    actual_seq_lengths_kv=None,
    sparse_block_size=1,
    layout="BSND",
    sparse_mode=3,
    pre_tokens=INT64_MAX,
    next_tokens=INT64_MAX,
    deterministic=False,
):
    """SFA backward (MLA-absorb, MQA); see module docstring.  ``value`` is
    only used for the dtype of d_value (value = key[..., :D])."""
    return _sfa_grad(query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
                     scale_value, query_rope, key_rope, actual_seq_lengths_query, actual_seq_lengths_kv,
                     sparse_block_size, layout, sparse_mode, pre_tokens, next_tokens, deterministic,
                     merge_kv=False)


def _sfa_grad(query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum, scale_value,
              query_rope, key_rope, actual_seq_lengths_query, actual_seq_lengths_kv, sparse_block_size,
              layout, sparse_mode, pre_tokens, next_tokens, deterministic, merge_kv):
    """Body of the backward.  With ``merge_kv`` the key gradient is dk + dv,
    summed in fp32 before the cast (the shared-latent gradient), and d_value
    is None."""
    pre_tokens, next_tokens = _band_args(pre_tokens, next_tokens)
    if sparse_mode not in (0, 3):
        raise ValueError("Only sparse_mode 0 (full) / 3 (rightDownCausal) supported")
    if query_rope is None or key_rope is None:
        raise ValueError("query_rope and key_rope are required (no empty rope)")
    if deterministic:
        # the reference rejects it (sparse_flash_attention_grad_triton.py:434-435); kept for
        # parity, although every output here is deterministic
        raise ValueError("deterministic=True is not supported (scatter-add path)")
    if sparse_block_size < 1 or (sparse_block_size & (sparse_block_size - 1)) != 0 \
            or sparse_block_size > 128:
        raise ValueError("sparse_block_size must be a power of 2 in [1,128]")
    if layout not in ("BSND", "TND"):
        raise ValueError(f"layout must be BSND or TND, got {layout}")
    is_tnd = layout == "TND"
    device = query.device

    if is_tnd:
        if actual_seq_lengths_query is None or actual_seq_lengths_kv is None:
            raise ValueError("TND layout requires cumulative actual sequence lengths")
        T1, N1, D = query.shape
        act_q = _seq_tensor(actual_seq_lengths_query, device)
        act_k = _seq_tensor(actual_seq_lengths_kv, device)
        B = act_q.numel()
        S1 = S2 = 0
        q_rows, kv_rows = T1, key.shape[0]
        if key.dim() != 3 or key.shape[1] != 1:
            raise ValueError("Only N2=1 (MQA) is supported")
    else:
        B, S1, N1, D = query.shape
        if key.dim() != 4 or key.shape[2] != 1:
            raise ValueError("Only N2=1 (MQA) is supported")
        S2 = key.shape[1]
        act_q = _seq_tensor(actual_seq_lengths_query, device)
        act_k = _seq_tensor(actual_seq_lengths_kv, device)
        q_rows, kv_rows = B * S1, B * S2
    D_ROPE = query_rope.shape[-1]
    if D not in _VALID_D:
        raise ValueError(f"D must be one of {_VALID_D}, got {D}")
    if D_ROPE != _D_ROPE:
        raise ValueError(f"rope dim must be {_D_ROPE}, got {D_ROPE}")
    if N1 not in _VALID_N1:
        raise ValueError(f"N1 must be one of {_VALID_N1}, got {N1}")
    if query.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("query dtype must be bfloat16 or float16")
    for t, nm in ((key, "key"), (query_rope, "query_rope"), (key_rope, "key_rope"), (d_out, "d_out"),
                  (out, "out")):
        if t.dtype != query.dtype:
            raise ValueError(f"{nm} must have the query dtype")
    K = sparse_indices.shape[-1]
    # every operand is indexed by these sizes in the kernel: check them before any launch
    if key.shape[-1] != D:
        raise ValueError(f"key head dim {key.shape[-1]} differs from the query's {D}")
    _expect_numel(sparse_indices, q_rows * K, "sparse_indices")
    _expect_numel(softmax_max, q_rows * N1, "softmax_max")
    _expect_numel(softmax_sum, q_rows * N1, "softmax_sum")
    _expect_shape(d_out, query.shape, "d_out")
    _expect_shape(out, query.shape, "out")
    _expect_shape(query_rope, tuple(query.shape[:-1]) + (D_ROPE,), "query_rope")
    _expect_shape(key_rope, tuple(key.shape[:-1]) + (D_ROPE,), "key_rope")
    if (act_k is not None and act_k.numel() != B) or (act_q is not None and act_q.numel() != B):
        raise ValueError("actual sequence length arrays must have one entry per batch")
    _check_device(query, key, query_rope, key_rope, sparse_indices, d_out, out, softmax_max, softmax_sum)

    dq = torch.empty_like(query)
    dqr = torch.empty_like(query_rope)
    dk = torch.empty_like(key)
    dkr = torch.empty_like(key_rope)
    if value is not None and value.dtype != key.dtype:
        raise ValueError("value dtype must equal the key dtype")
    dv = None if merge_kv else torch.empty(key.shape, dtype=key.dtype, device=device)
    lib = _lib.load()
    ws_bytes = lib.dsa_sfa_bwd_workspace_size(q_rows, kv_rows, N1, D, K, sparse_block_size, 1 if merge_kv else 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    c = [t.contiguous() for t in (query, query_rope, key, key_rope, d_out, out)]
    si = sparse_indices.to(torch.int32).contiguous()
    smax = softmax_max.to(torch.float32).contiguous()
    ssum = softmax_sum.to(torch.float32).contiguous()
    st = lib.dsa_sfa_bwd(
        c[0].data_ptr(), c[1].data_ptr(), c[2].data_ptr(), c[3].data_ptr(), si.data_ptr(),
        c[4].data_ptr(), c[5].data_ptr(), smax.data_ptr(), ssum.data_ptr(),
        _lib.ptr(act_q), _lib.ptr(act_k),
        dq.data_ptr(), dqr.data_ptr(), dk.data_ptr(), dkr.data_ptr(), _lib.ptr(dv),
        B, S1, S2, N1, D, D_ROPE, K, q_rows, kv_rows, sparse_block_size, sparse_mode,
        pre_tokens, next_tokens, _lib.LAYOUT[layout], _lib.dtype_code(query.dtype), float(scale_value),
        ws.data_ptr(), ws_bytes, _lib.stream_handle(device))
    _lib.check(st, "sparse_flash_attention_grad")
    return dq, dk, dv, dqr, dkr


class SparseFlashAttentionGradTriton(torch.nn.Module):
    """Module form (sparse_flash_attention_grad_triton.py:544-586)."""

    def __init__(self, scale_value=1.0, sparse_block_size=1, layout="BSND", sparse_mode=3,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX, deterministic=False):
        super().__init__()
        self.scale_value = scale_value
        self.sparse_block_size = sparse_block_size
        self.layout = layout
        self.sparse_mode = sparse_mode
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens
        self.deterministic = deterministic

    def forward(self, query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
                query_rope=None, key_rope=None, actual_seq_lengths_query=None,
                actual_seq_lengths_kv=None):
        return sparse_flash_attention_grad_triton(
            query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
            self.scale_value, query_rope, key_rope, actual_seq_lengths_query, actual_seq_lengths_kv,
            self.sparse_block_size, self.layout, self.sparse_mode, self.pre_tokens,
            self.next_tokens, self.deterministic)

    construct = forward
