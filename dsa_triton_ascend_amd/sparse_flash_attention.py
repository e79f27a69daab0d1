"""sparse_flash_attention forward on MI355X: the reference's public API over
the HIP library.

Drop-in for ``sparse_flash_attention_triton`` / ``SparseFlashAttentionTriton``
(sparse_flash_attention_triton.py:483-695): same argument names, defaults,
guards (ValueError on the same conditions, 529-539 and 579-586), layouts
(BSND / TND query; BSND / TND / PA_BSND key) and return tuple
``(attention_out, softmax_max, softmax_sum)``.  The host-side layout
normalisation of the reference (TND unpacking, PA de-paging, block-id
expansion, lines 551-611) is done inside the kernel instead: no host loops,
no device->host synchronisation.

Deliberate differences, all on inputs the reference does not handle:
* ``pre_tokens`` / ``next_tokens`` other than INT64_MAX (rejected by the
  reference, lines 531-532) select a band: token t of query row s1 is
  visible iff diag - pre_tokens <= t <= diag + next_tokens, with diag = s1
  in sparse_mode 0 and act_kv - act_q + s1 in sparse_mode 3 (the band of the
  Ascend FlashAttention operators; INT64_MAX leaves a side open);
* a block_table entry outside [0, blocks) reads as a zero row like -1
  (the reference would raise while slicing);
* ``block_size`` must equal key.shape[1] when given (the reference mixes the
  two sizes in its de-paging loop, lines 569-571 vs 388).
"""
import torch

from . import _lib

INT64_MAX = 9223372036854775807

_VALID_D = (128, 256, 512)
_D_ROPE = 64
_VALID_N1 = (1, 2, 4, 8, 16, 32, 64, 128)


# Device copies of sequence-length lists, by (device, lengths): building one
# is a host-to-device copy from pageable memory, which waits for the stream's
# queued work, so a call with a plain list would otherwise serialise with
# the kernels of the previous call.  The kernels only read these tensors.
_SEQ_CACHE = {}
_SEQ_CACHE_MAX = 64


def _seq_tensor(x, device):
    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=torch.int32).contiguous()
    key = (str(torch.device(device)), tuple(int(v) for v in x))
    t = _SEQ_CACHE.get(key)
    if t is None:
        t = torch.tensor(list(key[1]), dtype=torch.int32, device=device)
        if len(_SEQ_CACHE) >= _SEQ_CACHE_MAX:
            _SEQ_CACHE.pop(next(iter(_SEQ_CACHE)))
        _SEQ_CACHE[key] = t
    return t


def _expect_shape(t, shape, name):
    """Raise ValueError unless ``t`` has exactly ``shape``: the kernels index
    every operand by these sizes, so a mismatch would read out of bounds."""
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _expect_numel(t, n, name):
    if t.numel() != n:
        raise ValueError(f"{name} must have {n} elements, got {t.numel()} (shape {tuple(t.shape)})")


def _band_args(pre_tokens, next_tokens):
    """pre_tokens / next_tokens as Python ints in int64 range (the C-ABI
    takes int64_t; ctypes would wrap larger values silently)."""
    out = []
    for name, v in (("pre_tokens", pre_tokens), ("next_tokens", next_tokens)):
        if isinstance(v, torch.Tensor):
            v = v.item()
        if isinstance(v, bool) or int(v) != v:
            raise ValueError(f"{name} must be an integer, got {v!r}")
        v = int(v)
        if not -INT64_MAX - 1 <= v <= INT64_MAX:
            raise ValueError(f"{name} must fit in int64, got {v}")
        out.append(v)
    return tuple(out)


def _check_device(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("sparse_flash_attention requires tensors on a ROCm GPU device "
                             "(this implementation has no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def sparse_flash_attention_triton(
    query,
    key,
    value,
    sparse_indices,
    scale_value=1.0,
    block_table=None,
    actual_seq_lengths_query=None,
    actual_seq_lengths_kv=None,
    query_rope=None,
    key_rope=None,
    sparse_block_size=1,
    layout_query="BSND",
    layout_kv="BSND",
    sparse_mode=0,
    pre_tokens=INT64_MAX,
    next_tokens=INT64_MAX,
    attention_mode=2,
    return_softmax_lse=False,
    block_size=0,
):
    """Sparse flash attention forward (MLA-absorb, MQA); see module docstring.

    Args mirror sparse_flash_attention_triton.py:505-526.  ``value`` is
    ignored (value = key[..., :D]).  Returns (attention_out, softmax_max,
    softmax_sum); the stats are (B,1,S1,N1) for BSND queries or (1,T1,N1) for
    TND queries, fp32, zeros unless return_softmax_lse.
    """
    if attention_mode != 2:
        raise ValueError("Only attention_mode=2 (MLA-absorb) is supported")
    pre_tokens, next_tokens = _band_args(pre_tokens, next_tokens)
    if sparse_mode not in (0, 3):
        raise ValueError("Only sparse_mode 0 (full) / 3 (rightDownCausal) supported")
    if query_rope is None or key_rope is None:
        raise ValueError("query_rope and key_rope are required (no empty rope)")
    if sparse_block_size < 1 or (sparse_block_size & (sparse_block_size - 1)) != 0 \
            or sparse_block_size > 128:
        raise ValueError("sparse_block_size must be a power of 2 in [1,128]")
    if layout_query not in ("BSND", "TND"):
        raise ValueError(f"layout_query must be BSND or TND, got {layout_query}")
    if layout_kv not in ("BSND", "TND", "PA_BSND"):
        raise ValueError(f"layout_kv must be BSND, TND or PA_BSND, got {layout_kv}")

    is_tnd_q = layout_query == "TND"
    is_tnd_kv = layout_kv == "TND"
    is_pa = layout_kv == "PA_BSND"
    device = query.device

    # ---- shapes (reference 577-586) ----
    if is_tnd_q:
        if actual_seq_lengths_query is None:
            raise ValueError("TND layout requires actual_seq_lengths_query (cumulative)")
        T1, N1, D = query.shape
        act_q = _seq_tensor(actual_seq_lengths_query, device)
        B = act_q.numel()
        S1 = 0
        q_rows = T1
    else:
        B, S1, N1, D = query.shape
        act_q = _seq_tensor(actual_seq_lengths_query, device)
        q_rows = B * S1
    D_ROPE = query_rope.shape[-1]
    if is_pa:
        if block_table is None:
            raise ValueError("PA_BSND requires block_table")
        if actual_seq_lengths_kv is None:
            raise TypeError("PA_BSND requires actual_seq_lengths_kv")
        nblk, page, n2 = key.shape[0], key.shape[1], key.shape[2]
        if block_size and block_size != page:
            raise ValueError(f"block_size ({block_size}) must equal key.shape[1] ({page})")
        max_blocks = block_table.shape[1]
        S2 = max_blocks * page
        kv_rows = nblk * page
        act_k = _seq_tensor(actual_seq_lengths_kv, device)
        bt = block_table.to(dtype=torch.int32).contiguous()
    elif is_tnd_kv:
        if actual_seq_lengths_kv is None:
            raise ValueError("TND layout requires actual_seq_lengths_kv (cumulative)")
        kv_rows, n2 = key.shape[0], key.shape[1]
        act_k = _seq_tensor(actual_seq_lengths_kv, device)
        S2, max_blocks, page, bt = 0, 0, 0, None
    else:
        Bk, S2, n2 = key.shape[0], key.shape[1], key.shape[2]
        kv_rows = Bk * S2
        act_k = _seq_tensor(actual_seq_lengths_kv, device)
        max_blocks, page, bt = 0, 0, None
        if Bk != B:
            raise ValueError(f"key batch {Bk} != query batch {B}")

    if D not in _VALID_D:
        raise ValueError(f"D must be one of {_VALID_D}, got {D}")
    if D_ROPE != _D_ROPE:
        raise ValueError(f"rope dim must be {_D_ROPE}, got {D_ROPE}")
    if n2 != 1:
        raise ValueError("Only N2=1 (MQA) is supported")
    if N1 not in _VALID_N1:
        raise ValueError(f"N1 must be one of {_VALID_N1}, got {N1}")
    if query.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"query dtype must be bfloat16 or float16, got {query.dtype}")
    for name, t in (("key", key), ("query_rope", query_rope), ("key_rope", key_rope)):
        if t.dtype != query.dtype:
            raise ValueError(f"{name} dtype {t.dtype} differs from query dtype {query.dtype}")
    if (act_k is not None and act_k.numel() != B) or (act_q is not None and act_q.numel() != B):
        raise ValueError("actual sequence length arrays must have one entry per batch")

    K = sparse_indices.shape[-1]
    if sparse_indices.numel() != q_rows * K:
        raise ValueError(f"sparse_indices shape {tuple(sparse_indices.shape)} does not match "
                         f"{q_rows} query rows")
    if key.dim() != (3 if is_tnd_kv else 4) or key.shape[-1] != D:
        raise ValueError(f"key must be {'[T2,1,D]' if is_tnd_kv else '[B,S2,1,D]'} with D={D}, "
                         f"got {tuple(key.shape)}")
    _expect_shape(query_rope, tuple(query.shape[:-1]) + (D_ROPE,), "query_rope")
    _expect_shape(key_rope, tuple(key.shape[:-1]) + (D_ROPE,), "key_rope")
    if is_pa and (bt.dim() != 2 or bt.shape[0] < B):
        raise ValueError(f"block_table must be [B, max_blocks] with B={B} rows, got {tuple(bt.shape)}")
    _check_device(query, key, query_rope, key_rope, sparse_indices, block_table)

    q = query.contiguous()
    qr = query_rope.contiguous()
    k = key.contiguous()
    kr = key_rope.contiguous()
    si = sparse_indices.to(dtype=torch.int32).contiguous()

    out_shape = (q_rows, N1, D) if is_tnd_q else (B, S1, N1, D)
    lse_shape = (1, q_rows, N1) if is_tnd_q else (B, 1, S1, N1)
    out = torch.empty(out_shape, dtype=query.dtype, device=device)
    # the library writes the statistics, or zeros when they are not
    # requested (no fill kernels of torch's own per call)
    smax = torch.empty(lse_shape, dtype=torch.float32, device=device)
    ssum = torch.empty(lse_shape, dtype=torch.float32, device=device)
    if q_rows == 0:
        return out, smax, ssum

    lib = _lib.load()
    ws_bytes = lib.dsa_sfa_fwd_workspace_size(q_rows, N1, D, K, sparse_block_size)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device) if ws_bytes else None
    status = lib.dsa_sfa_fwd(
        _lib.ptr(q), _lib.ptr(qr), _lib.ptr(k), _lib.ptr(kr), _lib.ptr(si),
        _lib.ptr(out), _lib.ptr(smax), _lib.ptr(ssum),
        _lib.ptr(act_q), _lib.ptr(act_k), _lib.ptr(bt),
        B, S1, S2, N1, D, D_ROPE, K, q_rows, kv_rows, max_blocks, page,
        sparse_block_size, sparse_mode, pre_tokens, next_tokens, _lib.LAYOUT[layout_query],
        _lib.LAYOUT[layout_kv],
        _lib.dtype_code(query.dtype), float(scale_value), 1 if return_softmax_lse else 0,
        _lib.ptr(ws), ws_bytes, _lib.stream_handle(device))
    _lib.check(status, "dsa_sfa_fwd")
    return out, smax, ssum


class SparseFlashAttentionTriton(torch.nn.Module):
    """Module wrapper of sparse_flash_attention_triton (reference Cell at
    sparse_flash_attention_triton.py:644-695); ``forward`` takes the Cell's
    ``construct`` arguments in the same order."""

    def __init__(self, scale_value=1.0, sparse_block_size=1, layout_query="BSND",
                 layout_kv="BSND", sparse_mode=0, attention_mode=2, return_softmax_lse=False,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX, block_size=0):
        super().__init__()
        self.scale_value = scale_value
        self.sparse_block_size = sparse_block_size
        self.layout_query = layout_query
        self.layout_kv = layout_kv
        self.sparse_mode = sparse_mode
        self.attention_mode = attention_mode
        self.return_softmax_lse = return_softmax_lse
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens
        self.block_size = block_size

    def forward(self, query, key, value, sparse_indices, query_rope=None, key_rope=None,
                actual_seq_lengths_query=None, actual_seq_lengths_kv=None, block_table=None):
        needs_grad = torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (query, key, query_rope, key_rope))
        if needs_grad and self.layout_kv != "PA_BSND" and self.layout_query == self.layout_kv:
            # training: the forward/backward pair as one autograd op (the
            # reference's P.Morph bprop recipe, sparse_flash_attention_grad_triton.py:30-71)
            from .autograd import sparse_flash_attention_train
            if self.attention_mode != 2:
                raise ValueError("Only attention_mode=2 (MLA-absorb) is supported")
            out, smax, ssum = sparse_flash_attention_train(
                query, key, sparse_indices, scale_value=self.scale_value, query_rope=query_rope,
                key_rope=key_rope, actual_seq_lengths_query=actual_seq_lengths_query,
                actual_seq_lengths_kv=actual_seq_lengths_kv, sparse_block_size=self.sparse_block_size,
                layout=self.layout_query, sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens,
                next_tokens=self.next_tokens)
            if not self.return_softmax_lse:
                smax, ssum = torch.zeros_like(smax), torch.zeros_like(ssum)
            return out, smax, ssum
        return sparse_flash_attention_triton(
            query, key, value, sparse_indices,
            scale_value=self.scale_value, block_table=block_table,
            actual_seq_lengths_query=actual_seq_lengths_query,
            actual_seq_lengths_kv=actual_seq_lengths_kv,
            query_rope=query_rope, key_rope=key_rope,
            sparse_block_size=self.sparse_block_size, layout_query=self.layout_query,
            layout_kv=self.layout_kv, sparse_mode=self.sparse_mode,
            pre_tokens=self.pre_tokens, next_tokens=self.next_tokens,
            attention_mode=self.attention_mode, return_softmax_lse=self.return_softmax_lse,
            block_size=self.block_size)

    construct = forward
