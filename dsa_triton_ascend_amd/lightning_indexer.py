"""lightning_indexer on MI355X: the reference's public API over the HIP library.

Drop-in for ``lightning_indexer_triton`` / ``LightningIndexerTriton``
(lightning_indexer_triton.py:416-550): same argument names and defaults
(``sparse_count=2048``, ``sparse_mode=3``), the same guards (``block_table``
must be None, N1 divisible by N2) and the same return tuple
``(sparse_indices, sparse_values)``: int32 indices [B,S1,N2,K] (TND:
[T1,N2,K]) and values in the query dtype, zeros unless ``return_value``.

The score kernel and the top-k run on the GPU (``dsa_li_fwd``); TND rows are
resolved in the kernel from the cumulative lengths.  The top-k order is the
stable one the reference's readme specifies (readme.md:63-69): score
descending, index ascending on ties; entries whose score is -inf are -1.

Extension: ``layout_key="PA_BSND"`` with a ``block_table`` runs the indexer
over a paged key cache (``_lightning_indexer_paged``); the reference rejects
a block_table, and still does here with any other key layout.

Inputs: query / key in bfloat16, float16 or float32 (one dtype; fp32 runs
full-fp32 products), any head dim up to 256 whose rows are a whole number of
16 bytes (a multiple of 8 elements, or of 4 in fp32), N1 divisible by N2.

Deliberate differences, on inputs the reference does not handle:
* ``sparse_count`` larger than the key length pads with -1 (the reference's
  reshape fails, lines 341 vs 540);
* ``sparse_count`` is limited to 16384 (the top-k sorts in LDS).
"""
import torch

from . import _lib
from .sparse_flash_attention import INT64_MAX, _check_device, _seq_tensor

_MAX_K = 16384
_MAX_D = 256


def _check_dtypes_and_dim(query, key, D):
    if query.dtype not in (torch.bfloat16, torch.float16, torch.float32) or key.dtype != query.dtype:
        raise ValueError("query and key must share one dtype: bfloat16, float16 or float32")
    step = 4 if query.dtype == torch.float32 else 8
    if D < step or D > _MAX_D or D % step:
        raise ValueError(f"head dim must be a multiple of {step} in [{step}, {_MAX_D}], got {D}")


def _check_k(sparse_count):
    K = int(sparse_count)
    if K < 1 or K > _MAX_K:
        raise ValueError(f"sparse_count must be in [1, {_MAX_K}]")
    return K


def _weights_code(dt):
    if dt == torch.float32:
        return _lib.DTYPE_FP32
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float16:
        return _lib.DTYPE_FP16
    raise ValueError(f"weights dtype must be float32, bfloat16 or float16, got {dt}")


def lightning_indexer_triton(
    query,
    key,
    weights,
    actual_seq_lengths_query=None,
    actual_seq_lengths_key=None,
    block_table=None,
    layout_query="BSND",
    layout_key="BSND",
    sparse_count=2048,
    sparse_mode=3,
    pre_tokens=INT64_MAX,
    next_tokens=INT64_MAX,
    return_value=False,
):
    """Lightning indexer (scores + stable top-k); see module docstring.

    Args mirror lightning_indexer_triton.py:462-494.  ``pre_tokens`` and
    ``next_tokens`` are accepted and ignored, as in the reference.
    """
    if block_table is not None and layout_key != "PA_BSND":
        raise ValueError("PA_BSND / block_table not supported in triton lightning_indexer")
    if layout_query not in ("BSND", "TND"):
        raise ValueError(f"layout_query must be BSND or TND, got {layout_query}")
    if layout_key not in ("BSND", "TND", "PA_BSND"):
        raise ValueError(f"layout_key must be BSND, TND or PA_BSND, got {layout_key}")
    if layout_key == "PA_BSND":
        return _lightning_indexer_paged(query, key, weights, actual_seq_lengths_query, actual_seq_lengths_key,
                                        block_table, layout_query, sparse_count, sparse_mode, return_value)
    if sparse_mode not in (0, 3):
        raise ValueError("Only sparse_mode 0 (full) / 3 (rightDownCausal) supported")
    if query.dtype not in (torch.bfloat16, torch.float16, torch.float32) or key.dtype != query.dtype:
        raise ValueError("query and key must share one dtype: bfloat16, float16 or float32")
    device = _check_device(query, key, weights)
    is_tnd = layout_query == "TND"
    if not is_tnd and layout_key == "TND":
        raise ValueError("a TND key needs a TND query")

    if is_tnd:
        if actual_seq_lengths_query is None or actual_seq_lengths_key is None:
            raise ValueError("TND layout requires actual_seq_lengths_query and actual_seq_lengths_key")
        T1, N1, D = query.shape
        act_q = _seq_tensor(actual_seq_lengths_query, device)
        act_k = _seq_tensor(actual_seq_lengths_key, device)
        B = act_q.numel()
        S1 = 0
        q_rows = T1
        if layout_key == "TND":
            T2, N2, _ = key.shape
            # score-row width: the longest sequence (lengths given as a list are
            # read on the host; a device tensor costs one host read of B
            # lengths, as the reference's TND conversion does)
            if isinstance(actual_seq_lengths_key, torch.Tensor):
                kl = act_k.to("cpu", torch.int64)
            else:
                kl = torch.tensor([int(v) for v in actual_seq_lengths_key], dtype=torch.int64)
            S2 = int((kl - torch.cat([kl.new_zeros(1), kl[:-1]])).max().item()) if B > 0 else 0
            k_rows = T2
        else:
            _, S2, N2, _ = key.shape
            k_rows = key.shape[0] * S2
            if key.shape[0] != B:
                raise ValueError("BSND key batch must match the number of TND query sequences")
        w_shape = (T1, N1)
    else:
        B, S1, N1, D = query.shape
        if key.dim() != 4 or key.shape[0] != B:
            raise ValueError("key must be [B,S2,N2,D] with the query's batch")
        _, S2, N2, _ = key.shape
        act_q = _seq_tensor(actual_seq_lengths_query, device)
        act_k = _seq_tensor(actual_seq_lengths_key, device)
        q_rows = B * S1
        k_rows = B * S2
        w_shape = (B, S1, N1)
    if key.shape[-1] != D:
        raise ValueError("query and key head dims differ")
    if N1 % N2 != 0:
        raise ValueError(f"N1({N1}) must be divisible by N2({N2})")
    _check_dtypes_and_dim(query, key, D)
    if tuple(weights.shape) != w_shape:
        raise ValueError(f"weights must have shape {w_shape}, got {tuple(weights.shape)}")
    K = _check_k(sparse_count)

    out_shape = (q_rows, N2, K) if is_tnd else (B, S1, N2, K)
    # the library writes every entry: the selected scores, or zeros when they
    # are not requested (no fill kernel of torch's own per call)
    indices = torch.empty(out_shape, dtype=torch.int32, device=device)
    values = torch.empty(out_shape, dtype=query.dtype, device=device)
    if q_rows == 0 or S2 == 0:
        indices.fill_(-1)
        values.zero_()
        return indices, values

    lib = _lib.load()
    ws_bytes = lib.dsa_li_fwd_workspace_size(q_rows, N2, S2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    qc, kc, wc = query.contiguous(), key.contiguous(), weights.contiguous()
    st = lib.dsa_li_fwd(
        qc.data_ptr(), kc.data_ptr(), wc.data_ptr(), _lib.ptr(act_q), _lib.ptr(act_k),
        indices.data_ptr(), values.data_ptr(),
        B, S1, S2, N1, N2, D, K, q_rows, k_rows, sparse_mode,
        _lib.LAYOUT[layout_query], _lib.LAYOUT[layout_key], _lib.dtype_code(query.dtype),
        _weights_code(weights.dtype), 1 if return_value else 0,
        ws.data_ptr(), ws_bytes, _lib.stream_handle(device))
    _lib.check(st, "lightning_indexer")
    return indices, values


def _lightning_indexer_paged(query, key, weights, actual_seq_lengths_query, actual_seq_lengths_key,
                             block_table, layout_query, sparse_count, sparse_mode, return_value):
    """The indexer over a paged key cache [blocks, page, N2, D] (an extension:
    the reference rejects block_table, lightning_indexer_triton.py:497-498).
    Key s2 of batch b is cache row block_table[b, s2 // page] * page +
    s2 % page; a -1 block reads as zero key rows, as the reference's SFA
    de-paging leaves them (sparse_flash_attention_triton.py:382-403).
    ``actual_seq_lengths_key`` holds per-batch key lengths."""
    if block_table is None:
        raise ValueError("PA_BSND key layout requires block_table")
    if actual_seq_lengths_key is None:
        raise ValueError("PA_BSND key layout requires actual_seq_lengths_key")
    if sparse_mode not in (0, 3):
        raise ValueError("Only sparse_mode 0 (full) / 3 (rightDownCausal) supported")
    if key.dim() != 4 or block_table.dim() != 2:
        raise ValueError("PA_BSND key must be [blocks, page, N2, D] and block_table [B, max_blocks]")
    device = _check_device(query, key, weights, block_table)
    num_blocks, page, N2, Dk = key.shape
    max_blocks = block_table.shape[1]
    act_q = _seq_tensor(actual_seq_lengths_query, device)
    act_k = _seq_tensor(actual_seq_lengths_key, device)
    if layout_query == "TND":
        if act_q is None:
            raise ValueError("TND layout requires actual_seq_lengths_query")
        T1, N1, D = query.shape
        B, S1, q_rows = act_q.numel(), 0, T1
        w_shape = (T1, N1)
        out_shape = (q_rows, N2, int(sparse_count))
    else:
        B, S1, N1, D = query.shape
        q_rows = B * S1
        w_shape = (B, S1, N1)
        out_shape = (B, S1, N2, int(sparse_count))
    if block_table.shape[0] != B or act_k.numel() != B:
        raise ValueError("block_table and actual_seq_lengths_key need one row / entry per batch")
    if Dk != D:
        raise ValueError("query and key head dims differ")
    if N1 % N2 != 0:
        raise ValueError(f"N1({N1}) must be divisible by N2({N2})")
    _check_dtypes_and_dim(query, key, D)
    if tuple(weights.shape) != w_shape:
        raise ValueError(f"weights must have shape {w_shape}, got {tuple(weights.shape)}")
    K = _check_k(sparse_count)
    indices = torch.empty(out_shape, dtype=torch.int32, device=device)
    values = torch.empty(out_shape, dtype=query.dtype, device=device)
    if q_rows == 0:
        return indices, values
    lib = _lib.load()
    S2 = max_blocks * page
    ws_bytes = lib.dsa_li_fwd_workspace_size(q_rows, N2, S2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    qc, kc, wc = query.contiguous(), key.contiguous(), weights.contiguous()
    bt = block_table.to(torch.int32).contiguous()
    st = lib.dsa_li_fwd_paged(
        qc.data_ptr(), kc.data_ptr(), wc.data_ptr(), _lib.ptr(act_q), act_k.data_ptr(), bt.data_ptr(),
        indices.data_ptr(), values.data_ptr(),
        B, S1, N1, N2, D, K, q_rows, num_blocks, page, max_blocks, sparse_mode,
        _lib.LAYOUT[layout_query], _lib.dtype_code(query.dtype), _weights_code(weights.dtype),
        1 if return_value else 0, ws.data_ptr(), ws_bytes, _lib.stream_handle(device))
    _lib.check(st, "lightning_indexer (paged key)")
    return indices, values


class LightningIndexerTriton(torch.nn.Module):
    """Module form (lightning_indexer_triton.py:416-459).  The constructor
    takes the reference's positional order (419-427): sparse_count,
    sparse_mode, layout_query, layout_key, return_value, pre_tokens,
    next_tokens."""

    def __init__(self, sparse_count=2048, sparse_mode=3, layout_query="BSND", layout_key="BSND",
                 return_value=False, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
        super().__init__()
        self.sparse_count = sparse_count
        self.sparse_mode = sparse_mode
        self.layout_query = layout_query
        self.layout_key = layout_key
        self.return_value = return_value
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens

    def forward(self, query, key, weights, actual_seq_lengths_query=None,
                actual_seq_lengths_key=None, block_table=None):
        return lightning_indexer_triton(
            query, key, weights, actual_seq_lengths_query, actual_seq_lengths_key, block_table,
            self.layout_query, self.layout_key, self.sparse_count, self.sparse_mode,
            self.pre_tokens, self.next_tokens, self.return_value)

    construct = forward


def indexer_scores(query, key, weights, actual_seq_lengths_query=None, actual_seq_lengths_key=None,
                   sparse_mode=3):
    """fp32 scores [B*S1*N2, S2] of a BSND query (-inf where masked): the
    first stage of the indexer (``dsa_li_scores``), exposed for parity tests."""
    B, S1, N1, D = query.shape
    _, S2, N2, _ = key.shape
    device = _check_device(query, key, weights)
    act_q = _seq_tensor(actual_seq_lengths_query, device)
    act_k = _seq_tensor(actual_seq_lengths_key, device)
    scores = torch.empty((B * S1 * N2, S2), dtype=torch.float32, device=device)
    lib = _lib.load()
    qc, kc, wc = query.contiguous(), key.contiguous(), weights.contiguous()
    st = lib.dsa_li_scores(qc.data_ptr(), kc.data_ptr(), wc.data_ptr(), _lib.ptr(act_q), _lib.ptr(act_k),
                           scores.data_ptr(), B, S1, S2, N1, N2, D, B * S1, B * S2, sparse_mode,
                           _lib.LAYOUT["BSND"], _lib.LAYOUT["BSND"], _lib.dtype_code(query.dtype),
                           _weights_code(weights.dtype), _lib.stream_handle(device))
    _lib.check(st, "lightning_indexer scores")
    return scores


def stable_topk(scores, k):
    """Stable top-k of fp32 score rows [R, S2] on the GPU
    (``dsa_li_topk_from_scores``): (indices int32 [R, k], values fp32 [R, k])."""
    if scores.dtype != torch.float32 or scores.dim() != 2:
        raise ValueError("scores must be a 2-D float32 tensor")
    device = _check_device(scores)
    sc = scores.contiguous()
    R, S2 = sc.shape
    idx = torch.empty((R, k), dtype=torch.int32, device=device)
    val = torch.empty((R, k), dtype=torch.float32, device=device)
    lib = _lib.load()
    st = lib.dsa_li_topk_from_scores(sc.data_ptr(), R, S2, k, idx.data_ptr(), val.data_ptr(),
                                     _lib.stream_handle(device))
    _lib.check(st, "stable_topk")
    return idx, val
