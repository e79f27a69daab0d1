"""Sparse lightning-indexer KL-loss backward on MI355X: the reference's
public API over the HIP library.

Drop-in for ``sparse_lightning_indexer_grad_kl_loss_triton`` /
``SparseLightningIndexerGradKLLossTriton``
(sparse_lightning_indexer_grad_kl_loss_triton.py:467-556): same argument
names and defaults, the same guards (ValueError for a sparse_mode other than
3, AssertionError when Nidx2 != 1, lines 534-538), missing rope treated as
zero rope (543-546), and the same return tuple
``(d_query_index, d_key_index, d_weights, loss)`` with d_query_index /
d_key_index / d_weights in the dtype of query_index / key_index / weights
and loss a [1] fp32 tensor (the sum over all query rows).  pre_tokens,
next_tokens and deterministic are accepted and ignored, as in the
reference; every output of this implementation is deterministic.

Index shapes: D_idx any multiple of 8 up to 256, Nidx1 up to 128, any topK
(rows x topK < 2^31); the reference loops over any D_idx and Nidx1
(119-136, 219-262).  D_idx = 128, Nidx1 <= 64 and topK <= 7168 run the
fused row kernel, other shapes a generic path with the same outputs.

Extensions over the reference, which accepts BSND only (534-535):

* ``layout="TND"``: packed rows, query [T1, N1, D], key [T2, 1, D],
  query_index [T1, Nidx1, D_idx], key_index [T2, 1, D_idx], weights [T1, Nidx1],
  sparse_indices [T1, 1, topK], softmax statistics with T1 * N1 entries
  ([1, T1, N1] from the TND forward), and cumulative ``actual_seq_qlen`` /
  ``actual_seq_klen`` (required), as the TND forward takes them.  Token ids
  are clamped to the batch's own key length.
* ``block_table=`` [B, max_blocks] int32: key, key_rope and key_index are
  paged caches [blocks, page, 1, X] (the PA_BSND layout of the forward),
  ``actual_seq_klen`` holds per-batch lengths (required), and d_key_index
  comes back in the paged shape, summed over every slot that targets a
  cache row.  A -1 page reads as zero key rows and receives no gradient.
"""
import torch

from . import _lib
from .sparse_flash_attention import INT64_MAX, _check_device, _seq_tensor, _VALID_D

_D_ROPE = 64
_MAX_D_IDX = 256
_MAX_NIDX = 128
_MAX_N1 = 128


def sparse_lightning_indexer_grad_kl_loss_triton(
    query,
    key,
    query_index,
    key_index,
    weights,
    sparse_indices,
    softmax_max,
    softmax_sum,
    query_rope=None,
    key_rope=None,
    actual_seq_qlen=None,
    actual_seq_klen=None,
    scale_value=1.0,
    layout="BSND",
    sparse_mode=3,
    pre_tokens=INT64_MAX,
    next_tokens=INT64_MAX,
    deterministic=False,
    *,
    block_table=None,
):
    """Indexer KL-loss backward; see module docstring."""
    if layout not in ("BSND", "TND"):
        raise ValueError(f"layout must be BSND or TND, got {layout}")
    if sparse_mode != 3:
        raise ValueError("Only sparse_mode=3 (rightDownCausal) is supported")
    assert sparse_indices.shape[-2] == 1, "Nidx2 must be 1 (MQA constraint)"
    device = _check_device(query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                           softmax_sum, query_rope, key_rope, block_table)
    tnd = layout == "TND"
    paged = block_table is not None
    qdims = 3 if tnd else 4
    if query.dim() != qdims or query_index.dim() != qdims or weights.dim() != qdims - 1:
        raise ValueError(f"{layout} query tensors must be {qdims}-D (weights {qdims - 1}-D)")
    act_q = _seq_tensor(actual_seq_qlen, device)
    act_k = _seq_tensor(actual_seq_klen, device)
    if tnd:
        if act_q is None or (act_k is None and not paged):
            raise ValueError("TND layout requires cumulative actual_seq_qlen and actual_seq_klen")
        T1, N1, D = query.shape
        B, S1, q_rows = int(act_q.numel()), 0, T1
    else:
        B, S1, N1, D = query.shape
        q_rows = B * S1
    Nidx1, D_idx = query_index.shape[-2], query_index.shape[-1]
    kdims = 3 if (tnd and not paged) else 4
    if key.dim() != kdims or key.shape[-2] != 1:
        raise ValueError("Only N2=1 (MQA) is supported")
    if key_index.dim() != kdims or key_index.shape[-2] != 1:
        raise ValueError("Only Nidx2=1 is supported for key_index")
    max_blocks, page = 0, 1
    if paged:
        if block_table.dim() != 2 or block_table.shape[0] != B:
            raise ValueError("block_table must be [B, max_blocks]")
        if act_k is None:
            raise ValueError("a paged key requires actual_seq_klen (per-batch lengths)")
        nblk, page = key.shape[0], key.shape[1]
        max_blocks = block_table.shape[1]
        kv_rows, S2 = nblk * page, max_blocks * page
        layout_k = "PA_BSND"
    elif tnd:
        kv_rows, S2 = key.shape[0], 0
        layout_k = "TND"
    else:
        S2 = key.shape[1]
        if key.shape[0] != B:
            raise ValueError("key batch must match the query batch")
        kv_rows = B * S2
        layout_k = "BSND"
    if key_index.shape[:-1] != key.shape[:-1]:
        raise ValueError("key_index must have the key's rows")
    topK = sparse_indices.shape[-1]
    if D not in _VALID_D:
        raise ValueError(f"D must be one of {_VALID_D}, got {D}")
    if D_idx < 8 or D_idx > _MAX_D_IDX or D_idx % 8:
        raise ValueError(f"index head dim must be a multiple of 8 in [8, {_MAX_D_IDX}], got {D_idx}")
    if not 1 <= Nidx1 <= _MAX_NIDX:
        raise ValueError(f"Nidx1 must be in [1, {_MAX_NIDX}], got {Nidx1}")
    if not 1 <= N1 <= _MAX_N1:
        raise ValueError(f"N1 must be in [1, {_MAX_N1}], got {N1}")
    if query.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("query dtype must be bfloat16 or float16")
    if (query_rope is None) != (key_rope is None):
        raise ValueError("query_rope and key_rope must be given together")
    d_rope = 0
    if query_rope is not None:
        d_rope = query_rope.shape[-1]
        if d_rope != _D_ROPE or key_rope.shape[-1] != _D_ROPE:
            raise ValueError(f"rope dim must be {_D_ROPE}, got {d_rope}")
        if key_rope.shape[:-1] != key.shape[:-1] or query_rope.shape[:-1] != query.shape[:-1]:
            raise ValueError("rope tensors must have the rows and heads of query / key")
    for t, nm in ((key, "key"), (query_index, "query_index"), (key_index, "key_index"),
                  (query_rope, "query_rope"), (key_rope, "key_rope")):
        if t is not None and t.dtype != query.dtype:
            raise ValueError(f"{nm} must have the query dtype")
    if weights.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError("weights dtype must be float32, bfloat16 or float16")
    if sparse_indices.numel() != q_rows * topK or softmax_max.numel() != q_rows * N1 \
            or softmax_sum.numel() != q_rows * N1 or weights.numel() != q_rows * Nidx1:
        raise ValueError("sparse_indices / softmax statistics / weights do not match the query rows")

    d_qi = torch.empty_like(query_index)
    d_ki = torch.empty_like(key_index)
    d_w = torch.empty_like(weights)
    loss = torch.empty(1, dtype=torch.float32, device=device)
    lib = _lib.load()
    if layout_k == "BSND" and not tnd:
        ws_bytes = lib.dsa_kl_bwd_workspace_size(B, S1, S2, topK, D_idx)
    else:
        ws_bytes = lib.dsa_kl_bwd_ex_workspace_size(q_rows, kv_rows, topK, D_idx)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    q, k, qi, ki, w = (t.contiguous() for t in (query, key, query_index, key_index, weights))
    qr = query_rope.contiguous() if d_rope else None
    kr = key_rope.contiguous() if d_rope else None
    si = sparse_indices.to(torch.int32).contiguous()
    smax = softmax_max.to(torch.float32).contiguous()
    ssum = softmax_sum.to(torch.float32).contiguous()
    bt = block_table.to(device=device, dtype=torch.int32).contiguous() if paged else None
    stream = _lib.stream_handle(device)
    if layout_k == "BSND" and not tnd:  # the reference's boundary
        st = lib.dsa_kl_bwd(
            q.data_ptr(), k.data_ptr(), _lib.ptr(qr), _lib.ptr(kr), qi.data_ptr(), ki.data_ptr(), w.data_ptr(),
            si.data_ptr(), smax.data_ptr(), ssum.data_ptr(), _lib.ptr(act_q), _lib.ptr(act_k),
            d_qi.data_ptr(), d_ki.data_ptr(), d_w.data_ptr(), loss.data_ptr(),
            B, S1, S2, N1, D, d_rope, Nidx1, D_idx, topK,
            _lib.dtype_code(query.dtype), _lib.dtype_code(weights.dtype), float(scale_value),
            ws.data_ptr(), ws_bytes, stream)
        _lib.check(st, "sparse_lightning_indexer_grad_kl_loss")
        return d_qi, d_ki, d_w, loss
    st = lib.dsa_kl_bwd_ex(
        q.data_ptr(), k.data_ptr(), _lib.ptr(qr), _lib.ptr(kr), qi.data_ptr(), ki.data_ptr(), w.data_ptr(),
        si.data_ptr(), smax.data_ptr(), ssum.data_ptr(), _lib.ptr(act_q), _lib.ptr(act_k), _lib.ptr(bt),
        d_qi.data_ptr(), d_ki.data_ptr(), d_w.data_ptr(), loss.data_ptr(),
        B, S1, S2, N1, D, d_rope, Nidx1, D_idx, topK, q_rows, kv_rows, max_blocks, page,
        _lib.LAYOUT[layout], _lib.LAYOUT[layout_k], _lib.dtype_code(query.dtype),
        _lib.dtype_code(weights.dtype), float(scale_value), ws.data_ptr(), ws_bytes, stream)
    _lib.check(st, "sparse_lightning_indexer_grad_kl_loss")
    return d_qi, d_ki, d_w, loss


class SparseLightningIndexerGradKLLossTriton(torch.nn.Module):
    """Module form (sparse_lightning_indexer_grad_kl_loss_triton.py:467-516)."""

    def __init__(self, scale_value=1.0, layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX,
                 next_tokens=INT64_MAX, deterministic=False):
        super().__init__()
        self.scale_value = scale_value
        self.layout = layout
        self.sparse_mode = sparse_mode
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens
        self.deterministic = deterministic

    def forward(self, query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                softmax_sum, query_rope=None, key_rope=None, actual_seq_qlen=None, actual_seq_klen=None,
                block_table=None):
        return sparse_lightning_indexer_grad_kl_loss_triton(
            query, key, query_index, key_index, weights, sparse_indices, softmax_max, softmax_sum,
            query_rope=query_rope, key_rope=key_rope, actual_seq_qlen=actual_seq_qlen,
            actual_seq_klen=actual_seq_klen, scale_value=self.scale_value, layout=self.layout,
            sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens, next_tokens=self.next_tokens,
            deterministic=self.deterministic, block_table=block_table)

    construct = forward
