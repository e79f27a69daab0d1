"""Sparse lightning-indexer KL-loss backward on MI355X: the reference's
public API over the HIP library.

Drop-in for ``sparse_lightning_indexer_grad_kl_loss_triton`` /
``SparseLightningIndexerGradKLLossTriton``
(sparse_lightning_indexer_grad_kl_loss_triton.py:467-556): same argument
names and defaults, the same guards (ValueError for a layout other than
BSND or a sparse_mode other than 3, AssertionError when Nidx2 != 1, lines
534-538), missing rope treated as zero rope (543-546), and the same return
tuple ``(d_query_index, d_key_index, d_weights, loss)`` with d_query_index /
d_key_index / d_weights in the dtype of query_index / key_index / weights
and loss a [1] fp32 tensor (the sum over all query rows).  pre_tokens,
next_tokens and deterministic are accepted and ignored, as in the
reference; every output of this implementation is deterministic.
"""
import torch

from . import _lib
from .sparse_flash_attention import INT64_MAX, _check_device, _seq_tensor, _VALID_D

_D_ROPE = 64
_D_IDX = 128
_MAX_NIDX = 64
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
):
    """Indexer KL-loss backward; see module docstring."""
    if layout != "BSND":
        raise ValueError("Only BSND layout is supported")
    if sparse_mode != 3:
        raise ValueError("Only sparse_mode=3 (rightDownCausal) is supported")
    assert sparse_indices.shape[2] == 1, "Nidx2 must be 1 (MQA constraint)"
    device = _check_device(query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                           softmax_sum, query_rope, key_rope)
    B, S1, N1, D = query.shape
    S2 = key.shape[1]
    if key.dim() != 4 or key.shape[2] != 1:
        raise ValueError("Only N2=1 (MQA) is supported")
    Nidx1, D_idx = query_index.shape[2], query_index.shape[3]
    if key_index.dim() != 4 or key_index.shape[2] != 1:
        raise ValueError("Only Nidx2=1 is supported for key_index")
    topK = sparse_indices.shape[3]
    if D not in _VALID_D:
        raise ValueError(f"D must be one of {_VALID_D}, got {D}")
    if D_idx != _D_IDX:
        raise ValueError(f"index head dim must be {_D_IDX}, got {D_idx}")
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
        d_rope = query_rope.shape[3]
        if d_rope != _D_ROPE or key_rope.shape[3] != _D_ROPE:
            raise ValueError(f"rope dim must be {_D_ROPE}, got {d_rope}")
    for t, nm in ((key, "key"), (query_index, "query_index"), (key_index, "key_index"),
                  (query_rope, "query_rope"), (key_rope, "key_rope")):
        if t is not None and t.dtype != query.dtype:
            raise ValueError(f"{nm} must have the query dtype")
    if weights.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError("weights dtype must be float32, bfloat16 or float16")

    act_q = _seq_tensor(actual_seq_qlen, device)
    act_k = _seq_tensor(actual_seq_klen, device)
    d_qi = torch.empty_like(query_index)
    d_ki = torch.empty_like(key_index)
    d_w = torch.empty_like(weights)
    loss = torch.empty(1, dtype=torch.float32, device=device)
    lib = _lib.load()
    ws_bytes = lib.dsa_kl_bwd_workspace_size(B, S1, S2, topK, D_idx)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    q, k, qi, ki, w = (t.contiguous() for t in (query, key, query_index, key_index, weights))
    qr = query_rope.contiguous() if d_rope else None
    kr = key_rope.contiguous() if d_rope else None
    si = sparse_indices.to(torch.int32).contiguous()
    smax = softmax_max.to(torch.float32).contiguous()
    ssum = softmax_sum.to(torch.float32).contiguous()
    st = lib.dsa_kl_bwd(
        q.data_ptr(), k.data_ptr(), _lib.ptr(qr), _lib.ptr(kr), qi.data_ptr(), ki.data_ptr(), w.data_ptr(),
        si.data_ptr(), smax.data_ptr(), ssum.data_ptr(), _lib.ptr(act_q), _lib.ptr(act_k),
        d_qi.data_ptr(), d_ki.data_ptr(), d_w.data_ptr(), loss.data_ptr(),
        B, S1, S2, N1, D, d_rope, Nidx1, D_idx, topK,
        _lib.dtype_code(query.dtype), _lib.dtype_code(weights.dtype), float(scale_value),
        ws.data_ptr(), ws_bytes, _lib.stream_handle(device))
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
                softmax_sum, query_rope=None, key_rope=None, actual_seq_qlen=None, actual_seq_klen=None):
        return sparse_lightning_indexer_grad_kl_loss_triton(
            query, key, query_index, key_index, weights, sparse_indices, softmax_max, softmax_sum,
            query_rope=query_rope, key_rope=key_rope, actual_seq_qlen=actual_seq_qlen,
            actual_seq_klen=actual_seq_klen, scale_value=self.scale_value, layout=self.layout,
            sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens, next_tokens=self.next_tokens,
            deterministic=self.deterministic)
