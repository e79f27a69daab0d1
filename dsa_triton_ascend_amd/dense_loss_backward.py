"""Dense lightning-indexer softmax LSE and dense KL-loss backward on MI355X
(the dense warm-up stage of DSA indexer training): the reference's public
API over the HIP library.

Drop-in for dense_loss_backward_triton.py:752-988:
``dense_loss_backward_triton``, ``dense_lightning_indexer_softmax_lse_triton``
/ ``npu_dense_lightning_indexer_softmax_lse_triton``,
``dense_lightning_indexer_grad_kl_loss_triton`` /
``npu_dense_lightning_indexer_grad_kl_loss_triton`` and the module forms
``DenseLightningIndexerSoftmaxLseTriton``, ``DenseLossBackwardTriton`` and
``DenseLightningIndexerGradKLLossTriton``.  Same argument names and
defaults, the same guards (ValueError for a layout other than BSND, a
sparse_mode other than 3, non-default pre/next tokens or unsupported
shapes; TypeError for dtypes; lines 658-743), the same return values: the
LSE as two [B, 1, S1] fp32 tensors, the backward as ``(dQueryIndex,
dKeyIndex, dWeights, loss)`` in the index / weights dtypes with a [1] fp32
loss.  When the index statistics are omitted the backward computes them
(the reference's compatibility path, 794-809).

One bound the reference does not have: N1 <= 128 (the teacher kernel puts
the heads of a query row on 8 waves x 16 MFMA rows).  dKeyIndex and the loss
are deterministic here (the reference adds them with atomics, 317, 397).
"""
import torch

from . import _lib
from .sparse_flash_attention import INT64_MAX, _check_device, _seq_tensor

SUPPORTED_D = (128, 256, 512)
SUPPORTED_NIDX1 = (32, 64, 128)
_MAX_N1 = 128


def _check_in(name, value, supported):
    if value not in supported:
        raise ValueError(f"{name} must be one of {supported}, got {value}")


def _validate_dense_index_inputs(query_index, key_index, weights, layout, sparse_mode,
                                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """dense_loss_backward_triton.py:658-682."""
    if layout != "BSND":
        raise ValueError("Only BSND layout is supported")
    if sparse_mode != 3:
        raise ValueError("Only sparse_mode=3 (rightDownCausal) is supported")
    if pre_tokens != INT64_MAX or next_tokens != INT64_MAX:
        raise ValueError("pre_tokens/next_tokens only support the official default value")
    if query_index.dim() != 4 or key_index.dim() != 4:
        raise ValueError("query_index and key_index must be 4D BSND tensors")
    if weights.dim() != 3:
        raise ValueError("weights must be [B, S1, Nidx1]")
    B, S1, Nidx1, D_idx = query_index.shape
    if key_index.shape[0] != B or key_index.shape[2] != 1:
        raise ValueError("key_index must be [B, S2, 1, D_idx]")
    if tuple(weights.shape) != (B, S1, Nidx1):
        raise ValueError("weights must be [B, S1, Nidx1]")
    if key_index.shape[3] != D_idx:
        raise ValueError("query_index and key_index must share D_idx")
    _check_in("Nidx1", Nidx1, SUPPORTED_NIDX1)
    _check_in("D_idx", D_idx, SUPPORTED_D)


def _validate_index_dtypes(query_index, key_index, weights):
    if query_index.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"query_index dtype must be float16 or bfloat16, got {query_index.dtype}")
    if key_index.dtype != query_index.dtype:
        raise TypeError("query_index and key_index must share dtype")
    if weights.dtype not in (query_index.dtype, torch.float32):
        raise TypeError("weights dtype must match the index dtype or be float32")


def _validate_dense_dtypes(query, key, query_index, key_index, weights, softmax_max, softmax_sum):
    """dense_loss_backward_triton.py:685-697."""
    data_dtype = query.dtype
    if data_dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"query dtype must be float16 or bfloat16, got {data_dtype}")
    if key.dtype != data_dtype or query_index.dtype != data_dtype or key_index.dtype != data_dtype:
        raise TypeError("query, key, query_index, and key_index must share dtype")
    if weights.dtype != data_dtype and weights.dtype != torch.float32:
        raise TypeError("weights dtype must match query dtype or be float32")
    if softmax_max.dtype != torch.float32 or softmax_sum.dtype != torch.float32:
        raise TypeError("softmax_max and softmax_sum must be float32")


def _validate_rope_inputs(query, key, query_rope, key_rope):
    """dense_loss_backward_triton.py:700-717."""
    if (query_rope is None) != (key_rope is None):
        raise ValueError("query_rope and key_rope must be both provided or both omitted")
    if query_rope is None:
        return 0
    if query_rope.dim() != 4 or key_rope.dim() != 4:
        raise ValueError("query_rope and key_rope must be 4D BSND tensors")
    if query_rope.shape[:3] != query.shape[:3]:
        raise ValueError("query_rope must share [B, S1, N1] with query")
    if key_rope.shape[:3] != key.shape[:3]:
        raise ValueError("key_rope must share [B, S2, N2] with key")
    if query_rope.shape[3] != key_rope.shape[3]:
        raise ValueError("query_rope and key_rope must share Drope")
    if query_rope.shape[3] != 64:
        raise ValueError("Only Drope=64 is supported for query_rope/key_rope")
    if query_rope.dtype != query.dtype or key_rope.dtype != key.dtype:
        raise TypeError("query_rope/key_rope dtype must match query/key dtype")
    return query_rope.shape[3]


def _validate_dense_inputs(query, key, query_index, key_index, weights, softmax_max, softmax_sum, layout,
                           sparse_mode, query_rope=None, key_rope=None, pre_tokens=INT64_MAX,
                           next_tokens=INT64_MAX):
    """dense_loss_backward_triton.py:720-743."""
    if query.dim() != 4 or key.dim() != 4:
        raise ValueError("query and key must be 4D BSND tensors")
    _validate_dense_index_inputs(query_index, key_index, weights, layout, sparse_mode,
                                 pre_tokens=pre_tokens, next_tokens=next_tokens)
    _validate_dense_dtypes(query, key, query_index, key_index, weights, softmax_max, softmax_sum)
    B, S1, N1, D = query.shape
    if key.shape[0] != B or key.shape[3] != D:
        raise ValueError("key must be [B, S2, N2, D_attn]")
    N2 = key.shape[2]
    if N2 <= 0 or N1 % N2 != 0:
        raise ValueError("query N1 must be divisible by key N2")
    if query_index.shape[0] != B or query_index.shape[1] != S1:
        raise ValueError("query_index must share B and S1 with query")
    if key_index.shape[1] != key.shape[1]:
        raise ValueError("key_index S2 must match key S2")
    softmax_shape = (B, N2, S1, N1 // N2)
    if tuple(softmax_max.shape) != softmax_shape or tuple(softmax_sum.shape) != softmax_shape:
        raise ValueError(f"softmax_max and softmax_sum must be [B, N2, S1, G], got {tuple(softmax_max.shape)}")
    _check_in("D_attn", D, SUPPORTED_D)
    if N1 > _MAX_N1:
        raise ValueError(f"N1 must be <= {_MAX_N1}, got {N1}")
    return _validate_rope_inputs(query, key, query_rope, key_rope)


def _reshape_dense_index_stat(stat, B, S1, name):
    """dense_loss_backward_triton.py:746-753."""
    if tuple(stat.shape) in ((B, S1), (B * S1,), (B, 1, S1), (B, 1, S1, 1)):
        return stat.reshape(B * S1).contiguous()
    raise ValueError(f"{name} must have shape [B,S1], [B*S1], [B,1,S1], or [B,1,S1,1], got {tuple(stat.shape)}")


def npu_dense_lightning_indexer_softmax_lse_triton(query_index, key_index, weights, actual_seq_qlen=None,
                                                   actual_seq_klen=None, layout="BSND", sparse_mode=3,
                                                   pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Dense indexer softmax LSE (dense_loss_backward_triton.py:812-838):
    ``(softmax_max_index, softmax_sum_index)``, each [B, 1, S1] fp32."""
    _validate_dense_index_inputs(query_index, key_index, weights, layout, sparse_mode,
                                 pre_tokens=pre_tokens, next_tokens=next_tokens)
    _validate_index_dtypes(query_index, key_index, weights)
    device = _check_device(query_index, key_index, weights)
    B, S1, Nidx1, D_idx = query_index.shape
    S2 = key_index.shape[1]
    act_q = _seq_tensor(actual_seq_qlen, device)
    act_k = _seq_tensor(actual_seq_klen, device)
    mx = torch.empty(B, 1, S1, dtype=torch.float32, device=device)
    sm = torch.empty(B, 1, S1, dtype=torch.float32, device=device)
    qi, ki, w = (t.contiguous() for t in (query_index, key_index, weights))
    lib = _lib.load()
    st = lib.dsa_dense_li_softmax_lse(
        qi.data_ptr(), ki.data_ptr(), w.data_ptr(), _lib.ptr(act_q), _lib.ptr(act_k), mx.data_ptr(),
        sm.data_ptr(), B, S1, S2, Nidx1, D_idx, _lib.dtype_code(qi.dtype), _lib.dtype_code(w.dtype),
        _lib.stream_handle(device))
    _lib.check(st, "dense_lightning_indexer_softmax_lse")
    return mx, sm


def dense_lightning_indexer_softmax_lse_triton(query_index, key_index, weights, actual_seq_qlen=None,
                                               actual_seq_klen=None, layout="BSND", sparse_mode=3,
                                               pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Alias of ``npu_dense_lightning_indexer_softmax_lse_triton`` (841-859)."""
    return npu_dense_lightning_indexer_softmax_lse_triton(
        query_index, key_index, weights, actual_seq_qlen=actual_seq_qlen, actual_seq_klen=actual_seq_klen,
        layout=layout, sparse_mode=sparse_mode, pre_tokens=pre_tokens, next_tokens=next_tokens)


def dense_loss_backward_triton(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                               softmax_max_index=None, softmax_sum_index=None, scale_value=1.0,
                               query_rope=None, key_rope=None, actual_seq_qlen=None, actual_seq_klen=None,
                               layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Dense KL-loss backward (dense_loss_backward_triton.py:756-809):
    ``(dQueryIndex, dKeyIndex, dWeights, loss)``."""
    d_rope = _validate_dense_inputs(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                                    layout, sparse_mode, query_rope=query_rope, key_rope=key_rope,
                                    pre_tokens=pre_tokens, next_tokens=next_tokens)
    if (softmax_max_index is None) != (softmax_sum_index is None):
        raise ValueError("softmax_max_index and softmax_sum_index must be both provided or both omitted")
    device = _check_device(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                           softmax_max_index, softmax_sum_index, query_rope, key_rope)
    B, S1, N1, D = query.shape
    S2, N2 = key.shape[1], key.shape[2]
    Nidx1, D_idx = query_index.shape[2], query_index.shape[3]
    mx = sm = None
    if softmax_max_index is not None:
        if softmax_max_index.dtype != torch.float32 or softmax_sum_index.dtype != torch.float32:
            raise TypeError("softmax_max_index and softmax_sum_index must be float32")
        mx = _reshape_dense_index_stat(softmax_max_index, B, S1, "softmax_max_index")
        sm = _reshape_dense_index_stat(softmax_sum_index, B, S1, "softmax_sum_index")
    act_q = _seq_tensor(actual_seq_qlen, device)
    act_k = _seq_tensor(actual_seq_klen, device)
    d_qi = torch.empty_like(query_index)
    d_ki = torch.empty_like(key_index)
    d_w = torch.empty_like(weights)
    loss = torch.empty(1, dtype=torch.float32, device=device)
    lib = _lib.load()
    ws_bytes = lib.dsa_dense_kl_bwd_workspace_size(B, S1, S2, D_idx)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    q, k, qi, ki, w = (t.contiguous() for t in (query, key, query_index, key_index, weights))
    qr = query_rope.contiguous() if d_rope else None
    kr = key_rope.contiguous() if d_rope else None
    smax, ssum = softmax_max.contiguous(), softmax_sum.contiguous()
    st = lib.dsa_dense_kl_bwd(
        q.data_ptr(), k.data_ptr(), _lib.ptr(qr), _lib.ptr(kr), qi.data_ptr(), ki.data_ptr(), w.data_ptr(),
        smax.data_ptr(), ssum.data_ptr(), _lib.ptr(mx), _lib.ptr(sm), _lib.ptr(act_q), _lib.ptr(act_k),
        d_qi.data_ptr(), d_ki.data_ptr(), d_w.data_ptr(), loss.data_ptr(),
        B, S1, S2, N1, N2, D, d_rope, Nidx1, D_idx, _lib.dtype_code(query.dtype), _lib.dtype_code(weights.dtype),
        float(scale_value), ws.data_ptr(), ws_bytes, _lib.stream_handle(device))
    _lib.check(st, "dense_loss_backward")
    return d_qi, d_ki, d_w, loss


def dense_lightning_indexer_grad_kl_loss_triton(query, key, query_index, key_index, weights, softmax_max,
                                                softmax_sum, softmax_max_index, softmax_sum_index, scale_value,
                                                query_rope=None, key_rope=None, actual_seq_qlen=None,
                                                actual_seq_klen=None, layout="BSND", sparse_mode=3,
                                                pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Official-style wrapper (dense_loss_backward_triton.py:862-890)."""
    return dense_loss_backward_triton(
        query, key, query_index, key_index, weights, softmax_max, softmax_sum, softmax_max_index,
        softmax_sum_index, scale_value, query_rope=query_rope, key_rope=key_rope,
        actual_seq_qlen=actual_seq_qlen, actual_seq_klen=actual_seq_klen, layout=layout,
        sparse_mode=sparse_mode, pre_tokens=pre_tokens, next_tokens=next_tokens)


def npu_dense_lightning_indexer_grad_kl_loss_triton(query, key, query_index, key_index, weights, softmax_max,
                                                    softmax_sum, softmax_max_index, softmax_sum_index,
                                                    scale_value, query_rope=None, key_rope=None,
                                                    actual_seq_qlen=None, actual_seq_klen=None, layout="BSND",
                                                    sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Alias (dense_loss_backward_triton.py:893-921)."""
    return dense_lightning_indexer_grad_kl_loss_triton(
        query, key, query_index, key_index, weights, softmax_max, softmax_sum, softmax_max_index,
        softmax_sum_index, scale_value, query_rope=query_rope, key_rope=key_rope,
        actual_seq_qlen=actual_seq_qlen, actual_seq_klen=actual_seq_klen, layout=layout,
        sparse_mode=sparse_mode, pre_tokens=pre_tokens, next_tokens=next_tokens)


class DenseLightningIndexerSoftmaxLseTriton(torch.nn.Module):
    """Module form (dense_loss_backward_triton.py:924-945)."""

    def __init__(self, layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
        super().__init__()
        self.layout = layout
        self.sparse_mode = sparse_mode
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens

    def forward(self, query_index, key_index, weights, actual_seq_qlen=None, actual_seq_klen=None):
        return npu_dense_lightning_indexer_softmax_lse_triton(
            query_index, key_index, weights, actual_seq_qlen=actual_seq_qlen, actual_seq_klen=actual_seq_klen,
            layout=self.layout, sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens,
            next_tokens=self.next_tokens)

    construct = forward


class DenseLossBackwardTriton(torch.nn.Module):
    """Module form (dense_loss_backward_triton.py:948-984)."""

    def __init__(self, scale_value=1.0, layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX,
                 next_tokens=INT64_MAX):
        super().__init__()
        self.scale_value = scale_value
        self.layout = layout
        self.sparse_mode = sparse_mode
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens

    def forward(self, query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                softmax_max_index=None, softmax_sum_index=None, scale_value=None, query_rope=None,
                key_rope=None, actual_seq_qlen=None, actual_seq_klen=None):
        effective_scale = self.scale_value if scale_value is None else scale_value
        return dense_loss_backward_triton(
            query, key, query_index, key_index, weights, softmax_max, softmax_sum, softmax_max_index,
            softmax_sum_index, effective_scale, query_rope=query_rope, key_rope=key_rope,
            actual_seq_qlen=actual_seq_qlen, actual_seq_klen=actual_seq_klen, layout=self.layout,
            sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens, next_tokens=self.next_tokens)

    construct = forward


class DenseLightningIndexerGradKLLossTriton(DenseLossBackwardTriton):
    """Alias module (dense_loss_backward_triton.py:987-988)."""


__all__ = [
    "dense_loss_backward_triton", "npu_dense_lightning_indexer_softmax_lse_triton",
    "dense_lightning_indexer_softmax_lse_triton", "dense_lightning_indexer_grad_kl_loss_triton",
    "npu_dense_lightning_indexer_grad_kl_loss_triton", "DenseLightningIndexerSoftmaxLseTriton",
    "DenseLossBackwardTriton", "DenseLightningIndexerGradKLLossTriton",
]
