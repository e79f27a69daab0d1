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


# Guards.  Each public entry point runs an ordered list of rules, the first
# that fires raising its exception: the order of the checks and the exception
# types follow the reference's validators (dense_loss_backward_triton.py:
# 658-753), which is what a caller can observe; shape reads sit behind the
# rank checks that make them valid.  A rule is (fires, exception type,
# message); messages are callables so that they format lazily.
def _raise_first(rules):
    for fires, exc, msg in rules:
        if fires():
            raise exc(msg() if callable(msg) else msg)


def _index_rules(qi, ki, w, layout, sparse_mode, pre_tokens, next_tokens):
    """Layout, mode and band arguments, then the index tensors' ranks and
    shapes (reference 658-682)."""
    dims = lambda: tuple(qi.shape)  # noqa: E731  [B, S1, Nidx1, D_idx]
    return [
        (lambda: layout != "BSND", ValueError, "Only BSND layout is supported"),
        (lambda: sparse_mode != 3, ValueError, "Only sparse_mode=3 (rightDownCausal) is supported"),
        (lambda: pre_tokens != INT64_MAX or next_tokens != INT64_MAX, ValueError,
         "pre_tokens/next_tokens only support the official default value"),
        (lambda: qi.dim() != 4 or ki.dim() != 4, ValueError, "query_index and key_index must be 4D BSND tensors"),
        (lambda: w.dim() != 3, ValueError, "weights must be [B, S1, Nidx1]"),
        (lambda: ki.shape[0] != dims()[0] or ki.shape[2] != 1, ValueError, "key_index must be [B, S2, 1, D_idx]"),
        (lambda: tuple(w.shape) != dims()[:3], ValueError, "weights must be [B, S1, Nidx1]"),
        (lambda: ki.shape[3] != dims()[3], ValueError, "query_index and key_index must share D_idx"),
        (lambda: dims()[2] not in SUPPORTED_NIDX1, ValueError,
         lambda: f"Nidx1 must be one of {SUPPORTED_NIDX1}, got {dims()[2]}"),
        (lambda: dims()[3] not in SUPPORTED_D, ValueError,
         lambda: f"D_idx must be one of {SUPPORTED_D}, got {dims()[3]}"),
    ]


def _index_dtype_rules(qi, ki, w):
    """dtypes of the LSE's inputs."""
    half = (torch.float16, torch.bfloat16)
    return [
        (lambda: qi.dtype not in half, TypeError,
         lambda: f"query_index dtype must be float16 or bfloat16, got {qi.dtype}"),
        (lambda: ki.dtype != qi.dtype, TypeError, "query_index and key_index must share dtype"),
        (lambda: w.dtype not in (qi.dtype, torch.float32), TypeError,
         "weights dtype must match the index dtype or be float32"),
    ]


def _backward_rules(q, k, qi, ki, w, smax, ssum, qr, kr):
    """dtypes (reference 685-697), then the attention tensors' shapes against
    the index tensors and the statistics (720-743), then the optional rope
    pair (700-717)."""
    dt = q.dtype
    shp = lambda: tuple(q.shape)  # noqa: E731  [B, S1, N1, D]
    n2 = lambda: k.shape[2]  # noqa: E731
    stat_shape = lambda: (shp()[0], n2(), shp()[1], shp()[2] // n2())  # noqa: E731
    return [
        (lambda: dt not in (torch.float16, torch.bfloat16), TypeError,
         lambda: f"query dtype must be float16 or bfloat16, got {dt}"),
        (lambda: any(t.dtype != dt for t in (k, qi, ki)), TypeError,
         "query, key, query_index, and key_index must share dtype"),
        (lambda: w.dtype not in (dt, torch.float32), TypeError, "weights dtype must match query dtype or be float32"),
        (lambda: smax.dtype != torch.float32 or ssum.dtype != torch.float32, TypeError,
         "softmax_max and softmax_sum must be float32"),
        (lambda: k.shape[0] != shp()[0] or k.shape[3] != shp()[3], ValueError, "key must be [B, S2, N2, D_attn]"),
        (lambda: n2() <= 0 or shp()[2] % n2() != 0, ValueError, "query N1 must be divisible by key N2"),
        (lambda: tuple(qi.shape[:2]) != shp()[:2], ValueError, "query_index must share B and S1 with query"),
        (lambda: ki.shape[1] != k.shape[1], ValueError, "key_index S2 must match key S2"),
        (lambda: tuple(smax.shape) != stat_shape() or tuple(ssum.shape) != stat_shape(), ValueError,
         lambda: f"softmax_max and softmax_sum must be [B, N2, S1, G], got {tuple(smax.shape)}"),
        (lambda: shp()[3] not in SUPPORTED_D, ValueError,
         lambda: f"D_attn must be one of {SUPPORTED_D}, got {shp()[3]}"),
        (lambda: shp()[2] > _MAX_N1, ValueError, lambda: f"N1 must be <= {_MAX_N1}, got {shp()[2]}"),
        (lambda: (qr is None) != (kr is None), ValueError,
         "query_rope and key_rope must be both provided or both omitted"),
    ]


def _rope_rules(q, k, qr, kr):
    """The rope pair, when given."""
    return [
        (lambda: qr.dim() != 4 or kr.dim() != 4, ValueError, "query_rope and key_rope must be 4D BSND tensors"),
        (lambda: qr.shape[:3] != q.shape[:3], ValueError, "query_rope must share [B, S1, N1] with query"),
        (lambda: kr.shape[:3] != k.shape[:3], ValueError, "key_rope must share [B, S2, N2] with key"),
        (lambda: qr.shape[3] != kr.shape[3], ValueError, "query_rope and key_rope must share Drope"),
        (lambda: qr.shape[3] != 64, ValueError, "Only Drope=64 is supported for query_rope/key_rope"),
        (lambda: qr.dtype != q.dtype or kr.dtype != k.dtype, TypeError,
         "query_rope/key_rope dtype must match query/key dtype"),
    ]


def _guard_lse(qi, ki, w, layout, sparse_mode, pre_tokens, next_tokens):
    _raise_first(_index_rules(qi, ki, w, layout, sparse_mode, pre_tokens, next_tokens)
                 + _index_dtype_rules(qi, ki, w))


def _guard_backward(q, k, qi, ki, w, smax, ssum, layout, sparse_mode, qr, kr, pre_tokens, next_tokens):
    """Returns the rope width (0 without rope)."""
    _raise_first([(lambda: q.dim() != 4 or k.dim() != 4, ValueError, "query and key must be 4D BSND tensors")])
    _raise_first(_index_rules(qi, ki, w, layout, sparse_mode, pre_tokens, next_tokens)
                 + _backward_rules(q, k, qi, ki, w, smax, ssum, qr, kr))
    if qr is None:
        return 0
    _raise_first(_rope_rules(q, k, qr, kr))
    return qr.shape[3]


# shapes accepted for a per-row index statistic (reference 746-753)
def _row_stat(stat, B, S1, name):
    if tuple(stat.shape) not in ((B, S1), (B * S1,), (B, 1, S1), (B, 1, S1, 1)):
        raise ValueError(f"{name} must have shape [B,S1], [B*S1], [B,1,S1], or [B,1,S1,1], got {tuple(stat.shape)}")
    return stat.reshape(B * S1).contiguous()


def npu_dense_lightning_indexer_softmax_lse_triton(query_index, key_index, weights, actual_seq_qlen=None,
                                                   actual_seq_klen=None, layout="BSND", sparse_mode=3,
                                                   pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Dense indexer softmax LSE (dense_loss_backward_triton.py:812-838):
    ``(softmax_max_index, softmax_sum_index)``, each [B, 1, S1] fp32."""
    _guard_lse(query_index, key_index, weights, layout, sparse_mode, pre_tokens, next_tokens)
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
    d_rope = _guard_backward(query, key, query_index, key_index, weights, softmax_max, softmax_sum, layout,
                             sparse_mode, query_rope, key_rope, pre_tokens, next_tokens)
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
        mx = _row_stat(softmax_max_index, B, S1, "softmax_max_index")
        sm = _row_stat(softmax_sum_index, B, S1, "softmax_sum_index")
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
