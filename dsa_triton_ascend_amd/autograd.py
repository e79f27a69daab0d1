"""Autograd wiring of the DSA operators for PyTorch training.

The reference cannot differentiate through its forward op. Its docstring
gives callers a ``P.Morph`` bprop to paste in, which calls the backward op
and returns ``(dq, dk + dv, 0, dqr, dkr, ...)``
(sparse_flash_attention_grad_triton.py:30-71). ``SparseFlashAttentionFunction``
is that recipe as a ``torch.autograd.Function``:

* the forward runs ``sparse_flash_attention_triton`` with the softmax
  statistics kept for the backward;
* the backward runs the backward operator (``sparse_flash_attention_grad_triton``),
  in its merged-key form.

In MLA-absorb the value is ``key[..., :D]``: one latent feeds both the QK and
the PV product. The gradient of ``key`` is therefore the QK-path ``dk`` plus
the PV-path ``dv``. The library sums their fp32 accumulators before the
cast to the key dtype, so the merged gradient is rounded once.

``SparseLightningIndexerKLLossFunction`` makes the indexer KL loss a
differentiable scalar. The kernel (``sparse_lightning_indexer_grad_kl_loss_triton``)
computes the loss and its gradients for ``query_index``, ``key_index`` and
``weights`` in one pass. The forward returns the loss and keeps the
gradients; the backward scales them by the incoming gradient. The teacher
side (query, key, rope and the SFA statistics) carries no gradient, as in
DSA indexer training, where the KL loss trains only the indexer.
"""
import torch

from .sparse_flash_attention import INT64_MAX, sparse_flash_attention_triton
from .sparse_flash_attention_grad import _sfa_grad
from .sparse_lightning_indexer_grad_kl_loss import sparse_lightning_indexer_grad_kl_loss_triton


class SparseFlashAttentionFunction(torch.autograd.Function):
    """Differentiable SFA (MLA-absorb) over query, key, query_rope and key_rope.

    Returns ``(attention_out, softmax_max, softmax_sum)`` like the forward API;
    only ``attention_out`` carries gradient (the statistics are outputs for
    the caller's bookkeeping, as the reference's bprop ignores their dout).
    """

    @staticmethod
    def forward(ctx, query, key, query_rope, key_rope, sparse_indices, scale_value,
                actual_seq_lengths_query, actual_seq_lengths_kv, sparse_block_size, layout,
                sparse_mode, pre_tokens, next_tokens):
        out, smax, ssum = sparse_flash_attention_triton(
            query, key, None, sparse_indices, scale_value=scale_value,
            actual_seq_lengths_query=actual_seq_lengths_query,
            actual_seq_lengths_kv=actual_seq_lengths_kv, query_rope=query_rope, key_rope=key_rope,
            sparse_block_size=sparse_block_size, layout_query=layout, layout_kv=layout,
            sparse_mode=sparse_mode, pre_tokens=pre_tokens, next_tokens=next_tokens,
            return_softmax_lse=True)
        ctx.save_for_backward(query, key, query_rope, key_rope, sparse_indices, out, smax, ssum)
        ctx.args = (scale_value, actual_seq_lengths_query, actual_seq_lengths_kv, sparse_block_size,
                    layout, sparse_mode, pre_tokens, next_tokens)
        ctx.mark_non_differentiable(smax, ssum)
        return out, smax, ssum

    @staticmethod
    def backward(ctx, d_out, d_smax, d_ssum):
        query, key, query_rope, key_rope, sparse_indices, out, smax, ssum = ctx.saved_tensors
        scale_value, act_q, act_k, bs, layout, mode, pre, nxt = ctx.args
        if d_out is None:
            return (None,) * 13
        # shared latent: d_key = dk (QK path) + dv (PV path), summed in fp32
        dq, d_key, _, dqr, dkr = _sfa_grad(
            query, key, key, sparse_indices, d_out.contiguous(), out, smax, ssum, scale_value,
            query_rope, key_rope, act_q, act_k, bs, layout, mode, pre, nxt, False,
            merge_kv=True)
        return dq, d_key, dqr, dkr, None, None, None, None, None, None, None, None, None


def sparse_flash_attention_train(query, key, sparse_indices, scale_value=1.0, query_rope=None,
                                 key_rope=None, actual_seq_lengths_query=None,
                                 actual_seq_lengths_kv=None, sparse_block_size=1, layout="BSND",
                                 sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Differentiable SFA forward for training (BSND or TND; the backward has
    no paged-KV form, as in the reference).  Returns
    ``(attention_out, softmax_max, softmax_sum)``."""
    if layout not in ("BSND", "TND"):
        raise ValueError(f"layout must be BSND or TND for training, got {layout}")
    return SparseFlashAttentionFunction.apply(
        query, key, query_rope, key_rope, sparse_indices, scale_value, actual_seq_lengths_query,
        actual_seq_lengths_kv, sparse_block_size, layout, sparse_mode, pre_tokens, next_tokens)


class SparseLightningIndexerKLLossFunction(torch.autograd.Function):
    """Differentiable indexer KL loss over query_index, key_index and weights."""

    @staticmethod
    def forward(ctx, query_index, key_index, weights, query, key, sparse_indices, softmax_max,
                softmax_sum, query_rope, key_rope, actual_seq_qlen, actual_seq_klen, scale_value,
                sparse_mode):
        d_qi, d_ki, d_w, loss = sparse_lightning_indexer_grad_kl_loss_triton(
            query, key, query_index, key_index, weights, sparse_indices, softmax_max, softmax_sum,
            query_rope=query_rope, key_rope=key_rope, actual_seq_qlen=actual_seq_qlen,
            actual_seq_klen=actual_seq_klen, scale_value=scale_value, sparse_mode=sparse_mode)
        ctx.save_for_backward(d_qi, d_ki, d_w)
        return loss

    @staticmethod
    def backward(ctx, d_loss):
        d_qi, d_ki, d_w = ctx.saved_tensors
        g = d_loss.reshape(()).float()

        def scaled(t):
            return (t.float() * g).to(t.dtype)

        return scaled(d_qi), scaled(d_ki), scaled(d_w), *([None] * 11)


def sparse_lightning_indexer_kl_loss(query_index, key_index, weights, query, key, sparse_indices,
                                     softmax_max, softmax_sum, query_rope=None, key_rope=None,
                                     actual_seq_qlen=None, actual_seq_klen=None, scale_value=1.0,
                                     sparse_mode=3):
    """Indexer KL loss as a differentiable scalar ([1] fp32, summed over
    rows as the reference's loss, sparse_lightning_indexer_grad_kl_loss_triton.py:216);
    ``loss.backward()`` fills the gradients of query_index, key_index and weights."""
    return SparseLightningIndexerKLLossFunction.apply(
        query_index, key_index, weights, query.detach(), key.detach(), sparse_indices,
        softmax_max.detach(), softmax_sum.detach(),
        None if query_rope is None else query_rope.detach(),
        None if key_rope is None else key_rope.detach(),
        actual_seq_qlen, actual_seq_klen, scale_value, sparse_mode)


__all__ = ["SparseFlashAttentionFunction", "sparse_flash_attention_train",
           "SparseLightningIndexerKLLossFunction", "sparse_lightning_indexer_kl_loss", "INT64_MAX"]
