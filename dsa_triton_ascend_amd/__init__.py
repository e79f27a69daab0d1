"""MI355X-native DSA operator set (gfx950 HIP kernels behind a C ABI).

Public API, mirroring the reference's operator modules:

* ``sparse_flash_attention_triton`` / ``SparseFlashAttentionTriton``
* ``sparse_flash_attention_grad_triton`` / ``SparseFlashAttentionGradTriton``
* ``lightning_indexer_triton`` / ``LightningIndexerTriton``
* ``sparse_lightning_indexer_grad_kl_loss_triton`` /
  ``SparseLightningIndexerGradKLLossTriton``
* the dense warm-up stage: ``dense_lightning_indexer_softmax_lse_triton`` /
  ``DenseLightningIndexerSoftmaxLseTriton`` and ``dense_loss_backward_triton``
  / ``DenseLightningIndexerGradKLLossTriton`` (with their ``npu_`` aliases)

and the autograd pairing for training (``autograd.py``):
``sparse_flash_attention_train`` / ``SparseFlashAttentionFunction`` and
``sparse_lightning_indexer_kl_loss`` / ``SparseLightningIndexerKLLossFunction``.
"""
from .sparse_flash_attention import (  # noqa: F401
    INT64_MAX,
    SparseFlashAttentionTriton,
    sparse_flash_attention_triton,
)

from .sparse_flash_attention_grad import (  # noqa: F401
    SparseFlashAttentionGradTriton,
    sparse_flash_attention_grad_triton,
)

from .lightning_indexer import (  # noqa: F401
    LightningIndexerTriton,
    lightning_indexer_triton,
)

from .sparse_lightning_indexer_grad_kl_loss import (  # noqa: F401
    SparseLightningIndexerGradKLLossTriton,
    sparse_lightning_indexer_grad_kl_loss_triton,
)

from .dense_loss_backward import (  # noqa: F401
    DenseLightningIndexerGradKLLossTriton,
    DenseLightningIndexerSoftmaxLseTriton,
    DenseLossBackwardTriton,
    dense_lightning_indexer_grad_kl_loss_triton,
    dense_lightning_indexer_softmax_lse_triton,
    dense_loss_backward_triton,
    npu_dense_lightning_indexer_grad_kl_loss_triton,
    npu_dense_lightning_indexer_softmax_lse_triton,
)

sparse_flash_attention = sparse_flash_attention_triton
lightning_indexer = lightning_indexer_triton
sparse_flash_attention_grad = sparse_flash_attention_grad_triton
sparse_lightning_indexer_grad_kl_loss = sparse_lightning_indexer_grad_kl_loss_triton

from .autograd import (  # noqa: F401,E402
    SparseFlashAttentionFunction,
    SparseLightningIndexerKLLossFunction,
    sparse_flash_attention_train,
    sparse_lightning_indexer_kl_loss,
)
