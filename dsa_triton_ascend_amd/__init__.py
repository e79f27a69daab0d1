"""MI355X-native DSA operator set (gfx950 HIP kernels behind a C ABI).

Public API, mirroring the reference's operator modules:

* ``sparse_flash_attention_triton`` / ``SparseFlashAttentionTriton``
* ``lightning_indexer_triton`` / ``LightningIndexerTriton``
"""
from .sparse_flash_attention import (  # noqa: F401
    INT64_MAX,
    SparseFlashAttentionTriton,
    sparse_flash_attention_triton,
)

from .lightning_indexer import (  # noqa: F401
    LightningIndexerTriton,
    lightning_indexer_triton,
)

sparse_flash_attention = sparse_flash_attention_triton
lightning_indexer = lightning_indexer_triton
