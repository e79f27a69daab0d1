"""CPU oracle for the DSA operator set -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's CPU goldens and the semantics
of its device kernels.  It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
only as the checker.  The product path (``dsa_triton_ascend_amd``) never
imports it and has no CPU fallback: it fails loudly when the HIP library is
missing.

Modules and the reference code each one restates:

* ``common``     bf16 rounding, token-position scan, layout helpers
                 (sparse_flash_attention_numpy.py:26-60,
                  sparse_flash_attention_triton.py:338-421)
* ``sfa``        sparse flash attention forward
                 (sparse_flash_attention_numpy.py:63-160,
                  sparse_flash_attention_triton.py:483-641)
* ``sfa_grad``   sparse flash attention backward
                 (sparse_flash_attention_grad_numpy.py:34-143,
                  sparse_flash_attention_grad_triton.py:382-541)
* ``indexer``    lightning-indexer score and stable top-k
                 (lightning_indexer_triton.py:147-280, 339-357, 462-550)
* ``kl``         sparse lightning-indexer KL-loss backward
                 (sli_grad_kl_loss_numpy.py:16-152,
                  sparse_lightning_indexer_grad_kl_loss_triton.py:39-327)
* ``dense_kl``   dense indexer softmax LSE and dense KL-loss backward
                 (dense_loss_backward_triton.py:129-397,
                  test_dense_loss_backward_triton.py:101-138)

How each function is pinned (checks that are not a retyping of its formula)
is listed in the test files ``tests/test_oracle_*.py``.  Every function here
is pinned by at least one of: the committed golden fixtures written by the
reference's own numpy goldens (``tests/golden/``), a brute-force fp64
implementation written independently, finite differences, closed-form cases
or library routines (torch bf16 casts, ``np.lexsort``, ``torch.sort``).
"""
