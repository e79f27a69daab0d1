"""Host-side validation of the public API (CPU only, no kernel launch).

Every operand the kernels index is checked against the sizes they index it
by, before any launch: a malformed input raises ValueError instead of
becoming an out-of-bounds device read.  The checks run before the device
check, so CPU tensors reach them here.  Module constructors take the
reference's positional argument order.
"""
import pytest
import torch

import dsa_triton_ascend_amd as dsa
from dsa_triton_ascend_amd.sparse_flash_attention import INT64_MAX

BF = torch.bfloat16


def _bwd_args(B=1, S1=4, S2=16, N1=8, D=128, K=4):
    q = torch.zeros(B, S1, N1, D, dtype=BF)
    k = torch.zeros(B, S2, 1, D, dtype=BF)
    qr = torch.zeros(B, S1, N1, 64, dtype=BF)
    kr = torch.zeros(B, S2, 1, 64, dtype=BF)
    si = torch.zeros(B, S1, 1, K, dtype=torch.int32)
    st = torch.zeros(B, 1, S1, N1)
    return dict(query=q, key=k, value=k, sparse_indices=si, d_out=q.clone(), out=q.clone(),
                softmax_max=st, softmax_sum=st.clone(), query_rope=qr, key_rope=kr)


def _call_bwd(a):
    return dsa.sparse_flash_attention_grad_triton(
        a["query"], a["key"], a["value"], a["sparse_indices"], a["d_out"], a["out"], a["softmax_max"],
        a["softmax_sum"], query_rope=a["query_rope"], key_rope=a["key_rope"])


@pytest.mark.parametrize("field,bad,match", [
    ("sparse_indices", torch.zeros(1, 3, 1, 4, dtype=torch.int32), "sparse_indices"),
    ("softmax_max", torch.zeros(1, 1, 4, 4), "softmax_max"),
    ("softmax_sum", torch.zeros(1, 1, 2, 8), "softmax_sum"),
    ("d_out", torch.zeros(1, 4, 8, 64, dtype=BF), "d_out"),
    ("out", torch.zeros(1, 2, 8, 128, dtype=BF), "out"),
    ("query_rope", torch.zeros(1, 4, 4, 64, dtype=BF), "query_rope"),
    ("key_rope", torch.zeros(1, 8, 1, 64, dtype=BF), "key_rope"),
    ("key", torch.zeros(1, 16, 1, 256, dtype=BF), "head dim"),
])
def test_sfa_bwd_rejects_mismatched_operands(field, bad, match):
    a = _bwd_args()
    a[field] = bad
    if field == "key":
        a["value"] = bad
    with pytest.raises(ValueError, match=match):
        _call_bwd(a)


def test_sfa_bwd_wellformed_cpu_inputs_reach_the_device_check():
    with pytest.raises(ValueError, match="ROCm GPU device"):
        _call_bwd(_bwd_args())


def _fwd_args():
    q = torch.zeros(2, 3, 8, 128, dtype=BF)
    k = torch.zeros(2, 16, 1, 128, dtype=BF)
    return dict(query=q, key=k, value=k, sparse_indices=torch.zeros(2, 3, 1, 4, dtype=torch.int32),
                query_rope=torch.zeros(2, 3, 8, 64, dtype=BF), key_rope=torch.zeros(2, 16, 1, 64, dtype=BF))


@pytest.mark.parametrize("field,bad,match", [
    ("query_rope", torch.zeros(2, 3, 4, 64, dtype=BF), "query_rope"),
    ("query_rope", torch.zeros(1, 3, 8, 64, dtype=BF), "query_rope"),
    ("key_rope", torch.zeros(2, 8, 1, 64, dtype=BF), "key_rope"),
    ("key", torch.zeros(2, 16, 1, 256, dtype=BF), "key"),
    ("sparse_indices", torch.zeros(2, 2, 1, 4, dtype=torch.int32), "sparse_indices"),
])
def test_sfa_fwd_rejects_mismatched_operands(field, bad, match):
    a = _fwd_args()
    a[field] = bad
    with pytest.raises(ValueError, match=match):
        dsa.sparse_flash_attention_triton(a["query"], a["key"], a["value"], a["sparse_indices"],
                                          query_rope=a["query_rope"], key_rope=a["key_rope"])


def test_sfa_fwd_rejects_short_block_table():
    q = torch.zeros(2, 1, 8, 128, dtype=BF)
    cache = torch.zeros(4, 16, 1, 128, dtype=BF)
    rope = torch.zeros(4, 16, 1, 64, dtype=BF)
    bt = torch.zeros(1, 2, dtype=torch.int32)  # one row for two batches
    with pytest.raises(ValueError, match="block_table"):
        dsa.sparse_flash_attention_triton(q, cache, cache, torch.zeros(2, 1, 1, 4, dtype=torch.int32),
                                          block_table=bt, actual_seq_lengths_kv=[32, 32],
                                          query_rope=torch.zeros(2, 1, 8, 64, dtype=BF), key_rope=rope,
                                          layout_kv="PA_BSND")


def test_module_constructors_take_the_reference_positional_order():
    # lightning_indexer_triton.py:419-427
    li = dsa.LightningIndexerTriton(1024, 0, "TND", "TND", True, 5, 6)
    assert (li.sparse_count, li.sparse_mode, li.layout_query, li.layout_key) == (1024, 0, "TND", "TND")
    assert li.return_value is True and (li.pre_tokens, li.next_tokens) == (5, 6)
    assert dsa.LightningIndexerTriton(2048, 3, "BSND", "BSND", True).pre_tokens == INT64_MAX
    # sparse_flash_attention_triton.py:646-658
    sfa = dsa.SparseFlashAttentionTriton(0.5, 2, "TND", "PA_BSND", 3, 2, True, 7, 8, 64)
    assert (sfa.scale_value, sfa.sparse_block_size, sfa.layout_query, sfa.layout_kv, sfa.sparse_mode,
            sfa.attention_mode, sfa.return_softmax_lse, sfa.pre_tokens, sfa.next_tokens,
            sfa.block_size) == (0.5, 2, "TND", "PA_BSND", 3, 2, True, 7, 8, 64)
    # sparse_flash_attention_grad_triton.py:547-556
    g = dsa.SparseFlashAttentionGradTriton(0.5, 4, "TND", 0, 7, 8, True)
    assert (g.scale_value, g.sparse_block_size, g.layout, g.sparse_mode, g.pre_tokens, g.next_tokens,
            g.deterministic) == (0.5, 4, "TND", 0, 7, 8, True)
    # sparse_lightning_indexer_grad_kl_loss_triton.py:479-487
    kl = dsa.SparseLightningIndexerGradKLLossTriton(0.5, "BSND", 3, 7, 8, True)
    assert (kl.scale_value, kl.layout, kl.sparse_mode, kl.pre_tokens, kl.next_tokens,
            kl.deterministic) == (0.5, "BSND", 3, 7, 8, True)
    for m in (li, sfa, g, kl):
        assert type(m).construct is type(m).forward
