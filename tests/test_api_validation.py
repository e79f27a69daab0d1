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


# ---------------------------------------------------------------------------
# dense warm-up stage: every guard, in the reference's order (the first
# failing check decides the exception type; dense_loss_backward_triton.py:
# 658-753), on CPU tensors (the guards run before the device check)
# ---------------------------------------------------------------------------
def _dense_ok():
    z = lambda *s, dt=BF: torch.zeros(*s, dtype=dt)  # noqa: E731
    return dict(q=z(1, 2, 4, 128), k=z(1, 8, 1, 128), qi=z(1, 2, 32, 128), ki=z(1, 8, 1, 128),
                w=z(1, 2, 32, dt=torch.float32), smax=z(1, 1, 2, 4, dt=torch.float32),
                ssum=z(1, 1, 2, 4, dt=torch.float32), qr=z(1, 2, 4, 64), kr=z(1, 8, 1, 64))


def _dense_bwd(a, **kw):
    return dsa.dense_loss_backward_triton(a["q"], a["k"], a["qi"], a["ki"], a["w"], a["smax"], a["ssum"],
                                          query_rope=a["qr"], key_rope=a["kr"], **kw)


@pytest.mark.parametrize("change,kw,exc", [
    ({}, {"layout": "TND"}, ValueError),
    ({}, {"sparse_mode": 0}, ValueError),
    ({}, {"pre_tokens": 5}, ValueError),
    ({"q": torch.zeros(2, 4, 128, dtype=BF)}, {}, ValueError),                # query rank
    ({"qi": torch.zeros(2, 32, 128, dtype=BF)}, {}, ValueError),              # index rank
    ({"w": torch.zeros(1, 2, 32, 1)}, {}, ValueError),                        # weights rank
    ({"ki": torch.zeros(1, 8, 2, 128, dtype=BF)}, {}, ValueError),            # key_index N2 != 1
    ({"w": torch.zeros(1, 2, 16)}, {}, ValueError),                           # weights shape
    ({"ki": torch.zeros(1, 8, 1, 256, dtype=BF)}, {}, ValueError),            # D_idx differs
    ({"qi": torch.zeros(1, 2, 16, 128, dtype=BF), "w": torch.zeros(1, 2, 16)}, {}, ValueError),  # Nidx1
    ({"qi": torch.zeros(1, 2, 32, 64, dtype=BF), "ki": torch.zeros(1, 8, 1, 64, dtype=BF)}, {}, ValueError),
    ({"q": torch.zeros(1, 2, 4, 128)}, {}, TypeError),                        # query dtype
    ({"k": torch.zeros(1, 8, 1, 128, dtype=torch.float16)}, {}, TypeError),  # shared dtype
    ({"w": torch.zeros(1, 2, 32, dtype=torch.float16)}, {}, TypeError),      # weights dtype
    ({"smax": torch.zeros(1, 1, 2, 4, dtype=BF)}, {}, TypeError),             # stats dtype
    ({"k": torch.zeros(1, 8, 1, 256, dtype=BF)}, {}, ValueError),             # key D
    ({"k": torch.zeros(1, 8, 3, 128, dtype=BF)}, {}, ValueError),             # N1 % N2
    ({"qi": torch.zeros(1, 3, 32, 128, dtype=BF), "w": torch.zeros(1, 3, 32)}, {}, ValueError),  # S1
    ({"ki": torch.zeros(1, 9, 1, 128, dtype=BF)}, {}, ValueError),            # key_index S2
    ({"smax": torch.zeros(1, 1, 4, 2)}, {}, ValueError),                      # stats shape
    ({"q": torch.zeros(1, 2, 4, 96, dtype=BF), "k": torch.zeros(1, 8, 1, 96, dtype=BF)}, {}, ValueError),
    ({"q": torch.zeros(1, 2, 256, 128, dtype=BF), "smax": torch.zeros(1, 1, 2, 256),
      "ssum": torch.zeros(1, 1, 2, 256), "qr": torch.zeros(1, 2, 256, 64, dtype=BF)}, {}, ValueError),  # N1
    ({"kr": None}, {}, ValueError),                                           # rope pair
    ({"qr": torch.zeros(1, 2, 4, 32, dtype=BF), "kr": torch.zeros(1, 8, 1, 32, dtype=BF)}, {}, ValueError),
    ({"qr": torch.zeros(1, 2, 4, 64)}, {}, TypeError),                        # rope dtype
    ({}, {"softmax_max_index": torch.zeros(1, 2)}, ValueError),               # one of the two stats
])
def test_dense_guards_in_order(change, kw, exc):
    a = _dense_ok()
    a.update(change)
    with pytest.raises(exc) as ei:
        _dense_bwd(a, **kw)
    assert "GPU device" not in str(ei.value), "a guard must fire before the device check"


def test_dense_valid_arguments_reach_the_device_check():
    """The unchanged arguments pass every guard (so each case above fails on
    its own guard, not on the CPU tensors)."""
    with pytest.raises(ValueError, match="GPU device"):
        _dense_bwd(_dense_ok())
    a = _dense_ok()
    with pytest.raises(ValueError, match="GPU device"):
        dsa.dense_lightning_indexer_softmax_lse_triton(a["qi"], a["ki"], a["w"])


def test_dense_guards_order_layout_before_dtype():
    """Several faults at once: the earliest check in the reference's order
    decides (a bad layout is a ValueError even with an fp32 query)."""
    a = _dense_ok()
    a["q"] = a["q"].float()
    with pytest.raises(ValueError, match="BSND"):
        _dense_bwd(a, layout="TND")
    with pytest.raises(TypeError):  # dtype before the attention shapes
        a["k"] = torch.zeros(1, 8, 3, 128, dtype=BF)
        _dense_bwd(a)


def test_dense_lse_guards():
    a = _dense_ok()
    f = dsa.dense_lightning_indexer_softmax_lse_triton
    with pytest.raises(ValueError, match="BSND"):
        f(a["qi"], a["ki"], a["w"], layout="TND")
    with pytest.raises(TypeError):
        f(a["qi"].float(), a["ki"].float(), a["w"])
    with pytest.raises(TypeError):
        f(a["qi"], a["ki"].half(), a["w"])
    with pytest.raises(TypeError):
        f(a["qi"], a["ki"], a["w"].half())
