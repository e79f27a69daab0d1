"""CPU tests of the C-ABI library: it loads without a GPU, exports every
symbol include/dsa_capi.h declares, and rejects bad arguments with the right
status codes before touching HIP (so each error path runs here)."""
import ctypes
import os
import re

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dsa_capi.h")


def _lib():
    from dsa_triton_ascend_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libdsa_hip.so not built")
    return L, L.load()


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "dsa_sfa_fwd" in names and "dsa_last_error" in names


def test_library_exports_every_declared_symbol():
    L, lib = _lib()
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in L.SIGNATURES, f"{name} missing from the ctypes binding"


def test_binding_covers_only_declared_symbols():
    L, _ = _lib()
    assert sorted(L.SIGNATURES) == _declared()


def test_abi_version():
    _, lib = _lib()
    assert lib.dsa_abi_version() >= 1


def _sfa_args(**kw):
    a = dict(query=1, query_rope=1, key=1, key_rope=1, sparse_indices=1, attention_out=1,
             softmax_max=1, softmax_sum=1, actual_seq_q=None, actual_seq_kv=None, block_table=None,
             batch=1, s1=4, s2=256, n1=8, d=128, d_rope=64, sparse_count=64, q_rows=4, kv_rows=256,
             max_blocks=0, page_size=0, sparse_block_size=1, sparse_mode=0,
             pre_tokens=9223372036854775807, next_tokens=9223372036854775807, layout_query=0,
             layout_kv=0, dtype=0, scale=0.1, return_lse=1, workspace=None, workspace_bytes=0,
             stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(d=96), 2), (dict(d_rope=32), 2), (dict(n1=0), 2), (dict(n1=129), 2),
    (dict(sparse_mode=1), 2), (dict(sparse_block_size=3), 2), (dict(sparse_block_size=256), 2),
    (dict(dtype=2), 2), (dict(layout_query=2), 2), (dict(layout_kv=7), 2),
    (dict(query=None), 1), (dict(return_lse=1, softmax_max=None), 1),
    (dict(q_rows=5), 1), (dict(kv_rows=255), 1), (dict(layout_query=1), 1),
    (dict(layout_kv=1), 1), (dict(layout_kv=2), 1),
    (dict(layout_kv=2, block_table=1, actual_seq_kv=1, page_size=64, max_blocks=4, kv_rows=100), 1),
    (dict(sparse_count=0), 1), (dict(batch=0), 1),
])
def test_sfa_fwd_rejects_bad_arguments(kw, code):
    _, lib = _lib()
    st = lib.dsa_sfa_fwd(*_sfa_args(**kw))
    assert st == code
    assert lib.dsa_last_error().decode()


def test_last_error_is_thread_local_and_reset():
    import threading
    _, lib = _lib()
    assert lib.dsa_sfa_fwd(*_sfa_args(d=96)) == 2
    seen = []
    t = threading.Thread(target=lambda: seen.append(lib.dsa_last_error()))
    t.start(); t.join()
    assert seen == [b""]
    assert b"D must be one of" in lib.dsa_last_error()


def test_workspace_size_query():
    _, lib = _lib()
    assert lib.dsa_sfa_fwd_workspace_size(0, 8, 128, 64, 1) == 0
    # without a GPU the CU count defaults to 256: 4 rows split 1 way -> no workspace
    assert lib.dsa_sfa_fwd_workspace_size(8192, 128, 512, 2048, 1) == 0
    assert lib.dsa_sfa_fwd_workspace_size(32, 128, 512, 2048, 1) > 0


def _kl_ex_args(**kw):
    a = dict(query=1, key=1, query_rope=1, key_rope=1, query_index=1, key_index=1, weights=1,
             sparse_indices=1, softmax_max=1, softmax_sum=1, actual_seq_qlen=None, actual_seq_klen=None,
             block_table=None, d_query_index=1, d_key_index=1, d_weights=1, loss=1, batch=1, s1=4,
             s2=64, n1=8, d=128, d_rope=64, n_idx=8, d_idx=128, sparse_count=16, q_rows=4, kv_rows=64,
             max_blocks=0, page_size=1, layout_query=0, layout_key=0, dtype=0, weights_dtype=2,
             scale=0.1, workspace=None, workspace_bytes=0, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(d=96), 2), (dict(n_idx=129), 2), (dict(d_idx=260), 2), (dict(d_idx=100), 2),
    (dict(sparse_count=(1 << 20) + 1), 2), (dict(layout_query=2), 2),
    (dict(layout_key=5), 2), (dict(weights_dtype=7), 2),
    (dict(query=None), 1), (dict(loss=None), 1), (dict(q_rows=5), 1), (dict(kv_rows=63), 1),
    (dict(layout_query=1), 1),                                 # TND query without cumulative lengths
    (dict(layout_key=1), 1),                                   # TND key with a BSND query
    (dict(layout_key=2, actual_seq_klen=1, page_size=16, max_blocks=4), 1),   # no block_table
    (dict(layout_key=2, block_table=1, page_size=16, max_blocks=4), 1),      # no key lengths
    (dict(layout_key=2, block_table=1, actual_seq_klen=1, page_size=16, max_blocks=4, kv_rows=60), 1),
    (dict(layout_key=2, block_table=1, actual_seq_klen=1, page_size=0, max_blocks=4), 1),
    (dict(), 4),                                               # valid, but no workspace
    (dict(layout_query=1, layout_key=1, actual_seq_qlen=1, actual_seq_klen=1, s1=0, s2=0), 4),
    (dict(layout_key=2, block_table=1, actual_seq_klen=1, page_size=16, max_blocks=4), 4),
])
def test_kl_bwd_ex_rejects_bad_arguments(kw, code):
    _, lib = _lib()
    st = lib.dsa_kl_bwd_ex(*_kl_ex_args(**kw))
    assert st == code
    assert lib.dsa_last_error().decode()


def test_kl_workspace_sizes_agree():
    _, lib = _lib()
    assert lib.dsa_kl_bwd_ex_workspace_size(2 * 7, 2 * 80, 48, 128) == lib.dsa_kl_bwd_workspace_size(2, 7, 80, 48, 128)
    assert lib.dsa_kl_bwd_ex_workspace_size(0, 80, 48, 128) == 0
    assert lib.dsa_kl_bwd_ex_workspace_size(7, 80, 48, 100) == 0      # d_idx not a multiple of 8
    assert lib.dsa_kl_bwd_ex_workspace_size(7, 80, 48, 264) == 0      # d_idx above 256
    # the contribution buffer and the accumulators scale with d_idx
    assert lib.dsa_kl_bwd_ex_workspace_size(7, 80, 48, 64) < lib.dsa_kl_bwd_ex_workspace_size(7, 80, 48, 128)


@pytest.mark.parametrize("args,code", [
    ((None, 1 << 20, 0, None, None), 1),      # no buffer
    ((0x10000, 8, 0, None, None), 1),         # under 16 bytes
    ((0x10000, 1000, 0, None, None), 1),      # not a multiple of 16
    ((0x10008, 1 << 20, 1, None, None), 1),   # misaligned
])
def test_calib_stream_read_rejects_bad_arguments(args, code):
    _, lib = _lib()
    assert lib.dsa_calib_stream_read(*args) == code
    assert lib.dsa_last_error().decode()
