"""ctypes binding of libdsa_hip.so (declared in include/dsa_capi.h).

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already carries (both use the soname libamdhip64.so.7);
streams and device pointers handed over from torch are then valid inside the
library.  There is no CPU fallback: a missing library raises at first use.
"""
import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("DSA_HIP_LIB", os.path.join(_PKG, "libdsa_hip.so"))

DSA_OK = 0
DSA_ERR_INVALID = 1
DSA_ERR_UNSUPPORTED = 2
DSA_ERR_HIP = 3
DSA_ERR_WORKSPACE = 4

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2

LAYOUT = {"BSND": 0, "TND": 1, "PA_BSND": 2}

TEST_FORCE_GLOBAL_GATHER = 1
TEST_SMALL_BWD_CHUNKS = 2
TEST_KL_GENERIC = 4
TEST_FWD_WIDE = 8
TEST_LI_UNFUSED = 16
TEST_LI_NO_PAIR = 32

_c = ctypes
_vp = _c.c_void_p
_i32p = _c.c_void_p
_i64 = _c.c_int64
_i32 = _c.c_int32
_f32 = _c.c_float
_sz = _c.c_size_t

# name -> (restype, argtypes); mirrors include/dsa_capi.h
SIGNATURES = {
    "dsa_last_error": (_c.c_char_p, []),
    "dsa_abi_version": (_c.c_int, []),
    "dsa_set_test_flags": (None, [_i32]),
    "dsa_calib_stream_read": (_c.c_int, [_vp, _sz, _i32, _vp, _vp]),
    "dsa_sfa_fwd": (_c.c_int, [
        _vp, _vp, _vp, _vp, _i32p,           # query, query_rope, key, key_rope, sparse_indices
        _vp, _vp, _vp,                        # attention_out, softmax_max, softmax_sum
        _i32p, _i32p, _i32p,                  # actual_seq_q, actual_seq_kv, block_table
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, d, d_rope
        _i64, _i64, _i64, _i64, _i64,         # sparse_count, q_rows, kv_rows, max_blocks, page_size
        _i32, _i32, _i64, _i64,               # sparse_block_size, sparse_mode, pre_tokens, next_tokens
        _i32, _i32, _i32,                     # layout_q, layout_kv, dtype
        _f32, _i32,                           # scale_value, return_lse
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_sfa_fwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "dsa_sfa_fwd_noalloc": (_c.c_int, [
        _vp, _vp, _vp, _vp, _i32p,           # query, query_rope, key, key_rope, sparse_indices
        _vp, _vp, _vp,                        # attention_out, softmax_max, softmax_sum
        _i32p, _i32p, _i32p,                  # actual_seq_q, actual_seq_kv, block_table
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, d, d_rope
        _i64, _i64, _i64, _i64, _i64,         # sparse_count, q_rows, kv_rows, max_blocks, page_size
        _i32, _i32, _i64, _i64,               # sparse_block_size, sparse_mode, pre_tokens, next_tokens
        _i32, _i32, _i32,                     # layout_q, layout_kv, dtype
        _f32, _i32,                           # scale_value, return_lse
        _vp,                                  # stream
    ]),
    "dsa_sfa_bwd": (_c.c_int, [
        _vp, _vp, _vp, _vp, _i32p,           # query, query_rope, key, key_rope, sparse_indices
        _vp, _vp, _vp, _vp,                   # d_out, out, softmax_max, softmax_sum
        _i32p, _i32p,                         # actual_seq_q, actual_seq_kv
        _vp, _vp, _vp, _vp, _vp,              # d_query, d_query_rope, d_key, d_key_rope, d_value
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, d, d_rope
        _i64, _i64, _i64,                     # sparse_count, q_rows, kv_rows
        _i32, _i32, _i64, _i64,               # sparse_block_size, sparse_mode, pre_tokens, next_tokens
        _i32, _i32,                           # layout, dtype
        _f32,                                 # scale_value
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_sfa_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i32, _i32]),
    "dsa_kl_bwd": (_c.c_int, [
        _vp, _vp, _vp, _vp,                   # query, key, query_rope, key_rope
        _vp, _vp, _vp, _i32p,                 # query_index, key_index, weights, sparse_indices
        _vp, _vp, _i32p, _i32p,               # softmax_max, softmax_sum, actual_seq_qlen, actual_seq_klen
        _vp, _vp, _vp, _vp,                   # d_query_index, d_key_index, d_weights, loss
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, d, d_rope
        _i64, _i64, _i64,                     # n_idx, d_idx, sparse_count
        _i32, _i32, _f32,                     # dtype, weights_dtype, scale_value
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_kl_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "dsa_kl_bwd_ex": (_c.c_int, [
        _vp, _vp, _vp, _vp,                   # query, key, query_rope, key_rope
        _vp, _vp, _vp, _i32p,                 # query_index, key_index, weights, sparse_indices
        _vp, _vp, _i32p, _i32p, _i32p,        # softmax_max, softmax_sum, actual_seq_qlen, actual_seq_klen, block_table
        _vp, _vp, _vp, _vp,                   # d_query_index, d_key_index, d_weights, loss
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, d, d_rope
        _i64, _i64, _i64,                     # n_idx, d_idx, sparse_count
        _i64, _i64, _i64, _i64,               # q_rows, kv_rows, max_blocks, page_size
        _i32, _i32, _i32, _i32, _f32,         # layout_query, layout_key, dtype, weights_dtype, scale_value
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_kl_bwd_ex_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "dsa_dense_li_softmax_lse": (_c.c_int, [
        _vp, _vp, _vp, _i32p, _i32p,          # query_index, key_index, weights, actual_seq_qlen, actual_seq_klen
        _vp, _vp,                             # softmax_max_index, softmax_sum_index
        _i64, _i64, _i64, _i64, _i64,         # batch, s1, s2, n_idx, d_idx
        _i32, _i32, _vp,                      # dtype, weights_dtype, stream
    ]),
    "dsa_dense_kl_bwd": (_c.c_int, [
        _vp, _vp, _vp, _vp,                   # query, key, query_rope, key_rope
        _vp, _vp, _vp,                        # query_index, key_index, weights
        _vp, _vp, _vp, _vp,                   # softmax_max, softmax_sum, softmax_max_index, softmax_sum_index
        _i32p, _i32p,                         # actual_seq_qlen, actual_seq_klen
        _vp, _vp, _vp, _vp,                   # d_query_index, d_key_index, d_weights, loss
        _i64, _i64, _i64, _i64, _i64,         # batch, s1, s2, n1, n2
        _i64, _i64, _i64, _i64,               # d, d_rope, n_idx, d_idx
        _i32, _i32, _f32,                     # dtype, weights_dtype, scale_value
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_dense_kl_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "dsa_li_fwd": (_c.c_int, [
        _vp, _vp, _vp, _i32p, _i32p,          # query, key, weights, actual_seq_q, actual_seq_k
        _i32p, _vp,                           # sparse_indices, sparse_values
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, n2, d
        _i64, _i64, _i64,                     # sparse_count, q_rows, k_rows
        _i32, _i32, _i32, _i32, _i32, _i32,   # sparse_mode, layout_q, layout_k, dtype, w_dtype, return_value
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_li_fwd_workspace_size": (_sz, [_i64, _i64, _i64]),
    "dsa_li_scores": (_c.c_int, [
        _vp, _vp, _vp, _i32p, _i32p, _vp,     # query, key, weights, actual_seq_q, actual_seq_k, scores
        _i64, _i64, _i64, _i64, _i64, _i64,   # batch, s1, s2, n1, n2, d
        _i64, _i64,                           # q_rows, k_rows
        _i32, _i32, _i32, _i32, _i32,         # sparse_mode, layout_q, layout_k, dtype, w_dtype
        _vp,                                  # stream
    ]),
    "dsa_li_topk_from_scores": (_c.c_int, [_vp, _i64, _i64, _i64, _i32p, _vp, _vp]),
    "dsa_li_fwd_paged": (_c.c_int, [
        _vp, _vp, _vp, _i32p, _i32p, _i32p,   # query, key_cache, weights, actual_seq_q, actual_seq_k, block_table
        _i32p, _vp,                           # sparse_indices, sparse_values
        _i64, _i64, _i64, _i64, _i64,         # batch, s1, n1, n2, d
        _i64, _i64, _i64, _i64, _i64,         # sparse_count, q_rows, num_blocks, page_size, max_blocks
        _i32, _i32, _i32, _i32, _i32,         # sparse_mode, layout_q, dtype, w_dtype, return_value
        _vp, _sz, _vp,                        # workspace, workspace_bytes, stream
    ]),
    "dsa_li_scores_paged": (_c.c_int, [
        _vp, _vp, _vp, _i32p, _i32p, _i32p,   # query, key_cache, weights, actual_seq_q, actual_seq_k, block_table
        _vp,                                  # scores
        _i64, _i64, _i64, _i64, _i64,         # batch, s1, n1, n2, d
        _i64, _i64, _i64, _i64,               # q_rows, num_blocks, page_size, max_blocks
        _i32, _i32, _i32, _i32,               # sparse_mode, layout_q, dtype, w_dtype
        _vp,                                  # stream
    ]),
}

_lib = None


def load():
    """Load (once) and return the ctypes library; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libdsa_hip.so not found at {LIB_PATH}; build it with "
            "`python -m dsa_triton_ascend_amd.build_lib` (no CPU fallback exists)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status, what):
    if status == DSA_OK:
        return
    msg = load().dsa_last_error().decode(errors="replace")
    if status in (DSA_ERR_INVALID, DSA_ERR_UNSUPPORTED, DSA_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device):
    """The current stream of ``device`` as a raw handle.  torch's raw-stream
    query takes about 0.2 us where building the Stream object takes about 2
    (a decode call makes one per call); the public form is the fallback."""
    if _raw_stream is not None:
        if isinstance(device, torch.device):
            idx = device.index
        else:
            idx = device if isinstance(device, int) else torch.device(device).index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt):
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float16:
        return DTYPE_FP16
    if dt == torch.float32:
        return DTYPE_FP32
    raise ValueError(f"unsupported dtype {dt}")
