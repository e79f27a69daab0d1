// C-ABI entry points of libdsa_hip.so: argument validation (HIP-free, so
// every error path can be exercised without a GPU), workspace sizing and
// dispatch to the gfx950 kernels.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace dsa {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
  set_error("HIP error in %s: %s", what, hipGetErrorString(e));
  return DSA_ERR_HIP;
}

// sfa_fwd.hip
struct SfaFwdParams;
int sfa_fwd_splits(int64_t rows, int64_t n1, int64_t d, int64_t total_pos);
size_t sfa_fwd_workspace_bytes(int64_t rows, int64_t n1, int64_t d, int64_t total_pos);
int sfa_fwd_run(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                int64_t d, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                int32_t sparse_mode, int32_t layout_query, int32_t layout_kv, int32_t dtype,
                float scale_value, int32_t return_lse, void* workspace, hipStream_t stream);

static bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

}  // namespace dsa

using namespace dsa;

extern "C" {

const char* dsa_last_error(void) { return g_err; }

int dsa_abi_version(void) { return 1; }

size_t dsa_sfa_fwd_workspace_size(int64_t q_rows, int64_t n1, int64_t d, int64_t sparse_count,
                                  int32_t sparse_block_size) {
  if (q_rows <= 0 || n1 <= 0 || d <= 0 || sparse_count <= 0 || sparse_block_size <= 0) return 0;
  return sfa_fwd_workspace_bytes(q_rows, n1, d, sparse_count * (int64_t)sparse_block_size);
}

int dsa_sfa_fwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                int64_t d, int64_t d_rope, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                int32_t sparse_mode, int32_t layout_query, int32_t layout_kv, int32_t dtype,
                float scale_value, int32_t return_lse, void* workspace, size_t workspace_bytes,
                void* stream) {
  g_err[0] = '\0';
  DSA_CHECK_ARG(query && query_rope && key && key_rope && sparse_indices && attention_out,
                "null tensor pointer");
  DSA_CHECK_ARG(!return_lse || (softmax_max && softmax_sum),
                "return_softmax_lse requires softmax_max and softmax_sum buffers");
  DSA_CHECK_SUPPORTED(d == 128 || d == 256 || d == 512, "D must be one of (128, 256, 512), got %lld",
                      (long long)d);
  DSA_CHECK_SUPPORTED(d_rope == 64, "rope dim must be 64, got %lld", (long long)d_rope);
  DSA_CHECK_SUPPORTED(n1 >= 1 && n1 <= 128, "N1 must be in [1, 128], got %lld", (long long)n1);
  DSA_CHECK_SUPPORTED(sparse_mode == 0 || sparse_mode == 3,
                      "Only sparse_mode 0 (full) / 3 (rightDownCausal) supported");
  DSA_CHECK_SUPPORTED(is_pow2(sparse_block_size) && sparse_block_size <= 128,
                      "sparse_block_size must be a power of 2 in [1,128]");
  DSA_CHECK_SUPPORTED(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_FP16,
                      "query/key dtype must be bfloat16 or float16");
  DSA_CHECK_SUPPORTED(layout_query == DSA_LAYOUT_BSND || layout_query == DSA_LAYOUT_TND,
                      "layout_query must be BSND or TND");
  DSA_CHECK_SUPPORTED(layout_kv == DSA_LAYOUT_BSND || layout_kv == DSA_LAYOUT_TND ||
                          layout_kv == DSA_LAYOUT_PA_BSND,
                      "layout_kv must be BSND, TND or PA_BSND");
  DSA_CHECK_ARG(batch >= 1 && batch <= (1 << 24), "batch must be >= 1, got %lld", (long long)batch);
  DSA_CHECK_ARG(sparse_count >= 1, "sparse_count must be >= 1");
  DSA_CHECK_ARG(sparse_count * (int64_t)sparse_block_size <= (1ll << 30),
                "sparse_count * sparse_block_size too large");
  if (layout_query == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(actual_seq_q, "TND query layout requires cumulative actual_seq_lengths_query");
    DSA_CHECK_ARG(q_rows >= 1, "TND query must have at least one row");
  } else {
    DSA_CHECK_ARG(s1 >= 1, "S1 must be >= 1");
    DSA_CHECK_ARG(q_rows == batch * s1, "q_rows must equal B*S1 for BSND query");
  }
  DSA_CHECK_ARG(q_rows < (1ll << 31), "too many query rows");
  if (layout_kv == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(actual_seq_kv, "TND key layout requires cumulative actual_seq_lengths_kv");
  } else if (layout_kv == DSA_LAYOUT_PA_BSND) {
    DSA_CHECK_ARG(block_table, "PA_BSND requires block_table");
    DSA_CHECK_ARG(actual_seq_kv, "PA_BSND requires actual_seq_lengths_kv");
    DSA_CHECK_ARG(page_size >= 1 && max_blocks >= 1, "PA_BSND requires block_size and block_table columns");
    DSA_CHECK_ARG(kv_rows % page_size == 0, "paged key rows must be a multiple of block_size");
  } else {
    DSA_CHECK_ARG(s2 >= 1 && kv_rows == batch * s2, "kv_rows must equal B*S2 for BSND key");
  }
  DSA_CHECK_ARG(kv_rows >= 1 && kv_rows < (1ll << 31), "key must have between 1 and 2^31-1 rows");
  const size_t need = sfa_fwd_workspace_bytes(q_rows, n1, d, sparse_count * (int64_t)sparse_block_size);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  return sfa_fwd_run(query, query_rope, key, key_rope, sparse_indices, attention_out, softmax_max,
                     softmax_sum, actual_seq_q, actual_seq_kv, block_table, batch, s1, s2, n1, d,
                     sparse_count, q_rows, kv_rows, max_blocks, page_size, sparse_block_size,
                     sparse_mode, layout_query, layout_kv, dtype, scale_value, return_lse,
                     workspace, (hipStream_t)stream);
}

}  // extern "C"
