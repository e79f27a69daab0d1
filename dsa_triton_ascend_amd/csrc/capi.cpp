// C-ABI entry points of libdsa_hip.so: argument validation (HIP-free, so
// every error path can be exercised without a GPU), workspace sizing and
// dispatch to the gfx950 kernels.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "common.h"

namespace dsa {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

static std::atomic<int> g_test_flags{0};
int test_flags() { return g_test_flags.load(std::memory_order_relaxed); }

int hip_fail(hipError_t e, const char* what) {
  set_error("HIP error in %s: %s", what, hipGetErrorString(e));
  return DSA_ERR_HIP;
}

int device_cu_count() {
  // per-device cache; concurrent first calls store the same value
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (!cus) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// sfa_fwd.hip
struct SfaFwdParams;
int sfa_fwd_splits(int64_t rows, int64_t n1, int64_t d, int64_t total_pos, bool one_list);
size_t sfa_fwd_workspace_bytes(int64_t rows, int64_t n1, int64_t d, int64_t total_pos, bool one_list);
size_t sfa_fwd_scratch_bytes();
int sfa_fwd_scratch(void** ptr);
int sfa_fwd_run(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                int64_t d, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                int32_t sparse_mode, int64_t pre_tokens, int64_t next_tokens, int32_t layout_query,
                int32_t layout_kv, int32_t dtype, float scale_value, int32_t return_lse, void* workspace,
                hipStream_t stream, bool one_list);

// sfa_bwd.hip
size_t sfa_bwd_workspace_bytes(int64_t q_rows, int64_t kv_rows, int64_t n1, int64_t d, int64_t total_pos,
                               bool merge);
// kl_bwd.hip
size_t kl_bwd_workspace_bytes(int64_t q_rows, int64_t kv_rows, int64_t topk, int64_t d_idx);
int kl_bwd_max_topk();
int kl_bwd_max_nidx();
int kl_bwd_max_didx();
// index head dims of the KL backward: 16-byte rows up to kl_bwd_max_didx()
static bool kl_didx_ok(int64_t d_idx) { return d_idx >= 8 && d_idx <= kl_bwd_max_didx() && d_idx % 8 == 0; }
int kl_bwd_run(const void* query, const void* key, const void* query_rope, const void* key_rope,
               const void* query_index, const void* key_index, const void* weights, const int32_t* sparse_indices,
               const float* softmax_max, const float* softmax_sum, const int32_t* act_q, const int32_t* act_k,
               const int32_t* block_table, void* d_query_index, void* d_key_index, void* d_weights, float* loss,
               int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t d_rope, int64_t nidx,
               int64_t d_idx, int64_t topk, int64_t q_rows, int64_t kv_rows, int64_t max_blocks, int64_t page_size,
               int32_t layout_q, int32_t layout_k, int32_t dtype, int32_t w_dtype, float scale_value,
               void* workspace, hipStream_t stream);
int sfa_bwd_run(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, const void* d_out, const void* out, const float* softmax_max,
                const float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                void* d_query, void* d_query_rope, void* d_key, void* d_key_rope, void* d_value,
                int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t sparse_count,
                int64_t q_rows, int64_t kv_rows, int32_t sparse_block_size, int32_t sparse_mode,
                int64_t pre_tokens, int64_t next_tokens, int32_t layout, int32_t dtype, float scale_value,
                void* workspace, hipStream_t stream);

// dense_kl.hip
size_t dense_kl_workspace_bytes(int64_t batch, int64_t s1, int64_t s2, int64_t di);
int dense_lse_run(const void* query_index, const void* key_index, const void* weights, const int32_t* act_q,
                  const int32_t* act_k, float* max_index, float* sum_index, int64_t batch, int64_t s1,
                  int64_t s2, int64_t nidx, int64_t di, int32_t dtype, int32_t w_dtype, hipStream_t stream);
int dense_kl_run(const void* query, const void* key, const void* query_rope, const void* key_rope,
                 const void* query_index, const void* key_index, const void* weights, const float* softmax_max,
                 const float* softmax_sum, const float* max_index, const float* sum_index, const int32_t* act_q,
                 const int32_t* act_k, void* d_query_index, void* d_key_index, void* d_weights, float* loss,
                 int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t n2, int64_t d, int64_t d_rope,
                 int64_t nidx, int64_t di, int32_t dtype, int32_t w_dtype, float scale_value, void* workspace,
                 hipStream_t stream);

// li_fwd.hip
int li_scores_run(const void* query, const void* key, const void* weights, const int32_t* act_q,
                  const int32_t* act_k, float* scores, int64_t batch, int64_t s1, int64_t s2,
                  int64_t n1, int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows,
                  int32_t sparse_mode, int32_t layout_q, int32_t layout_k, int32_t dtype,
                  int32_t w_dtype, hipStream_t stream, const int32_t* block_table = nullptr,
                  int64_t max_blocks = 0, int64_t page_size = 1);
int li_topk_run(const float* scores, int64_t rows, int64_t s2, int64_t k, int32_t* indices,
                void* values, int32_t val_dtype, hipStream_t stream, bool values_zero = false);
// scores and top-k: one fused launch where the shapes allow, else the two
int li_fwd_run(const void* query, const void* key, const void* weights, const int32_t* act_q,
               const int32_t* act_k, float* scores, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
               int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows, int32_t sparse_mode, int32_t layout_q,
               int32_t layout_k, int32_t dtype, int32_t w_dtype, int64_t k, int32_t* indices, void* values,
               hipStream_t stream, const int32_t* block_table = nullptr, int64_t max_blocks = 0,
               int64_t page_size = 1, bool values_zero = false);
constexpr int64_t kLiMaxK = 16384;  // the top-k sorts up to 16384 entries (LDS and per-wave registers)
// calib.hip
int calib_stream_read_run(const void* buf, size_t bytes, int nontemporal, unsigned* sink, hipStream_t stream);

static bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// Overflow-safe products for argument checks: false when either factor is
// negative or a * b does not fit in int64.
static bool mul_eq(int64_t a, int64_t b, int64_t want) {
  int64_t r;
  return a >= 0 && b >= 0 && !__builtin_mul_overflow(a, b, &r) && r == want;
}
static bool mul_lt(int64_t a, int64_t b, int64_t lim) {
  int64_t r;
  return a >= 0 && b >= 0 && !__builtin_mul_overflow(a, b, &r) && r < lim;
}
static bool mul_le(int64_t a, int64_t b, int64_t lim) {
  int64_t r;
  return a >= 0 && b >= 0 && !__builtin_mul_overflow(a, b, &r) && r <= lim;
}

// shared validation of the indexer score inputs
static int li_check_scores(const void* query, const void* key, const void* weights,
                           const int32_t* act_q, const int32_t* act_k, int64_t batch, int64_t s1,
                           int64_t s2, int64_t n1, int64_t n2, int64_t d, int64_t q_rows,
                           int64_t k_rows, int32_t sparse_mode, int32_t layout_q,
                           int32_t layout_k, int32_t dtype, int32_t w_dtype, bool allow_pa = false) {
  DSA_CHECK_ARG(query && key && weights, "null tensor pointer");
  DSA_CHECK_SUPPORTED(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_FP16 || dtype == DSA_DTYPE_FP32,
                      "query/key dtype must be bfloat16, float16 or float32");
  // 16-byte rows: a multiple of 8 elements (16-bit types) or of 4 (fp32)
  DSA_CHECK_SUPPORTED(d >= 1 && d <= 256 && d % (dtype == DSA_DTYPE_FP32 ? 4 : 8) == 0,
                      "head dim D must be a multiple of %d in [%d, 256], got %lld", dtype == DSA_DTYPE_FP32 ? 4 : 8,
                      dtype == DSA_DTYPE_FP32 ? 4 : 8, (long long)d);
  DSA_CHECK_ARG(n2 >= 1 && n1 >= 1, "N1 and N2 must be >= 1");
  DSA_CHECK_ARG(n1 % n2 == 0, "N1(%lld) must be divisible by N2(%lld)", (long long)n1, (long long)n2);
  DSA_CHECK_SUPPORTED(n1 / n2 <= 128, "N1/N2 (query heads per key head) must be <= 128, got %lld",
                      (long long)(n1 / n2));
  DSA_CHECK_SUPPORTED(sparse_mode == 0 || sparse_mode == 3,
                      "Only sparse_mode 0 (full) / 3 (rightDownCausal) supported");
  DSA_CHECK_SUPPORTED(w_dtype == DSA_DTYPE_BF16 || w_dtype == DSA_DTYPE_FP16 || w_dtype == DSA_DTYPE_FP32,
                      "weights dtype must be bfloat16, float16 or float32");
  DSA_CHECK_SUPPORTED(layout_q == DSA_LAYOUT_BSND || layout_q == DSA_LAYOUT_TND,
                      "layout_query must be BSND or TND");
  DSA_CHECK_SUPPORTED(layout_k == DSA_LAYOUT_BSND || layout_k == DSA_LAYOUT_TND ||
                          (allow_pa && layout_k == DSA_LAYOUT_PA_BSND),
                      "layout_key must be BSND or TND here (a paged key cache goes through the _paged entry points)");
  DSA_CHECK_ARG(!(layout_q == DSA_LAYOUT_BSND && layout_k == DSA_LAYOUT_TND),
                "a TND key needs a TND query");
  DSA_CHECK_ARG(batch >= 1 && batch <= (1 << 24), "batch must be >= 1");
  DSA_CHECK_ARG(s2 >= 1 && s2 <= 65535ll * 1024, "S2 must be in [1, 67107840]");
  if (layout_k == DSA_LAYOUT_PA_BSND)
    DSA_CHECK_ARG(act_k, "PA_BSND key requires actual_seq_lengths_key (per-batch lengths)");
  if (layout_q == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(act_q && act_k, "TND layout requires cumulative actual_seq_lengths_query and _key");
    DSA_CHECK_ARG(q_rows >= 1, "TND query must have at least one row");
  } else {
    DSA_CHECK_ARG(s1 >= 1 && mul_eq(batch, s1, q_rows), "q_rows must equal B*S1 for BSND query");
  }
  if (layout_k == DSA_LAYOUT_BSND) DSA_CHECK_ARG(mul_eq(batch, s2, k_rows), "k_rows must equal B*S2 for BSND key");
  DSA_CHECK_ARG(k_rows >= 1 && k_rows < (1ll << 31), "key must have between 1 and 2^31-1 rows");
  DSA_CHECK_ARG(mul_lt(q_rows, n2, 1ll << 31), "too many query rows");
  return DSA_OK;
}

}  // namespace dsa

namespace dsa {
// argument checks shared by dsa_sfa_fwd and dsa_sfa_fwd_noalloc (HIP-free)
static int sfa_fwd_check(const void* query, const void* query_rope, const void* key, const void* key_rope,
                         const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                         float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                         const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                         int64_t d, int64_t d_rope, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                         int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                         int32_t sparse_mode, int32_t layout_query, int32_t layout_kv, int32_t dtype,
                         int32_t return_lse) {
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
  DSA_CHECK_ARG(mul_le(sparse_count, sparse_block_size, 1ll << 30),
                "sparse_count * sparse_block_size too large");
  if (layout_query == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(actual_seq_q, "TND query layout requires cumulative actual_seq_lengths_query");
    DSA_CHECK_ARG(q_rows >= 1, "TND query must have at least one row");
  } else {
    DSA_CHECK_ARG(s1 >= 1, "S1 must be >= 1");
    DSA_CHECK_ARG(mul_eq(batch, s1, q_rows), "q_rows must equal B*S1 for BSND query");
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
    DSA_CHECK_ARG(s2 >= 1 && mul_eq(batch, s2, kv_rows), "kv_rows must equal B*S2 for BSND key");
  }
  DSA_CHECK_ARG(kv_rows >= 1 && kv_rows < (1ll << 31), "key must have between 1 and 2^31-1 rows");
  return DSA_OK;
}
}  // namespace dsa

using namespace dsa;

extern "C" {

const char* dsa_last_error(void) { return g_err; }

int dsa_abi_version(void) { return 3; }

void dsa_set_test_flags(int32_t flags) { g_test_flags.store(flags, std::memory_order_relaxed); }

size_t dsa_sfa_fwd_workspace_size(int64_t q_rows, int64_t n1, int64_t d, int64_t sparse_count,
                                  int32_t sparse_block_size) {
  // sizes the entry point rejects need no workspace
  if (q_rows <= 0 || q_rows >= (1ll << 31) || n1 <= 0 || n1 > 128 || d <= 0 || d > 512 || sparse_count <= 0 ||
      sparse_block_size <= 0 || !mul_le(sparse_count, sparse_block_size, 1ll << 30))
    return 0;
  return sfa_fwd_workspace_bytes(q_rows, n1, d, sparse_count * (int64_t)sparse_block_size, true);
}

int dsa_sfa_fwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                int64_t d, int64_t d_rope, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                int32_t sparse_mode, int64_t pre_tokens, int64_t next_tokens, int32_t layout_query,
                int32_t layout_kv, int32_t dtype, float scale_value, int32_t return_lse, void* workspace,
                size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  const int st = sfa_fwd_check(query, query_rope, key, key_rope, sparse_indices, attention_out, softmax_max, softmax_sum,
                                 actual_seq_q, actual_seq_kv, block_table, batch, s1, s2, n1, d, d_rope,
                                 sparse_count, q_rows, kv_rows, max_blocks, page_size, sparse_block_size,
                                 sparse_mode, layout_query, layout_kv, dtype, return_lse);
  if (st != DSA_OK) return st;
  const size_t need = sfa_fwd_workspace_bytes(q_rows, n1, d, sparse_count * (int64_t)sparse_block_size, true);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  return sfa_fwd_run(query, query_rope, key, key_rope, sparse_indices, attention_out, softmax_max,
                     softmax_sum, actual_seq_q, actual_seq_kv, block_table, batch, s1, s2, n1, d,
                     sparse_count, q_rows, kv_rows, max_blocks, page_size, sparse_block_size,
                     sparse_mode, pre_tokens, next_tokens, layout_query, layout_kv, dtype, scale_value, return_lse,
                     workspace, (hipStream_t)stream, true);
}

int dsa_sfa_fwd_noalloc(const void* query, const void* query_rope, const void* key, const void* key_rope,
                        const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                        float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                        const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                        int64_t d, int64_t d_rope, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                        int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                        int32_t sparse_mode, int64_t pre_tokens, int64_t next_tokens, int32_t layout_query,
                        int32_t layout_kv, int32_t dtype, float scale_value, int32_t return_lse,
                        void* stream) {
  g_err[0] = '\0';
  const int st = sfa_fwd_check(query, query_rope, key, key_rope, sparse_indices, attention_out, softmax_max, softmax_sum,
                                 actual_seq_q, actual_seq_kv, block_table, batch, s1, s2, n1, d, d_rope,
                                 sparse_count, q_rows, kv_rows, max_blocks, page_size, sparse_block_size,
                                 sparse_mode, layout_query, layout_kv, dtype, return_lse);
  if (st != DSA_OK) return st;
  // the one-list splits when their partials fit the scratch, else the
  // splits that fill the CUs (long ranges then run chunked)
  const int64_t total_pos = sparse_count * (int64_t)sparse_block_size;
  const bool one_list = sfa_fwd_workspace_bytes(q_rows, n1, d, total_pos, true) <= sfa_fwd_scratch_bytes();
  const size_t need = sfa_fwd_workspace_bytes(q_rows, n1, d, total_pos, one_list);
  void* ws = nullptr;
  if (need > 0) {
    DSA_CHECK_SUPPORTED(need <= sfa_fwd_scratch_bytes(),
                        "these sizes need %zu bytes of split workspace, above the %zu-byte scratch of "
                        "dsa_sfa_fwd_noalloc; call dsa_sfa_fwd with a workspace",
                        need, sfa_fwd_scratch_bytes());
    const int sst = sfa_fwd_scratch(&ws);
    if (sst != DSA_OK) return sst;
  }
  return sfa_fwd_run(query, query_rope, key, key_rope, sparse_indices, attention_out, softmax_max,
                     softmax_sum, actual_seq_q, actual_seq_kv, block_table, batch, s1, s2, n1, d,
                     sparse_count, q_rows, kv_rows, max_blocks, page_size, sparse_block_size,
                     sparse_mode, pre_tokens, next_tokens, layout_query, layout_kv, dtype, scale_value, return_lse, ws,
                     (hipStream_t)stream, one_list);
}

size_t dsa_sfa_bwd_workspace_size(int64_t q_rows, int64_t kv_rows, int64_t n1, int64_t d, int64_t sparse_count,
                                  int32_t sparse_block_size, int32_t merge_kv) {
  if (q_rows < 0 || q_rows >= (1ll << 31) || kv_rows <= 0 || kv_rows >= (1ll << 31) || n1 <= 0 || n1 > 128 ||
      d <= 0 || d > 512 || sparse_count <= 0 || sparse_block_size <= 0 ||
      !mul_le(sparse_count, sparse_block_size, 1ll << 30))
    return 0;
  return sfa_bwd_workspace_bytes(q_rows, kv_rows, n1, d, sparse_count * (int64_t)sparse_block_size, merge_kv != 0);
}

int dsa_sfa_bwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, const void* d_out, const void* out, const float* softmax_max,
                const float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                void* d_query, void* d_query_rope, void* d_key, void* d_key_rope, void* d_value,
                int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t d_rope,
                int64_t sparse_count, int64_t q_rows, int64_t kv_rows, int32_t sparse_block_size,
                int32_t sparse_mode, int64_t pre_tokens, int64_t next_tokens, int32_t layout, int32_t dtype,
                float scale_value, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  DSA_CHECK_ARG(query && query_rope && key && key_rope && sparse_indices && d_out && out && softmax_max &&
                    softmax_sum,
                "null input tensor pointer");
  DSA_CHECK_ARG(d_query && d_query_rope && d_key && d_key_rope, "null output tensor pointer");
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
  DSA_CHECK_SUPPORTED(layout == DSA_LAYOUT_BSND || layout == DSA_LAYOUT_TND, "layout must be BSND or TND");
  DSA_CHECK_ARG(batch >= 1 && batch <= (1 << 24), "batch must be >= 1");
  DSA_CHECK_ARG(sparse_count >= 1 && mul_le(sparse_count, sparse_block_size, 1ll << 30),
                "sparse_count out of range");
  if (layout == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(actual_seq_q && actual_seq_kv, "TND layout requires cumulative actual sequence lengths");
    DSA_CHECK_ARG(q_rows >= 1, "TND query must have at least one row");
  } else {
    DSA_CHECK_ARG(s1 >= 1 && mul_eq(batch, s1, q_rows), "q_rows must equal B*S1 for BSND");
    DSA_CHECK_ARG(s2 >= 1 && mul_eq(batch, s2, kv_rows), "kv_rows must equal B*S2 for BSND");
  }
  DSA_CHECK_ARG(q_rows < (1ll << 31) && kv_rows >= 1 && kv_rows < (1ll << 31), "row counts out of range");
  const size_t need = sfa_bwd_workspace_bytes(q_rows, kv_rows, n1, d, sparse_count * (int64_t)sparse_block_size,
                                             d_value == nullptr);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  return sfa_bwd_run(query, query_rope, key, key_rope, sparse_indices, d_out, out, softmax_max, softmax_sum,
                     actual_seq_q, actual_seq_kv, d_query, d_query_rope, d_key, d_key_rope, d_value, batch, s1,
                     s2, n1, d, sparse_count, q_rows, kv_rows, sparse_block_size, sparse_mode, pre_tokens, next_tokens, layout, dtype,
                     scale_value, workspace, (hipStream_t)stream);
}

size_t dsa_kl_bwd_workspace_size(int64_t batch, int64_t s1, int64_t s2, int64_t sparse_count, int64_t d_idx) {
  if (batch <= 0 || !mul_lt(batch, s1, 1ll << 31) || !mul_lt(batch, s2, 1ll << 31) || s1 <= 0 || s2 <= 0 ||
      sparse_count <= 0 || sparse_count > kl_bwd_max_topk() || !kl_didx_ok(d_idx))
    return 0;
  return kl_bwd_workspace_bytes(batch * s1, batch * s2, sparse_count, d_idx);
}

size_t dsa_kl_bwd_ex_workspace_size(int64_t q_rows, int64_t kv_rows, int64_t sparse_count, int64_t d_idx) {
  if (q_rows <= 0 || q_rows >= (1ll << 31) || kv_rows <= 0 || kv_rows >= (1ll << 31) || sparse_count <= 0 ||
      sparse_count > kl_bwd_max_topk() || !kl_didx_ok(d_idx))
    return 0;
  return kl_bwd_workspace_bytes(q_rows, kv_rows, sparse_count, d_idx);
}

// Validation shared by dsa_kl_bwd and dsa_kl_bwd_ex.  For a TND side s1 / s2
// are not used; for a paged key s2 = max_blocks * page_size.
static int kl_check(const void* query, const void* key, const void* query_rope, const void* key_rope,
                    const void* query_index, const void* key_index, const void* weights,
                    const int32_t* sparse_indices, const float* softmax_max, const float* softmax_sum,
                    const int32_t* act_q, const int32_t* act_k, const int32_t* block_table,
                    const void* d_query_index, const void* d_key_index, const void* d_weights, const float* loss,
                    int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t d_rope, int64_t n_idx,
                    int64_t d_idx, int64_t sparse_count, int64_t q_rows, int64_t kv_rows, int64_t max_blocks,
                    int64_t page_size, int32_t layout_q, int32_t layout_k, int32_t dtype, int32_t weights_dtype,
                    const void* workspace, size_t workspace_bytes) {
  DSA_CHECK_ARG(query && key && query_index && key_index && weights && sparse_indices && softmax_max &&
                    softmax_sum,
                "null input tensor pointer");
  DSA_CHECK_ARG(d_query_index && d_key_index && d_weights && loss, "null output tensor pointer");
  DSA_CHECK_SUPPORTED(d == 128 || d == 256 || d == 512, "D must be one of (128, 256, 512), got %lld",
                      (long long)d);
  DSA_CHECK_SUPPORTED(d_rope == 0 || d_rope == 64, "rope dim must be 64 (or 0 for no rope), got %lld",
                      (long long)d_rope);
  DSA_CHECK_ARG(d_rope == 0 || (query_rope && key_rope), "null rope tensor pointer");
  DSA_CHECK_SUPPORTED(kl_didx_ok(d_idx), "index head dim must be a multiple of 8 in [8, %d], got %lld",
                      kl_bwd_max_didx(), (long long)d_idx);
  DSA_CHECK_SUPPORTED(n_idx >= 1 && n_idx <= kl_bwd_max_nidx(), "Nidx1 must be in [1, %d], got %lld",
                      kl_bwd_max_nidx(), (long long)n_idx);
  DSA_CHECK_SUPPORTED(n1 >= 1 && n1 <= 128, "N1 must be in [1, 128], got %lld", (long long)n1);
  DSA_CHECK_SUPPORTED(sparse_count >= 1 && sparse_count <= kl_bwd_max_topk(), "topK must be in [1, %d], got %lld",
                      kl_bwd_max_topk(), (long long)sparse_count);
  DSA_CHECK_SUPPORTED(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_FP16,
                      "query/key/index dtype must be bfloat16 or float16");
  DSA_CHECK_SUPPORTED(weights_dtype == DSA_DTYPE_FP32 || weights_dtype == DSA_DTYPE_BF16 ||
                          weights_dtype == DSA_DTYPE_FP16,
                      "weights dtype must be float32, bfloat16 or float16");
  DSA_CHECK_SUPPORTED(layout_q == DSA_LAYOUT_BSND || layout_q == DSA_LAYOUT_TND, "layout_query must be BSND or TND");
  DSA_CHECK_SUPPORTED(layout_k == DSA_LAYOUT_BSND || layout_k == DSA_LAYOUT_TND || layout_k == DSA_LAYOUT_PA_BSND,
                      "layout_key must be BSND, TND or PA_BSND");
  DSA_CHECK_ARG(!(layout_q == DSA_LAYOUT_BSND && layout_k == DSA_LAYOUT_TND), "a TND key needs a TND query");
  DSA_CHECK_ARG(batch >= 1 && batch <= (1 << 24), "batch must be in [1, 2^24]");
  DSA_CHECK_ARG(q_rows >= 1 && kv_rows >= 1, "the query and the key need at least one row");
  DSA_CHECK_ARG(mul_lt(q_rows, sparse_count, 1ll << 31) && kv_rows < (1ll << 31),
                "rows x topK and the key rows must stay below 2^31");
  if (layout_q == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(act_q, "TND query requires cumulative actual_seq_qlen");
  } else {
    DSA_CHECK_ARG(s1 >= 1 && mul_eq(batch, s1, q_rows), "q_rows must equal B*S1 for a BSND query");
  }
  if (layout_k == DSA_LAYOUT_TND) {
    DSA_CHECK_ARG(act_k, "TND key requires cumulative actual_seq_klen");
  } else if (layout_k == DSA_LAYOUT_PA_BSND) {
    DSA_CHECK_ARG(block_table, "PA_BSND key requires a block_table");
    DSA_CHECK_ARG(act_k, "PA_BSND key requires actual_seq_klen (per-batch lengths)");
    DSA_CHECK_ARG(page_size >= 1 && page_size <= (1 << 20), "page (block) size must be in [1, 2^20]");
    DSA_CHECK_ARG(max_blocks >= 1 && mul_lt(max_blocks, page_size, 1ll << 31),
                  "max_blocks * page size must be in [1, 2^31)");
    DSA_CHECK_ARG(kv_rows % page_size == 0, "the paged key rows must be a whole number of pages");
  } else {
    DSA_CHECK_ARG(s2 >= 1 && mul_eq(batch, s2, kv_rows), "kv_rows must equal B*S2 for a BSND key");
  }
  const size_t need = kl_bwd_workspace_bytes(q_rows, kv_rows, sparse_count, d_idx);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  return DSA_OK;
}

int dsa_kl_bwd(const void* query, const void* key, const void* query_rope, const void* key_rope,
               const void* query_index, const void* key_index, const void* weights,
               const int32_t* sparse_indices, const float* softmax_max, const float* softmax_sum,
               const int32_t* actual_seq_qlen, const int32_t* actual_seq_klen, void* d_query_index,
               void* d_key_index, void* d_weights, float* loss, int64_t batch, int64_t s1, int64_t s2,
               int64_t n1, int64_t d, int64_t d_rope, int64_t n_idx, int64_t d_idx, int64_t sparse_count,
               int32_t dtype, int32_t weights_dtype, float scale_value, void* workspace,
               size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  DSA_CHECK_ARG(batch >= 1 && batch <= (1 << 24) && s1 >= 1 && s1 < (1ll << 31) && s2 >= 1 && s2 < (1ll << 31),
                "batch must be in [1, 2^24], S1 and S2 in [1, 2^31)");
  const int st = kl_check(query, key, query_rope, key_rope, query_index, key_index, weights, sparse_indices,
                          softmax_max, softmax_sum, actual_seq_qlen, actual_seq_klen, nullptr, d_query_index,
                          d_key_index, d_weights, loss, batch, s1, s2, n1, d, d_rope, n_idx, d_idx, sparse_count,
                          batch * s1, batch * s2, 0, 1, DSA_LAYOUT_BSND, DSA_LAYOUT_BSND, dtype, weights_dtype,
                          workspace, workspace_bytes);
  if (st != DSA_OK) return st;
  return kl_bwd_run(query, key, d_rope ? query_rope : nullptr, d_rope ? key_rope : nullptr, query_index,
                    key_index, weights, sparse_indices, softmax_max, softmax_sum, actual_seq_qlen,
                    actual_seq_klen, nullptr, d_query_index, d_key_index, d_weights, loss, batch, s1, s2, n1, d,
                    d_rope, n_idx, d_idx, sparse_count, batch * s1, batch * s2, 0, 1, DSA_LAYOUT_BSND,
                    DSA_LAYOUT_BSND, dtype, weights_dtype, scale_value, workspace, (hipStream_t)stream);
}

int dsa_kl_bwd_ex(const void* query, const void* key, const void* query_rope, const void* key_rope,
                  const void* query_index, const void* key_index, const void* weights,
                  const int32_t* sparse_indices, const float* softmax_max, const float* softmax_sum,
                  const int32_t* actual_seq_qlen, const int32_t* actual_seq_klen, const int32_t* block_table,
                  void* d_query_index, void* d_key_index, void* d_weights, float* loss, int64_t batch,
                  int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t d_rope, int64_t n_idx, int64_t d_idx,
                  int64_t sparse_count, int64_t q_rows, int64_t kv_rows, int64_t max_blocks, int64_t page_size,
                  int32_t layout_query, int32_t layout_key, int32_t dtype, int32_t weights_dtype,
                  float scale_value, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  if (layout_key == DSA_LAYOUT_PA_BSND) {
    DSA_CHECK_ARG(max_blocks >= 1 && page_size >= 1 && mul_lt(max_blocks, page_size, 1ll << 31),
                  "max_blocks * page size must be in [1, 2^31)");
    s2 = max_blocks * page_size;
  }
  const int st = kl_check(query, key, query_rope, key_rope, query_index, key_index, weights, sparse_indices,
                          softmax_max, softmax_sum, actual_seq_qlen, actual_seq_klen, block_table, d_query_index,
                          d_key_index, d_weights, loss, batch, s1, s2, n1, d, d_rope, n_idx, d_idx, sparse_count,
                          q_rows, kv_rows, max_blocks, page_size, layout_query, layout_key, dtype, weights_dtype,
                          workspace, workspace_bytes);
  if (st != DSA_OK) return st;
  return kl_bwd_run(query, key, d_rope ? query_rope : nullptr, d_rope ? key_rope : nullptr, query_index,
                    key_index, weights, sparse_indices, softmax_max, softmax_sum, actual_seq_qlen,
                    actual_seq_klen, layout_key == DSA_LAYOUT_PA_BSND ? block_table : nullptr, d_query_index,
                    d_key_index, d_weights, loss, batch, s1, s2, n1, d, d_rope, n_idx, d_idx, sparse_count, q_rows,
                    kv_rows, max_blocks, page_size, layout_query, layout_key, dtype, weights_dtype, scale_value,
                    workspace, (hipStream_t)stream);
}

// shared validation of the dense index inputs (the reference's
// _validate_dense_index_inputs / dtype checks, dense_loss_backward_triton.py:658-697)
static int dense_check_index(const void* query_index, const void* key_index, const void* weights, int64_t batch,
                             int64_t s1, int64_t s2, int64_t n_idx, int64_t d_idx, int32_t dtype,
                             int32_t weights_dtype) {
  DSA_CHECK_ARG(query_index && key_index && weights, "null index tensor pointer");
  DSA_CHECK_SUPPORTED(d_idx == 128 || d_idx == 256 || d_idx == 512, "D_idx must be one of (128, 256, 512), got %lld",
                      (long long)d_idx);
  DSA_CHECK_SUPPORTED(n_idx >= 1 && n_idx <= 128, "Nidx1 must be in [1, 128], got %lld", (long long)n_idx);
  DSA_CHECK_SUPPORTED(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_FP16, "index dtype must be bfloat16 or float16");
  DSA_CHECK_SUPPORTED(weights_dtype == DSA_DTYPE_FP32 || weights_dtype == DSA_DTYPE_BF16 ||
                          weights_dtype == DSA_DTYPE_FP16,
                      "weights dtype must be float32, bfloat16 or float16");
  DSA_CHECK_ARG(batch >= 1 && batch <= (1 << 24) && s1 >= 1 && s1 < (1ll << 31) && s2 >= 1 && s2 < (1ll << 31),
                "batch must be in [1, 2^24], S1 and S2 in [1, 2^31)");
  DSA_CHECK_ARG(mul_lt(batch, s1, 1ll << 31) && mul_lt(batch, s2, 1ll << 31) && s2 < (1ll << 30),
                "B*S1, B*S2 and S2 must stay below 2^31");
  return DSA_OK;
}

int dsa_dense_li_softmax_lse(const void* query_index, const void* key_index, const void* weights,
                             const int32_t* actual_seq_qlen, const int32_t* actual_seq_klen,
                             float* softmax_max_index, float* softmax_sum_index, int64_t batch, int64_t s1,
                             int64_t s2, int64_t n_idx, int64_t d_idx, int32_t dtype, int32_t weights_dtype,
                             void* stream) {
  g_err[0] = '\0';
  const int st = dense_check_index(query_index, key_index, weights, batch, s1, s2, n_idx, d_idx, dtype,
                                   weights_dtype);
  if (st != DSA_OK) return st;
  DSA_CHECK_ARG(softmax_max_index && softmax_sum_index, "null output tensor pointer");
  return dense_lse_run(query_index, key_index, weights, actual_seq_qlen, actual_seq_klen, softmax_max_index,
                       softmax_sum_index, batch, s1, s2, n_idx, d_idx, dtype, weights_dtype, (hipStream_t)stream);
}

size_t dsa_dense_kl_bwd_workspace_size(int64_t batch, int64_t s1, int64_t s2, int64_t d_idx) {
  if (batch <= 0 || s1 <= 0 || s2 <= 0 || !mul_lt(batch, s1, 1ll << 31) || !mul_lt(batch, s2, 1ll << 31) ||
      !(d_idx == 128 || d_idx == 256 || d_idx == 512))
    return 0;
  return dense_kl_workspace_bytes(batch, s1, s2, d_idx);
}

int dsa_dense_kl_bwd(const void* query, const void* key, const void* query_rope, const void* key_rope,
                     const void* query_index, const void* key_index, const void* weights,
                     const float* softmax_max, const float* softmax_sum, const float* softmax_max_index,
                     const float* softmax_sum_index, const int32_t* actual_seq_qlen,
                     const int32_t* actual_seq_klen, void* d_query_index, void* d_key_index, void* d_weights,
                     float* loss, int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t n2, int64_t d,
                     int64_t d_rope, int64_t n_idx, int64_t d_idx, int32_t dtype, int32_t weights_dtype,
                     float scale_value, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  int st = dense_check_index(query_index, key_index, weights, batch, s1, s2, n_idx, d_idx, dtype, weights_dtype);
  if (st != DSA_OK) return st;
  DSA_CHECK_ARG(query && key && softmax_max && softmax_sum, "null input tensor pointer");
  DSA_CHECK_ARG(d_query_index && d_key_index && d_weights && loss, "null output tensor pointer");
  DSA_CHECK_ARG((softmax_max_index == nullptr) == (softmax_sum_index == nullptr),
                "softmax_max_index and softmax_sum_index must be both provided or both omitted");
  DSA_CHECK_SUPPORTED(d == 128 || d == 256 || d == 512, "D must be one of (128, 256, 512), got %lld", (long long)d);
  DSA_CHECK_SUPPORTED(d_rope == 0 || d_rope == 64, "rope dim must be 64 (or 0 for no rope), got %lld",
                      (long long)d_rope);
  DSA_CHECK_ARG(d_rope == 0 || (query_rope && key_rope), "null rope tensor pointer");
  DSA_CHECK_ARG(n2 >= 1 && n1 >= 1 && n1 % n2 == 0, "query N1 must be divisible by key N2");
  DSA_CHECK_SUPPORTED(n1 <= 128, "N1 must be <= 128, got %lld", (long long)n1);
  const size_t need = dense_kl_workspace_bytes(batch, s1, s2, d_idx);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  return dense_kl_run(query, key, d_rope ? query_rope : nullptr, d_rope ? key_rope : nullptr, query_index,
                      key_index, weights, softmax_max, softmax_sum, softmax_max_index, softmax_sum_index,
                      actual_seq_qlen, actual_seq_klen, d_query_index, d_key_index, d_weights, loss, batch, s1, s2,
                      n1, n2, d, d_rope, n_idx, d_idx, dtype, weights_dtype, scale_value, workspace,
                      (hipStream_t)stream);
}

size_t dsa_li_fwd_workspace_size(int64_t q_rows, int64_t n2, int64_t s2) {
  if (q_rows <= 0 || q_rows >= (1ll << 31) || n2 <= 0 || n2 > (1 << 16) || s2 <= 0 || s2 > 65535ll * 1024)
    return 0;
  return (size_t)q_rows * n2 * s2 * sizeof(float);
}

int dsa_li_scores(const void* query, const void* key, const void* weights, const int32_t* actual_seq_q,
                  const int32_t* actual_seq_k, float* scores, int64_t batch, int64_t s1, int64_t s2,
                  int64_t n1, int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows,
                  int32_t sparse_mode, int32_t layout_query, int32_t layout_key, int32_t dtype,
                  int32_t weights_dtype, void* stream) {
  g_err[0] = '\0';
  int st = li_check_scores(query, key, weights, actual_seq_q, actual_seq_k, batch, s1, s2, n1, n2, d,
                           q_rows, k_rows, sparse_mode, layout_query, layout_key, dtype, weights_dtype);
  if (st != DSA_OK) return st;
  DSA_CHECK_ARG(scores, "null scores pointer");
  return li_scores_run(query, key, weights, actual_seq_q, actual_seq_k, scores, batch, s1, s2, n1, n2,
                       d, q_rows, k_rows, sparse_mode, layout_query, layout_key, dtype, weights_dtype,
                       (hipStream_t)stream);
}

int dsa_li_topk_from_scores(const float* scores, int64_t rows, int64_t s2, int64_t sparse_count,
                            int32_t* indices, float* values, void* stream) {
  g_err[0] = '\0';
  DSA_CHECK_ARG(scores && indices, "null tensor pointer");
  DSA_CHECK_ARG(rows >= 0 && rows < (1ll << 31), "rows out of range");
  DSA_CHECK_ARG(s2 >= 1 && s2 < (1ll << 31), "S2 must be >= 1");
  DSA_CHECK_SUPPORTED(sparse_count >= 1 && sparse_count <= kLiMaxK,
                      "sparse_count must be in [1, %lld], got %lld", (long long)kLiMaxK,
                      (long long)sparse_count);
  return li_topk_run(scores, rows, s2, sparse_count, indices, values, DSA_DTYPE_FP32, (hipStream_t)stream);
}

int dsa_li_fwd(const void* query, const void* key, const void* weights, const int32_t* actual_seq_q,
               const int32_t* actual_seq_k, int32_t* sparse_indices, void* sparse_values,
               int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t n2, int64_t d,
               int64_t sparse_count, int64_t q_rows, int64_t k_rows, int32_t sparse_mode,
               int32_t layout_query, int32_t layout_key, int32_t dtype, int32_t weights_dtype,
               int32_t return_value, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  int st = li_check_scores(query, key, weights, actual_seq_q, actual_seq_k, batch, s1, s2, n1, n2, d,
                           q_rows, k_rows, sparse_mode, layout_query, layout_key, dtype, weights_dtype);
  if (st != DSA_OK) return st;
  DSA_CHECK_ARG(sparse_indices, "null sparse_indices pointer");
  DSA_CHECK_ARG(!return_value || sparse_values, "return_value requires a sparse_values buffer");
  DSA_CHECK_SUPPORTED(sparse_count >= 1 && sparse_count <= kLiMaxK,
                      "sparse_count must be in [1, %lld], got %lld", (long long)kLiMaxK,
                      (long long)sparse_count);
  const size_t need = dsa_li_fwd_workspace_size(q_rows, n2, s2);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  float* scores = (float*)workspace;
  return li_fwd_run(query, key, weights, actual_seq_q, actual_seq_k, scores, batch, s1, s2, n1, n2, d, q_rows,
                    k_rows, sparse_mode, layout_query, layout_key, dtype, weights_dtype, sparse_count,
                    sparse_indices, sparse_values, (hipStream_t)stream, nullptr, 0, 1,
                    !return_value && sparse_values);
}

static int li_check_paged(const int32_t* block_table, int64_t num_blocks, int64_t page_size,
                          int64_t max_blocks) {
  DSA_CHECK_ARG(block_table, "PA_BSND key requires a block_table");
  DSA_CHECK_ARG(page_size >= 1 && page_size <= (1 << 20), "page (block) size must be in [1, 2^20]");
  DSA_CHECK_ARG(num_blocks >= 1 && max_blocks >= 1, "the cache and the block table need at least one block");
  DSA_CHECK_ARG(mul_le(max_blocks, page_size, 65535ll * 1024), "max_blocks * page size must be <= 67107840");
  DSA_CHECK_ARG(mul_lt(num_blocks, page_size, 1ll << 31), "the key cache must have fewer than 2^31 rows");
  return DSA_OK;
}

int dsa_li_scores_paged(const void* query, const void* key_cache, const void* weights,
                        const int32_t* actual_seq_q, const int32_t* actual_seq_k, const int32_t* block_table,
                        float* scores, int64_t batch, int64_t s1, int64_t n1, int64_t n2, int64_t d,
                        int64_t q_rows, int64_t num_blocks, int64_t page_size, int64_t max_blocks,
                        int32_t sparse_mode, int32_t layout_query, int32_t dtype, int32_t weights_dtype,
                        void* stream) {
  g_err[0] = '\0';
  int st = li_check_paged(block_table, num_blocks, page_size, max_blocks);
  if (st != DSA_OK) return st;
  const int64_t s2 = max_blocks * page_size, k_rows = num_blocks * page_size;
  st = li_check_scores(query, key_cache, weights, actual_seq_q, actual_seq_k, batch, s1, s2, n1, n2, d, q_rows,
                       k_rows, sparse_mode, layout_query, DSA_LAYOUT_PA_BSND, dtype, weights_dtype, true);
  if (st != DSA_OK) return st;
  DSA_CHECK_ARG(scores, "null scores pointer");
  return li_scores_run(query, key_cache, weights, actual_seq_q, actual_seq_k, scores, batch, s1, s2, n1, n2, d,
                       q_rows, k_rows, sparse_mode, layout_query, DSA_LAYOUT_PA_BSND, dtype, weights_dtype,
                       (hipStream_t)stream, block_table, max_blocks, page_size);
}

int dsa_li_fwd_paged(const void* query, const void* key_cache, const void* weights, const int32_t* actual_seq_q,
                     const int32_t* actual_seq_k, const int32_t* block_table, int32_t* sparse_indices,
                     void* sparse_values, int64_t batch, int64_t s1, int64_t n1, int64_t n2, int64_t d,
                     int64_t sparse_count, int64_t q_rows, int64_t num_blocks, int64_t page_size,
                     int64_t max_blocks, int32_t sparse_mode, int32_t layout_query, int32_t dtype,
                     int32_t weights_dtype, int32_t return_value, void* workspace, size_t workspace_bytes,
                     void* stream) {
  g_err[0] = '\0';
  int st = li_check_paged(block_table, num_blocks, page_size, max_blocks);
  if (st != DSA_OK) return st;
  const int64_t s2 = max_blocks * page_size, k_rows = num_blocks * page_size;
  st = li_check_scores(query, key_cache, weights, actual_seq_q, actual_seq_k, batch, s1, s2, n1, n2, d, q_rows,
                       k_rows, sparse_mode, layout_query, DSA_LAYOUT_PA_BSND, dtype, weights_dtype, true);
  if (st != DSA_OK) return st;
  DSA_CHECK_ARG(sparse_indices, "null sparse_indices pointer");
  DSA_CHECK_ARG(!return_value || sparse_values, "return_value requires a sparse_values buffer");
  DSA_CHECK_SUPPORTED(sparse_count >= 1 && sparse_count <= kLiMaxK,
                      "sparse_count must be in [1, %lld], got %lld", (long long)kLiMaxK,
                      (long long)sparse_count);
  const size_t need = dsa_li_fwd_workspace_size(q_rows, n2, s2);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace of %zu bytes required, %zu given", need, workspace_bytes);
    return DSA_ERR_WORKSPACE;
  }
  float* scores = (float*)workspace;
  return li_fwd_run(query, key_cache, weights, actual_seq_q, actual_seq_k, scores, batch, s1, s2, n1, n2, d,
                    q_rows, k_rows, sparse_mode, layout_query, DSA_LAYOUT_PA_BSND, dtype, weights_dtype,
                    sparse_count, sparse_indices, sparse_values, (hipStream_t)stream, block_table, max_blocks,
                    page_size, !return_value && sparse_values);
}

int dsa_calib_stream_read(const void* buffer, size_t bytes, int32_t nontemporal, uint32_t* sink, void* stream) {
  g_err[0] = '\0';
  DSA_CHECK_ARG(buffer, "null buffer pointer");
  DSA_CHECK_ARG(bytes >= 16 && bytes % 16 == 0, "bytes must be a positive multiple of 16, got %zu", bytes);
  DSA_CHECK_ARG(((uintptr_t)buffer & 15) == 0, "buffer must be 16-byte aligned");
  return calib_stream_read_run(buffer, bytes, nontemporal, sink, (hipStream_t)stream);
}

}  // extern "C"
