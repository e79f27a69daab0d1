// Row / token addressing shared by the sparse indexer KL-loss kernels
// (kl_bwd.hip: the fused row kernel and the dKi reduction; kl_generic.hip:
// the path for index shapes the fused kernel does not take).
#pragma once

#include "kl_common.h"

namespace dsa {

// Query-row and key-row addressing of one call.  Query rows are b*S1 + s1
// (BSND) or packed with cumulative lengths (TND); key rows are b*S2 + t
// (BSND), packed (TND) or pages of a cache through a block table (PA_BSND).
// Length arrays are cumulative for a TND side, per-batch lengths otherwise.
struct KlMap {
  const int32_t* act_q;
  const int32_t* act_k;
  const int32_t* block_table;  // [batch, max_blocks] (PA_BSND key)
  int64_t kv_rows;             // key rows in memory
  int32_t batch, s1, s2, rows, topk, max_blocks, page_size;
  int32_t layout_q, layout_k;
};

struct KlRow {
  int b, s1, n;
  int klen;       // clamp bound of the row's token ids (S2, or the packed / paged length)
  int64_t kbase;  // first key row of the row's batch (BSND / TND)
  bool active;
};

// A row's batch, position and slot count n = min(topK, max(act_k - act_q +
// s1 + 1, 0)) (kernel line 107); inactive rows (s1 >= act_q) have n = 0.
__device__ __forceinline__ KlRow kl_row_info(const KlMap& m, int row) {
  KlRow r;
  int aq, ak;
  if (m.layout_q == DSA_LAYOUT_TND) {
    int lo = 0, hi = m.batch - 1;  // first b with cu[b] > row
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (m.act_q[mid] > row) hi = mid; else lo = mid + 1;
    }
    r.b = lo;
    const int start = lo ? m.act_q[lo - 1] : 0;
    r.s1 = row - start;
    aq = m.act_q[lo] - start;
  } else {
    r.b = row / m.s1;
    r.s1 = row - r.b * m.s1;
    aq = m.act_q ? m.act_q[r.b] : m.s1;
  }
  if (m.layout_k == DSA_LAYOUT_TND) {
    const int start = r.b ? m.act_k[r.b - 1] : 0;
    r.kbase = start;
    ak = m.act_k[r.b] - start;
    r.klen = ak;
  } else if (m.layout_k == DSA_LAYOUT_PA_BSND) {
    r.kbase = 0;
    r.klen = m.max_blocks * m.page_size;
    ak = m.act_k ? m.act_k[r.b] : r.klen;
  } else {
    r.kbase = (int64_t)r.b * m.s2;
    r.klen = m.s2;
    ak = m.act_k ? m.act_k[r.b] : m.s2;
  }
  r.active = r.s1 < aq;
  r.n = r.active ? min(m.topk, max(ak - aq + r.s1 + 1, 0)) : 0;
  return r;
}

// Key row of slot k: the token id clamped to [0, klen) with no -1 test (lines
// 58, 63, 300), then translated through the block table for a paged cache.
// -1 marks a token in a -1 (or out-of-range) page: it reads as a zero key
// row and receives no gradient.  Key rows past the end of the key tensor
// (cumulative lengths larger than it) are treated the same way.
__device__ __forceinline__ int kl_token(const KlMap& m, const KlRow& r, const int32_t* idx, int row, int k) {
  const int t = min(max(idx[(int64_t)row * m.topk + k], 0), r.klen - 1);
  if (m.layout_k != DSA_LAYOUT_PA_BSND) {
    const int64_t g = r.kbase + t;
    return g < m.kv_rows ? (int)g : -1;
  }
  const int blk = m.block_table[(int64_t)r.b * m.max_blocks + t / m.page_size];
  const int64_t phys = (int64_t)blk * m.page_size + t % m.page_size;
  return (blk < 0 || phys >= m.kv_rows) ? -1 : (int)phys;
}

// The generic path (kl_generic.hip): Nidx1 up to kGenMaxNidx, an index head
// dim up to kGenMaxDi with 16-byte rows, any topK.
constexpr int kGenMaxNidx = 128;
constexpr int kGenMaxDi = 256;

struct KlGenParams {
  KlMap m;
  const void* q;
  const void* qr;
  const void* k;
  const void* kr;
  const void* qi;
  const void* ki;
  const void* w;
  const int32_t* idx;
  const float* smax;
  const float* ssum;
  void* dqi;
  void* dw;
  _Float16* cbuf;    // dKi contribution c (di values) as fp16 c * 2^rowexp, at the slot's bucket place
  float* rowmax;     // [rows] max |c|
  int32_t* rowexp;   // [rows]
  const int32_t* offs;  // [tokens + 1] bucket starts
  const int32_t* rank;  // [rows * topK] the slot's place in its token's bucket (within its row chunk)
  const int32_t* cbase; // [chunks][tokens] the row chunk's start within each bucket, or null
  int32_t chunk_rows, tokens;
  int32_t* posrow;      // [rows * topK] row of the contribution at each bucket position
  uint32_t* tokmax;     // [tokens] largest row maximum among the token's slots (float bits)
  float* loss_part;  // [rows]
  float* pi;         // [rows][topK][2]: teacher p (then dI) and index score I
  int32_t n1, nidx, di, dip, topk, w_dtype;
  float scale_log2;
};

hipError_t kl_gen_run(const KlGenParams& p, int rows, int d, int dr, bool bf16_io, hipStream_t stream);

}  // namespace dsa
