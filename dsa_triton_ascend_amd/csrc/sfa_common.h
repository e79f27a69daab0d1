// Row and index resolution shared by the sparse flash attention kernels
// (forward and backward): the masks of the reference kernels
// (sparse_flash_attention_triton.py:247-254, 270-272;
// sparse_flash_attention_grad_triton.py:204-208, 246) and the layout
// handling the reference does on the host (TND cumulative lengths, PA_BSND
// block_table, block-wise ids; sparse_flash_attention_triton.py:345-421).
// The parameter structs of both kernels carry the fields used here.
//
// Band mask: the reference accepts only pre_tokens = next_tokens = INT64_MAX
// (sparse_flash_attention_triton.py:531-532).  Other values select the band
// of the Ascend FlashAttention operators: token t of a row is visible iff
// diag - pre_tokens <= t <= diag + next_tokens, with diag = s1 in mode 0 and
// act_k - act_q + s1 in mode 3.  The host clamps both to +-kBandOpen, which
// keeps the sums below in int64 range and makes INT64_MAX an open side
// (|diag| < 2^32 and tokens lie in [0, 2^31)).
#pragma once

#include "common.h"

namespace dsa {

constexpr int64_t kBandOpen = 1ll << 40;

__host__ __device__ inline int64_t band_clamp(int64_t v) {
  return v > kBandOpen ? kBandOpen : (v < -kBandOpen ? -kBandOpen : v);
}

struct RowInfo {
  int b, s1, act_q, act_k;
  // tokens lo <= t < hi are attended: hi = min(act_k, causal threshold,
  // next_tokens bound), lo = the pre_tokens bound (0 without a band)
  int lo, hi;
  int64_t kv_base;
  bool active;
};

template <typename P>
__device__ __forceinline__ RowInfo sfa_row_info(const P& p, int row) {
  RowInfo ri;
  if (p.layout_q == DSA_LAYOUT_TND) {
    // cumulative lengths: first b with cu[b] > row
    int lo = 0, hi = p.batch - 1;
    while (lo < hi) {
      int mid = (lo + hi) >> 1;
      if (p.act_q[mid] > row) hi = mid; else lo = mid + 1;
    }
    ri.b = lo;
    int start = lo ? p.act_q[lo - 1] : 0;
    ri.s1 = row - start;
    ri.act_q = p.act_q[lo] - start;
  } else {
    ri.b = row / p.s1;
    ri.s1 = row - ri.b * p.s1;
    ri.act_q = p.act_q ? p.act_q[ri.b] : p.s1;
  }
  if (p.layout_kv == DSA_LAYOUT_TND) {
    int start = ri.b ? p.act_k[ri.b - 1] : 0;
    ri.kv_base = start;
    ri.act_k = p.act_k[ri.b] - start;
  } else {
    ri.kv_base = (int64_t)ri.b * p.s2;  // unused for PA_BSND
    ri.act_k = p.act_k ? p.act_k[ri.b] : p.s2;
  }
  const int64_t thr = p.mode == 0 ? ri.act_k : (int64_t)ri.act_k - ri.act_q + ri.s1 + 1;
  const int64_t diag = p.mode == 0 ? (int64_t)ri.s1 : (int64_t)ri.act_k - ri.act_q + ri.s1;
  // band_pre / band_next are clamped to +-kBandOpen on the host
  const int64_t hi = min(min(thr, (int64_t)ri.act_k), diag + p.band_next + 1);
  const int64_t lo = diag - p.band_pre;
  ri.hi = (int)max(hi, (int64_t)0);
  ri.lo = (int)min(max(lo, (int64_t)0), (int64_t)0x7fffffff);
  // a row with no visible token resolves nothing (its outputs stay zero,
  // like a row of -1 ids)
  ri.active = (ri.s1 < ri.act_q) && (ri.hi > ri.lo);
  return ri;
}

// Resolve index position `pos` of a row to a physical KV row.
// Returns false if the position is not attended; *phys = -1 marks a token that
// is attended but lives in a -1 / out-of-range page (reads as a zero row, as
// the reference's de-paging leaves such spans zero, lines 391-397).
// The index entry of position `pos` (split from the resolution below so the
// load need not wait for the row's length loads).
template <typename P>
__device__ __forceinline__ int sfa_load_id(const P& p, const int32_t* idx_row, int pos) {
  return idx_row[pos / p.bs];
}

// `tab` is the row's block-table row (PA_BSND), in global memory or staged
// in LDS by the caller.
template <typename P>
__device__ __forceinline__ bool sfa_resolve_id(const P& p, const RowInfo& ri, int id, int pos, int* phys,
                                               const int32_t* tab) {
  if (id < 0) return false;
  int64_t tok = (int64_t)id * p.bs + (pos % p.bs);
  if (tok >= ri.hi || tok < ri.lo) return false;
  if (p.layout_kv == DSA_LAYOUT_PA_BSND) {
    if (tok >= (int64_t)p.max_blocks * p.page_size) return false;
    int blk = tab[tok / p.page_size];
    int64_t r = (int64_t)blk * p.page_size + tok % p.page_size;
    *phys = (blk < 0 || r >= p.kv_rows) ? -1 : (int)r;
    return true;
  }
  if (p.layout_kv == DSA_LAYOUT_BSND && tok >= p.s2) return false;
  int64_t r = ri.kv_base + tok;
  if (r >= p.kv_rows) return false;
  *phys = (int)r;
  return true;
}

template <typename P>
__device__ __forceinline__ bool sfa_resolve(const P& p, const RowInfo& ri, const int32_t* idx_row,
                                            int pos, int* phys) {
  const int32_t* tab = p.layout_kv == DSA_LAYOUT_PA_BSND ? p.block_table + (int64_t)ri.b * p.max_blocks : nullptr;
  return sfa_resolve_id(p, ri, sfa_load_id(p, idx_row, pos), pos, phys, tab);
}

}  // namespace dsa
