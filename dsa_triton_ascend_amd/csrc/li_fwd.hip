// Lightning indexer for gfx950: MFMA score kernel + stable radix top-k.
//
// Semantics follow the reference score kernel
// `_lightning_indexer_score_kernel` (lightning_indexer_triton.py:147-280) and
// the stable top-k the readme specifies (readme.md:63-69; `_stable_topk`,
// lightning_indexer_triton.py:339-357):
//   score[b, s1, n2, s2] = sum_g max(q[b,s1,n2*G+g,:] . k[b,s2,n2,:], 0) * w[b,s1,n2*G+g]
// in fp32 with no scale (264-269); keys s2 >= act_k are masked (274); in
// sparse_mode 3 keys s2 >= min(max(act_k-act_q+s1+1, 0), S2) are masked
// (219-224, 272-273); rows with s1 >= act_q see nothing (227, 275-276).
// Masked entries are -inf.  The top-k order is score descending, index
// ascending on ties; -inf entries (and padding when fewer than K keys are
// visible) are reported as index -1 with value -inf.
//
// Score kernel: one workgroup per (query row, n2, chunk of keys).  The G
// heads of the row live in registers as MFMA A operands (16 heads x 32 d per
// fragment); K fragments (32 d x 16 keys) are loaded straight from HBM as B
// operands, 16 bytes per lane, two groups ahead, so the kernel streams K at
// the memory rate (decode is HBM-bound: 64 flop per key byte at G=64, D=128).
// C[head][key] is reduced over heads after ReLU and weighting: lane-local
// over registers and head tiles, then a 4-lane butterfly.
//
// Top-k kernel: one workgroup (1024 threads) per row.  Scores map to
// order-preserving uint32 keys.  Rows of up to 32768 scores take the fast
// selection (li_topk_kernel below): a 4096-bin histogram of the 12 key bits
// under the common prefix of the row's finite keys finds the bin holding
// the K-th largest key; the candidates in that bin and above are counting-
// sorted by bin, and each one's final position is its bin start plus its
// rank within the bin by the composite (~key << 32 | index), which is
// exactly score descending / index ascending.  Wider rows, more than 4096
// candidates, or a crowded bin take the general selection: a radix select
// of the K-th largest key, an ordered selection of the ties, and a bitonic
// sort of the selected composites in LDS.
#include <type_traits>

#include "common.h"

namespace dsa {

// ---------------------------------------------------------------------------
// score kernel
// ---------------------------------------------------------------------------
struct LiParams {
  const void* q;
  const void* k;
  const void* w;
  const int32_t* act_q;
  const int32_t* act_k;
  float* scores;       // [q_rows * n2, s2] (row stride s2)
  int64_t q_rows, k_rows;
  int32_t batch, s1, s2, n1, n2, g;
  int32_t d;           // head dim (the row stride of q and k)
  int32_t mode, layout_q, layout_k, w_dtype;
  int32_t chunk;       // keys per workgroup
  int32_t row_tiles;   // multi-row kernel: 64-key tiles per workgroup (blockIdx.y), 0 = the whole row
  int32_t xcd_group;   // one-row kernel: query rows per batch placed on one XCD (0: blockIdx.x order)
  // PA_BSND key cache [blocks, page, N2, D]: key s2 of batch b is row
  // block_table[b, s2 / page] * page + s2 % page (k_rows = blocks * page)
  const int32_t* block_table;
  int32_t max_blocks, page_size;
  int32_t page_shift;  // log2(page_size) for a power of two, else -1
};

// Page of key `key` and its row in the page: a shift and a mask for the
// usual power-of-two page sizes, where an integer division by the runtime
// page size costs some tens of instructions per key
__device__ __forceinline__ int li_page(const LiParams& p, int key) {
  if (p.page_shift >= 0) return key >> p.page_shift;
  return key / p.page_size;
}
__device__ __forceinline__ int li_in_page(const LiParams& p, int key) {
  if (p.page_shift >= 0) return key & (p.page_size - 1);
  return key % p.page_size;
}

constexpr int kLiThreads = 256;

constexpr int kLiChunk = 1024;  // default keys per workgroup (resized at launch)

struct LiRow {
  int b, s1, lim;       // visible keys are [0, lim)
  int64_t k_base;       // first key row of batch b
};

__device__ __forceinline__ LiRow li_row_info(const LiParams& p, int row) {
  LiRow r;
  int aq, ak;
  if (p.layout_q == DSA_LAYOUT_TND) {
    int lo = 0, hi = p.batch - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (p.act_q[mid] > row) hi = mid; else lo = mid + 1;
    }
    r.b = lo;
    const int start = lo ? p.act_q[lo - 1] : 0;
    r.s1 = row - start;
    aq = p.act_q[lo] - start;
  } else {
    r.b = row / p.s1;
    r.s1 = row - r.b * p.s1;
    aq = p.act_q ? p.act_q[r.b] : p.s1;
  }
  if (p.layout_k == DSA_LAYOUT_PA_BSND) {
    // paged keys: per-batch lengths whatever the query layout (as the SFA
    // forward's PA_BSND key); rows come from the block table
    r.k_base = 0;
    ak = p.act_k[r.b];
  } else if (p.layout_k == DSA_LAYOUT_TND || p.layout_q == DSA_LAYOUT_TND) {
    // with a TND query both length arrays are cumulative (the reference
    // converts both, lightning_indexer_triton.py:500-506)
    const int start = r.b ? p.act_k[r.b - 1] : 0;
    r.k_base = p.layout_k == DSA_LAYOUT_TND ? (int64_t)start : (int64_t)r.b * p.s2;
    ak = p.act_k[r.b] - start;
  } else {
    r.k_base = (int64_t)r.b * p.s2;
    ak = p.act_k ? p.act_k[r.b] : p.s2;
  }
  int lim;
  if (r.s1 >= aq) lim = 0;
  else if (p.mode == 3) lim = min(ak, min(max(ak - aq + r.s1 + 1, 0), p.s2));
  else lim = min(ak, p.s2);
  r.lim = max(lim, 0);
  return r;
}

__device__ __forceinline__ float li_load_w(const LiParams& p, int64_t idx) {
  if (p.w_dtype == DSA_DTYPE_FP32) return ((const float*)p.w)[idx];
  if (p.w_dtype == DSA_DTYPE_BF16) return (float)((const bf16*)p.w)[idx];
  return (float)((const f16*)p.w)[idx];
}

// D = head dim, GT = head tiles of 16 (G <= 16*GT).  The chunk's scores
// collect in LDS and leave in coalesced 16-byte stores at the end.  At the
// decode shape one workgroup per CU streams K at about 6.7 TB/s in its
// steady state (about 5.5 TB/s over the whole launch, with the start-up
// and the tail); a plain streaming read of 1 GiB reaches 6.2-6.45 TB/s.
// PAD: the head dim p.d is below D (a multiple of 8); the 8-element chunks
// at or past p.d load as zeros, so the MFMAs see zero-padded rows of D.
constexpr int kLiMaxChunk = 8192;  // keys per workgroup (LDS score buffer)

// Scores of the chunk [c0, c1) from s_sc to the row, in coalesced 16-byte
// stores where the destination is 16-byte aligned; keys in -1 (or
// out-of-range) pages of a paged cache are zero rows, score 0 while visible.
// s_bt: the chunk's block-table entries staged in LDS from entry bt0 (null:
// read the table in memory).
__device__ __forceinline__ void li_store_chunk(const LiParams& p, const LiRow& ri, const int32_t* btab, float* s_sc,
                                               float* srow, int c0, int c1, const int* s_bt = nullptr,
                                               int bt0 = 0) {
  const int n = c1 - c0;
  if (p.layout_k == DSA_LAYOUT_PA_BSND) {
    const int64_t nblk = p.k_rows / p.page_size;
    for (int j = threadIdx.x; j < n; j += kLiThreads) {
      const int key = c0 + j;
      if (key < ri.lim) {
        const int e = li_page(p, key);
        const int blk = s_bt ? s_bt[e - bt0] : btab[e];
        if (blk < 0 || blk >= nblk) s_sc[j] = 0.f;
      }
    }
    __syncthreads();
  }
  float* dst = srow + c0;
  const int head = (int)(((16 - ((uintptr_t)dst & 15)) & 15) >> 2);  // scalars before 16-byte alignment
  const int h = head < n ? head : n;
  for (int j = threadIdx.x; j < h; j += kLiThreads) dst[j] = s_sc[j];
  const int n4 = (n - h) >> 2;
  for (int j = threadIdx.x; j < n4; j += kLiThreads) {
    const float4 v = make_float4(s_sc[h + 4 * j], s_sc[h + 4 * j + 1], s_sc[h + 4 * j + 2], s_sc[h + 4 * j + 3]);
    *(float4*)(dst + h + 4 * j) = v;
  }
  for (int j = h + 4 * n4 + threadIdx.x; j < n; j += kLiThreads) dst[j] = s_sc[j];
}

// Physical key row of visible key `key` of a row (clamped into the tensor).
__device__ __forceinline__ int64_t li_key_row(const LiParams& p, const LiRow& ri, const int32_t* btab, int key) {
  int64_t krow = ri.k_base + key;
  if (p.layout_k == DSA_LAYOUT_PA_BSND) {
    // a -1 or out-of-range page reads row 0; its scores are set to zero
    // when the chunk is stored (a zero key row, as de-paging leaves it)
    const int blk = btab[key / p.page_size];
    krow = (int64_t)(blk < 0 ? 0 : blk) * p.page_size + key % p.page_size;
  }
  return krow < p.k_rows ? krow : p.k_rows - 1;  // inconsistent cumulative lengths stay in bounds
}

// Paged keys: the block-table entries a chunk's key loads use, staged in
// LDS before the key ring starts, so that each key load waits for an LDS
// read instead of a dependent load of its table entry from memory (and the
// page check at the store reads LDS too).  Launches size the chunks so that
// their entries fit kLiBtStage (li_paged_chunk_cap).
constexpr int kLiBtStage = 1024;
constexpr int kLiBtPer = kLiBtStage / kLiThreads;  // entries per thread

__device__ __forceinline__ int64_t li_key_row_staged(const LiParams& p, const LiRow& ri, const int* s_bt, int bt0,
                                                     int key) {
  int64_t krow = ri.k_base + key;
  if (p.layout_k == DSA_LAYOUT_PA_BSND) {
    const int blk = s_bt[li_page(p, key) - bt0];  // a -1 page reads row 0; scored 0 at the store
    krow = (int64_t)(blk < 0 ? 0 : blk) * p.page_size + li_in_page(p, key);
  }
  return krow < p.k_rows ? krow : p.k_rows - 1;
}

// The table loads of the chunk's keys [c0, kend), issued unconditionally
// (indices clamped into the range: a load under a lane condition is waited
// for on the spot); li_tab_stage_store writes them to LDS after the
// caller's other prologue loads are issued, then a barrier.
__device__ __forceinline__ void li_tab_stage_load(const LiParams& p, const int32_t* btab, int c0, int kend,
                                                  int (&tv)[kLiBtPer], int& bt0, int& ne) {
  bt0 = c0 / p.page_size;
  ne = min((kend - 1) / p.page_size - bt0 + 1, kLiBtStage);  // the launch cap keeps it below the bound
#pragma unroll
  for (int u = 0; u < kLiBtPer; ++u) tv[u] = btab[bt0 + min(u * kLiThreads + (int)threadIdx.x, ne - 1)];
}
__device__ __forceinline__ void li_tab_stage_store(int* s_bt, const int (&tv)[kLiBtPer], int ne) {
#pragma unroll
  for (int u = 0; u < kLiBtPer; ++u)
    if (u * kLiThreads + (int)threadIdx.x < ne) s_bt[u * kLiThreads + threadIdx.x] = tv[u];
  __syncthreads();
}

// NT: non-temporal key loads, for launches where no other query row reads
// the same keys (one query row per batch, as at decode): the keys then have
// no reuse to keep in the caches.
template <int D, typename T, int GT, bool PAD, bool NT>
__global__ __launch_bounds__(kLiThreads) void li_score_kernel(LiParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 32;
  const int dstride = PAD ? p.d : D;
  __shared__ __attribute__((aligned(16))) float s_sc[kLiMaxChunk];
  __shared__ int s_bt[kLiBtStage];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  // row * n2 + n2 index.  With xcd_group = G (BSND, N2 = 1, G query rows
  // per batch, rows a multiple of 8 G) the G rows of a batch, which read the
  // same keys, go to one XCD (workgroup x runs on XCD x % 8) so that the
  // keys one of them brings into that XCD's L2 serve the others
  int rn = blockIdx.x;
  if (p.xcd_group > 1) {
    const int G = p.xcd_group, xcd = rn & 7, j = rn >> 3;
    rn = ((j / G) * 8 + xcd) * G + j % G;
  }
  const int row = rn / p.n2;
  const int kh = rn - row * p.n2;
  const LiRow ri = li_row_info(p, row);
  const int c0 = blockIdx.y * p.chunk;
  const int c1 = min(p.s2, c0 + p.chunk);
  float* srow = p.scores + (int64_t)rn * p.s2;
  if (c0 >= ri.lim) {
    // nothing visible in this chunk
    for (int j = c0 + threadIdx.x; j < c1; j += kLiThreads) srow[j] = -INFINITY;
    return;
  }

  // paged keys: the chunk's table entries are loaded first (staged in LDS
  // after the weight and Q loads are issued)
  const bool paged = p.layout_k == DSA_LAYOUT_PA_BSND;
  const int32_t* btab = paged ? p.block_table + (int64_t)ri.b * p.max_blocks : nullptr;
  const int ngroups = (c1 - c0 + 15) >> 4;
  int tv[kLiBtPer], bt0 = 0, ne = 0;
  if (paged) li_tab_stage_load(p, btab, c0, min(c0 + 16 * ngroups, ri.lim), tv, bt0, ne);
  // weight of head ht*16 + 4*lg + r (the C-layout rows of this lane),
  // loaded first, as raw bits under one width branch, and converted only
  // after the first key groups are issued: loads issued before the branch,
  // or a conversion inside it, make the compiler wait for them there
  uint32_t wraw[GT][4];
  const int64_t wbase = (int64_t)row * p.n1 + kh * p.g;
  auto load_w = [&](auto* wp) {
#pragma unroll
    for (int ht = 0; ht < GT; ++ht)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gg = ht * 16 + lg * 4 + r;
        wraw[ht][r] = wp[wbase + (gg < p.g ? gg : 0)];  // unconditional: no branch per load
      }
  };
  if (p.w_dtype == DSA_DTYPE_FP32) load_w((const uint32_t*)p.w);
  else load_w((const uint16_t*)p.w);
  // Q fragments (A operand): lane -> head ht*16 + li, d = ks*32 + 8*lg ..
  V8 qf[GT][KS];
#pragma unroll
  for (int ht = 0; ht < GT; ++ht) {
    const int g = ht * 16 + li;
    const bool gv = g < p.g;
    const int64_t qrow = (int64_t)row * p.n1 + kh * p.g + (gv ? g : 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bool dv = !PAD || ks * 32 + lg * 8 < p.d;
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 v = dv ? *(const u32x4*)((const T*)p.q + qrow * dstride + (dv ? ks * 32 + lg * 8 : 0)) : z;
      qf[ht][ks] = as_v8<V8>(gv ? v : z);
    }
  }

  if (paged) li_tab_stage_store(s_bt, tv, ne);
  // key groups of 16: wave w takes groups w, w+4, ...; K fragment of group
  // kg (B operand): lane -> key kg*16 + li, d = ks*32 + 8*lg ..
  const int lastvis = ri.lim - 1;
  // NP groups in flight per wave (ring of K fragment registers).  Loads are
  // issued unconditionally (groups past the end reload the last one), so no
  // load sits under a branch.
  auto kload = [&](int grp, u32x4 (&kf)[KS]) {
    int key = c0 + grp * 16 + li;
    key = key < lastvis ? key : lastvis;  // stays in the batch's rows; masked below
    const int64_t krow = li_key_row_staged(p, ri, s_bt, bt0, key);
    const T* kp = (const T*)p.k + (krow * p.n2 + kh) * dstride + lg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (!PAD || ks * 32 + lg * 8 < p.d) {
        if constexpr (NT) kf[ks] = __builtin_nontemporal_load((const u32x4*)(kp + ks * 32));
        else kf[ks] = *(const u32x4*)(kp + ks * 32);
      }
      else kf[ks] = (u32x4){0u, 0u, 0u, 0u};
    }
  };
  constexpr int NP = 4;
  u32x4 kf[NP][KS];
#pragma unroll
  for (int i = 0; i < NP; ++i) kload(min(wave + 4 * i, ngroups - 1), kf[i]);
  float wv[GT][4];
#pragma unroll
  for (int ht = 0; ht < GT; ++ht)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t b = wraw[ht][r];
      const float x = p.w_dtype == DSA_DTYPE_FP32 ? __uint_as_float(b)
                      : p.w_dtype == DSA_DTYPE_BF16 ? __uint_as_float(b << 16)
                                                    : (float)__builtin_bit_cast(f16, (uint16_t)b);
      wv[ht][r] = ht * 16 + lg * 4 + r < p.g ? x : 0.f;
    }
  auto process = [&](int gi, const u32x4 (&kf)[KS]) {
    f32x4 acc[GT];
#pragma unroll
    for (int ht = 0; ht < GT; ++ht) acc[ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const V8 bv = as_v8<V8>(kf[ks]);
#pragma unroll
      for (int ht = 0; ht < GT; ++ht) acc[ht] = E::mfma(qf[ht][ks], bv, acc[ht]);
    }
    float s = 0.f;
#pragma unroll
    for (int ht = 0; ht < GT; ++ht)
#pragma unroll
      for (int r = 0; r < 4; ++r) s += relu_bits(acc[ht][r]) * wv[ht][r];
    s = xgroup_sum(s);
    const int key = c0 + gi * 16 + li;
    if (lg == 0 && key < c1) s_sc[gi * 16 + li] = key < ri.lim ? s : -INFINITY;
  };
  for (int grp = wave; grp < ngroups; grp += 4 * NP) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int gi = grp + 4 * i;
      if (gi < ngroups) process(gi, kf[i]);
      kload(min(gi + 4 * NP, ngroups - 1), kf[i]);
    }
  }
  __syncthreads();
  li_store_chunk(p, ri, btab, s_sc, srow, c0, c1, s_bt, bt0);
}

// ---------------------------------------------------------------------------
// Two query rows per batch (BSND query, N2 = 1, S1 = 2: multi-token decode
// with one draft token; exact head dims, 16-bit inputs).  A workgroup takes
// both rows of a batch over one key chunk: every K fragment is loaded once
// (non-temporal: no other workgroup reads these keys) and multiplied with
// both rows' Q fragments, where the one-row kernel streamed each key once
// per row.  The key range is the union of the two rows' visible ranges;
// each row masks its own limit.  NP groups of 16 keys in flight per wave.
// ---------------------------------------------------------------------------
constexpr int kLiPairMaxChunk = 4096;  // keys per workgroup (two LDS score rows)
constexpr int kLiPairRing = 4;         // groups of 16 keys in flight per wave

template <int D, typename T, int GT, int NP>
__global__ __launch_bounds__(kLiThreads) void li_score_pair_kernel(LiParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 32;
  __shared__ __attribute__((aligned(16))) float s_sc[2][kLiPairMaxChunk];
  __shared__ int s_bt[kLiBtStage];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int row0 = 2 * (int)blockIdx.x;
  const LiRow ri0 = li_row_info(p, row0);
  const LiRow ri1 = li_row_info(p, row0 + 1);
  const int lim = max(ri0.lim, ri1.lim);
  const int c0 = blockIdx.y * p.chunk;
  const int c1 = min(p.s2, c0 + p.chunk);
  float* srow0 = p.scores + (int64_t)row0 * p.s2;
  float* srow1 = srow0 + p.s2;
  if (c0 >= lim) {
    for (int j = c0 + threadIdx.x; j < c1; j += kLiThreads) {
      srow0[j] = -INFINITY;
      srow1[j] = -INFINITY;
    }
    return;
  }
  const bool paged = p.layout_k == DSA_LAYOUT_PA_BSND;
  const int32_t* btab = paged ? p.block_table + (int64_t)ri0.b * p.max_blocks : nullptr;
  const int ngroups = (c1 - c0 + 15) >> 4;
  int tv[kLiBtPer], bt0 = 0, ne = 0;
  if (paged) li_tab_stage_load(p, btab, c0, min(c0 + 16 * ngroups, lim), tv, bt0, ne);
  // weights as raw bits (converted after the first key groups are issued)
  uint32_t wraw[2][GT][4];
  auto load_w = [&](auto* wp) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int ht = 0; ht < GT; ++ht)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int gg = ht * 16 + lg * 4 + e;
          wraw[r][ht][e] = wp[(int64_t)(row0 + r) * p.n1 + (gg < p.g ? gg : 0)];
        }
  };
  if (p.w_dtype == DSA_DTYPE_FP32) load_w((const uint32_t*)p.w);
  else load_w((const uint16_t*)p.w);
  V8 qf[2][GT][KS];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ht = 0; ht < GT; ++ht) {
      const int g = ht * 16 + li;
      const bool gv = g < p.g;
      const int64_t qrow = (int64_t)(row0 + r) * p.n1 + (gv ? g : 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        const u32x4 v = *(const u32x4*)((const T*)p.q + qrow * D + ks * 32 + lg * 8);
        qf[r][ht][ks] = as_v8<V8>(gv ? v : z);
      }
    }
  if (paged) li_tab_stage_store(s_bt, tv, ne);
  const int lastvis = lim - 1;
  auto kload = [&](int grp, u32x4 (&kf)[KS]) {
    int key = c0 + grp * 16 + li;
    key = key < lastvis ? key : lastvis;
    const int64_t krow = li_key_row_staged(p, ri0, s_bt, bt0, key);
    const T* kp = (const T*)p.k + krow * D + lg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = __builtin_nontemporal_load((const u32x4*)(kp + ks * 32));
  };
  u32x4 kf[NP][KS];
#pragma unroll
  for (int i = 0; i < NP; ++i) kload(min(wave + 4 * i, ngroups - 1), kf[i]);
  float wv[2][GT][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ht = 0; ht < GT; ++ht)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b = wraw[r][ht][e];
        const float x = p.w_dtype == DSA_DTYPE_FP32 ? __uint_as_float(b)
                        : p.w_dtype == DSA_DTYPE_BF16 ? __uint_as_float(b << 16)
                                                      : (float)__builtin_bit_cast(f16, (uint16_t)b);
        wv[r][ht][e] = ht * 16 + lg * 4 + e < p.g ? x : 0.f;
      }
  auto process = [&](int gi, const u32x4 (&kf)[KS]) {
    const int key = c0 + gi * 16 + li;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      f32x4 acc[GT];
#pragma unroll
      for (int ht = 0; ht < GT; ++ht) acc[ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8 bv = as_v8<V8>(kf[ks]);
#pragma unroll
        for (int ht = 0; ht < GT; ++ht) acc[ht] = E::mfma(qf[r][ht][ks], bv, acc[ht]);
      }
      float sc = 0.f;
#pragma unroll
      for (int ht = 0; ht < GT; ++ht)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc += relu_bits(acc[ht][e]) * wv[r][ht][e];
      sc = xgroup_sum(sc);
      const int rl = r == 0 ? ri0.lim : ri1.lim;
      if (lg == 0 && key < c1) s_sc[r][gi * 16 + li] = key < rl ? sc : -INFINITY;
    }
  };
  for (int grp = wave; grp < ngroups; grp += 4 * NP) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int gi = grp + 4 * i;
      if (gi < ngroups) process(gi, kf[i]);
      kload(min(gi + 4 * NP, ngroups - 1), kf[i]);
    }
  }
  __syncthreads();
  li_store_chunk(p, ri0, btab, s_sc[0], srow0, c0, c1, s_bt, bt0);
  li_store_chunk(p, ri1, btab, s_sc[1], srow1, c0, c1, s_bt, bt0);
}

// ---------------------------------------------------------------------------
// Multi-row score kernel (BSND query, several query rows per batch, exact
// head dims 64 / 128 / 256, 16-bit inputs).  One workgroup = kLiRows (4)
// consecutive query rows s0 .. s0+3 of one (batch, key head); wave w owns
// row s0 + w.  The rows share every key tile: tiles of 64 keys go HBM/L2 ->
// LDS by LDS-DMA (global_load_lds_dwordx4, 1 KB per instruction) into a
// 3-buffer ring, and each wave reads its K fragments (B operands) from LDS
// while its row's G heads of Q stay in registers (A operands).  One query
// row per workgroup (the chunked kernel above) re-reads every visible key
// per row, which at the cfg2 prefill shape is 4.3 GB of L2 reads; here each
// key row is read once per 4 query rows.  Four rows (one wave per SIMD, 49
// KB of LDS, three workgroups per CU) measured faster than eight (two waves
// per SIMD, one workgroup per CU): cfg2 373 -> 351 us.  Key rows are stored in LDS with 16-byte
// chunk c of tile row r at chunk c ^ (r & 15) (r & 7 at D = 64), so the 16
// lanes of a fragment read (16 rows, one chunk column) hit distinct banks.
// Workgroups run the longest causal rows first.  A wave's vector-memory
// operations per tile are exactly its NDW DMAs and one 64-key score store
// (inline asm, so the count cannot change), which the ring's vmcnt waits
// count on.
// ---------------------------------------------------------------------------
constexpr int kLiRows = 4;       // query rows per workgroup (one per wave, one wave per SIMD)
constexpr int kLiRowTile = 64;   // keys per LDS tile

__device__ __forceinline__ void li_dma16(unsigned lds_base, const void* gaddr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_base), "v"(gaddr) : "memory");
}
__device__ __forceinline__ void li_store_f32(float* addr, float v) {
  asm volatile("global_store_dword %0, %1, off" :: "v"(addr), "v"(v) : "memory");
}
template <int N> __device__ __forceinline__ void li_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// Zero key row: the DMA source of keys in -1 (or out-of-range) pages of a
// paged cache, which de-paging leaves as zero rows (score 0 while visible).
__device__ __attribute__((aligned(16))) unsigned char g_li_zero_row[512];

constexpr int kLiRowBufs = 3;   // LDS ring of key tiles
template <int D> constexpr int li_row_tile_bytes() { return kLiRowTile * D * 2; }

// The score rows of one workgroup (body of the kernels below): s_k is the
// kLiRowBufs-tile ring, s_lim kLiRows words, s_bt kLiBtRows words.
constexpr int kLiBtRows = kLiRows * 64;  // staged table entries (one per thread)
// PG: the keys are a paged cache (a separate instantiation, so that the
// dense-key code carries none of the page handling)
template <int D, typename T, int GT, bool PG>
__device__ __forceinline__ void li_rows_scores(const LiParams& p, unsigned char (*s_k)[li_row_tile_bytes<D>()],
                                               int* s_lim, int* s_bt, int tnd_seq = -1) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 32;                       // k-steps
  constexpr int CPR = D / 8;                       // 16-byte chunks per key row
  constexpr int RPD = 64 / CPR;                    // key rows per 1 KB DMA
  constexpr int TB = li_row_tile_bytes<D>();       // tile bytes
  constexpr int NDW = TB / 1024 / kLiRows;         // DMAs per wave per tile
  constexpr int SWM = CPR < 16 ? CPR - 1 : 15;     // chunk swizzle mask
  constexpr int NBUF = kLiRowBufs;
  static_assert(NDW >= 1 && NDW * kLiRows * 1024 == TB, "tile DMAs");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  int kh = 0, row;
  bool active;
  LiRow ri, rs;  // this wave's row; a row of the sequence whose keys the tiles hold
  if (tnd_seq < 0) {
    const int nbk = p.batch * p.n2;
    const int ngroups = (p.s1 + kLiRows - 1) / kLiRows;
    const int bk = blockIdx.x % nbk;
    const int grp = ngroups - 1 - (int)(blockIdx.x / nbk);  // longest rows first
    const int b = bk / p.n2;
    kh = bk - b * p.n2;
    const int s1 = grp * kLiRows + wave;
    active = s1 < p.s1;
    row = b * p.s1 + (active ? s1 : 0);
    ri = li_row_info(p, row);
    rs = ri;
  } else {
    // packed (TND) rows, one key head: group g = four consecutive rows, the
    // last groups (longest causal ranges) first; a group whose rows span
    // several sequences runs once per sequence (tnd_seq), with the rows of
    // the other sequences idle
    const int g = (int)((p.q_rows + kLiRows - 1) / kLiRows) - 1 - (int)blockIdx.x;
    const int prow = g * kLiRows + wave;
    row = prow < p.q_rows ? prow : g * kLiRows;
    ri = li_row_info(p, row);
    active = prow < p.q_rows && ri.b == tnd_seq;
    const int qstart = tnd_seq > 0 ? p.act_q[tnd_seq - 1] : 0;
    rs = li_row_info(p, max(g * kLiRows, qstart));
  }
  const int lim = active ? ri.lim : 0;
  if (lane == 0) s_lim[wave] = lim;
  float* srow = p.scores + ((int64_t)row * p.n2 + kh) * p.s2;

  // weights (C-layout rows of this lane) and Q fragments (A operands)
  const int64_t wbase = (int64_t)row * p.n1 + kh * p.g;
  float wv[GT][4];
#pragma unroll
  for (int ht = 0; ht < GT; ++ht)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gg = ht * 16 + lg * 4 + r;
      const float x = li_load_w(p, wbase + (gg < p.g ? gg : 0));
      wv[ht][r] = gg < p.g ? x : 0.f;
    }
  V8 qf[GT][KS];
#pragma unroll
  for (int ht = 0; ht < GT; ++ht) {
    const int g = ht * 16 + li;
    const int64_t qrow = (int64_t)row * p.n1 + kh * p.g + (g < p.g ? g : 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 v = *(const u32x4*)((const T*)p.q + qrow * D + ks * 32 + lg * 8);
      qf[ht][ks] = as_v8<V8>(g < p.g ? v : z);
    }
  }
  lds_barrier();
  int kend = 0;
#pragma unroll
  for (int w = 0; w < kLiRows; ++w) kend = max(kend, s_lim[w]);
  // this workgroup's tiles [tb, te) of the rows' ntiles: all of them, or
  // (p.row_tiles > 0, few rows per batch) chunk blockIdx.y of row_tiles
  // tiles, so that the chunks fill the CUs; keys of the chunk past the
  // rows' visible keys are masked below
  const int ntiles = (kend + kLiRowTile - 1) / kLiRowTile;
  const int ct = p.row_tiles > 0 ? p.row_tiles : (p.s2 + kLiRowTile - 1) / kLiRowTile;
  const int tb = (int)blockIdx.y * ct;
  const int te = max(tb, min(ntiles, tb + ct));
  const int key_end = (int)min((int64_t)p.s2, (int64_t)(tb + ct) * kLiRowTile);

  // DMA j of this wave covers tile rows (j * kLiRows + wave) * RPD .. +RPD-1;
  // lane L: row + L / CPR, LDS chunk L % CPR <- source chunk (L % CPR) ^ swz
  constexpr bool paged = PG;
  const int32_t* btab = paged ? p.block_table + (int64_t)rs.b * p.max_blocks : nullptr;
  const int64_t nblk = paged ? p.k_rows / p.page_size : 0;
  // the last key a DMA loads: the rows' last visible key, kept inside the
  // key tensor (dense keys: row kbase + key <= k_rows - 1, as li_key_row
  // clamps inconsistent cumulative lengths)
  int lastkey = kend > 0 ? kend - 1 : 0;
  const int64_t kbase = rs.k_base < p.k_rows ? rs.k_base : p.k_rows - 1;
  if (!paged && kbase + lastkey > p.k_rows - 1) lastkey = (int)(p.k_rows - 1 - kbase);
  // paged keys: the table entries of every key this workgroup's DMAs load
  // (tiles tb .. te + 1, clamped to lastkey) staged in LDS where they fit
  // (kLiBtRows entries), so that a tile's DMAs wait for LDS reads rather
  // than for dependent loads of their entries from memory
  int bt0 = 0;
  bool staged = false;
  if (paged) {
    const int klo = min(tb * kLiRowTile, lastkey);
    const int khi = min(lastkey, (te + 2) * kLiRowTile - 1);
    bt0 = klo / p.page_size;
    const int ne = khi / p.page_size - bt0 + 1;
    staged = ne <= kLiBtRows;
    if (staged) {
      const int v = btab[bt0 + min((int)threadIdx.x, ne - 1)];
      if ((int)threadIdx.x < ne) s_bt[threadIdx.x] = v;
      lds_barrier();
    }
  }
  // loop-invariant per DMA: tile row, source chunk, and (dense keys) the
  // address of key 0's chunk; a key adds key * n2 * D elements
  int tr_j[NDW], ch_j[NDW];
  const T* base_j[NDW];
#pragma unroll
  for (int j = 0; j < NDW; ++j) {
    tr_j[j] = (j * kLiRows + wave) * RPD + lane / CPR;
    ch_j[j] = (lane % CPR) ^ (tr_j[j] & SWM);
    base_j[j] = (const T*)p.k + (kbase * p.n2 + kh) * D + ch_j[j] * 8;
  }
  const int64_t key_stride = (int64_t)p.n2 * D;
  auto issue_tile = [&](int t, int buf) {
#pragma unroll
    for (int j = 0; j < NDW; ++j) {
      const int d = j * kLiRows + wave;
      int key = t * kLiRowTile + tr_j[j];
      key = key < lastkey ? key : lastkey;  // past the rows' keys: reload the last one
      const T* src = base_j[j] + key * key_stride;
      if (paged) {
        int blk;
        if (staged) blk = s_bt[li_page(p, key) - bt0];
        else blk = btab[li_page(p, key)];
        const bool zero = blk < 0 || (int64_t)blk >= nblk;
        const int64_t krow = (int64_t)(zero ? 0 : blk) * p.page_size + li_in_page(p, key);
        src = zero ? (const T*)g_li_zero_row + ch_j[j] * 8 : (const T*)p.k + (krow * p.n2 + kh) * D + ch_j[j] * 8;
      }
      li_dma16((unsigned)(uintptr_t)&s_k[buf][d * 1024], src);
    }
  };
  issue_tile(tb, 0);
  issue_tile(tb + 1, 1);

  for (int t = tb; t < te; ++t) {
    const int it = t - tb;
    const int buf = it % NBUF;
    if (active) {
      if (it == 0) li_wait_vm<NDW>();
      else if (it == 1) li_wait_vm<NDW + 1>();
      else li_wait_vm<NDW + 2>();
    } else {
      li_wait_vm<NDW>();
    }
    lds_barrier();
    issue_tile(t + 2, (it + 2) % NBUF);  // into the buffer tile t-1 used
    if (!active) continue;
    const unsigned char* tb = s_k[buf];
    auto kread = [&](int kg, int ks) -> V8 {
      const int tr = kg * 16 + li;
      const int c = ks * 4 + lg;
      return as_v8<V8>(*(const u32x4*)(tb + tr * (D * 2) + ((c ^ (tr & SWM)) * 16)));
    };
    // software-pipelined over the tile's four key groups: the MFMAs of
    // group kg + 1 go out before the ReLU / weight / head sum of group kg,
    // so the wave does not wait on its own products
    float outv = -INFINITY;
    constexpr int NKG = kLiRowTile / 16;
    auto products = [&](int kg, f32x4 (&acc)[GT]) {
      V8 kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = kread(kg, ks);
#pragma unroll
      for (int ht = 0; ht < GT; ++ht) acc[ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int ht = 0; ht < GT; ++ht) acc[ht] = E::mfma(qf[ht][ks], kf[ks], acc[ht]);
    };
    auto head_sum = [&](int kg, const f32x4 (&acc)[GT]) {
      float s = 0.f;
#pragma unroll
      for (int ht = 0; ht < GT; ++ht)
#pragma unroll
        for (int r = 0; r < 4; ++r) s += relu_bits(acc[ht][r]) * wv[ht][r];
      s = xgroup_sum(s);
      const int key = t * kLiRowTile + kg * 16 + li;
      if (lg == kg) outv = key < lim ? s : -INFINITY;
    };
    f32x4 acc0[GT], acc1[GT];
    products(0, acc0);
#pragma unroll
    for (int kg = 0; kg < NKG; kg += 2) {
      products(kg + 1, acc1);
      head_sum(kg, acc0);
      if (kg + 2 < NKG) products(kg + 2, acc0);
      head_sum(kg + 1, acc1);
    }
    // lane L holds key t*64 + L; lanes past the row's end store the last
    // entry's value to the last entry (one store instruction per tile)
    const int key = t * kLiRowTile + lane;
    const int last = p.s2 - 1 - t * kLiRowTile;
    const float vlast = __shfl(outv, last < 63 ? last : 63);
    li_store_f32(srow + (key < p.s2 ? key : p.s2 - 1), key < p.s2 ? outv : vlast);
  }
  li_wait_vm<0>();
  // keys of the chunk past the tiles are masked
  if (active)
    for (int key = te * kLiRowTile + lane; key < key_end; key += 64) srow[key] = -INFINITY;
}

template <int D, typename T, int GT, bool PG>
__global__ __launch_bounds__(kLiRows * 64) void li_score_rows_kernel(LiParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char s_k[kLiRowBufs][li_row_tile_bytes<D>()];
  __shared__ int s_lim[kLiRows];
  __shared__ int s_bt[kLiBtRows];
  if (p.layout_q != DSA_LAYOUT_TND) {
    li_rows_scores<D, T, GT, PG>(p, s_k, s_lim, s_bt);
    return;
  }
  // packed rows: one pass per sequence among the group's four rows
  const int g = (int)((p.q_rows + kLiRows - 1) / kLiRows) - 1 - (int)blockIdx.x;
  const int seq0 = li_row_info(p, g * kLiRows).b;
  const int seq1 = li_row_info(p, (int)min((int64_t)g * kLiRows + kLiRows - 1, p.q_rows - 1)).b;
  for (int sq = seq0; sq <= seq1; ++sq) {
    const int qs = sq > 0 ? p.act_q[sq - 1] : 0;
    if (p.act_q[sq] == qs) continue;  // an empty sequence (uniform: same for every thread)
    __syncthreads();                  // the previous pass's LDS reads are done
    li_rows_scores<D, T, GT, PG>(p, s_k, s_lim, s_bt, sq);
  }
}

// fp32 query / key (and weights): the products run on v_mfma_f32_16x16x4f32
// in full fp32.  A lane loads 16 bytes (4 consecutive d) of a Q row and of a
// K row, as the 16-bit kernel does, and feeds them to four MFMAs, element t
// to the t-th: MFMA t of 16-column block c takes d = 16c + 4*lg + t from the
// lanes of group lg, for the A and the B operand alike, so every d of the
// block is summed once.  The G heads run in passes of 16 (Q of one head
// tile stays in registers); each pass streams the chunk's keys again and
// adds its heads' ReLU-weighted sums to the key's score.  PAD as above, for
// a head dim p.d (a multiple of 4) below D.
template <int D, bool PAD>
__global__ __launch_bounds__(kLiThreads) void li_score_f32_kernel(LiParams p) {
  constexpr int KC = D / 16;  // 16-column blocks
  const int dstride = PAD ? p.d : D;
  __shared__ __attribute__((aligned(16))) float s_sc[kLiMaxChunk];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int rn = blockIdx.x;
  const int row = rn / p.n2;
  const int kh = rn - row * p.n2;
  const LiRow ri = li_row_info(p, row);
  const int c0 = blockIdx.y * p.chunk;
  const int c1 = min(p.s2, c0 + p.chunk);
  float* srow = p.scores + (int64_t)rn * p.s2;
  if (c0 >= ri.lim) {
    for (int j = c0 + threadIdx.x; j < c1; j += kLiThreads) srow[j] = -INFINITY;
    return;
  }
  const int ngroups = (c1 - c0 + 15) >> 4;
  const int lastvis = ri.lim - 1;
  const int32_t* btab = p.layout_k == DSA_LAYOUT_PA_BSND ? p.block_table + (int64_t)ri.b * p.max_blocks : nullptr;
  const int64_t wbase = (int64_t)row * p.n1 + kh * p.g;
  const int npass = (p.g + 15) >> 4;
  for (int pass = 0; pass < npass; ++pass) {
    const int g0 = pass * 16;
    f32x4 qf[KC];
    {
      const int g = g0 + li;
      const bool gv = g < p.g;
      const float* qp = (const float*)p.q + (wbase + (gv ? g : 0)) * dstride + lg * 4;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const bool dv = gv && (!PAD || c * 16 + lg * 4 < p.d);
        qf[c] = dv ? *(const f32x4*)(qp + c * 16) : (f32x4){0.f, 0.f, 0.f, 0.f};
      }
    }
    float wv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gg = g0 + lg * 4 + r;
      wv[r] = gg < p.g ? li_load_w(p, wbase + gg) : 0.f;
    }
    auto kload = [&](int grp, f32x4 (&kf)[KC]) {
      int key = c0 + grp * 16 + li;
      key = key < lastvis ? key : lastvis;
      const int64_t krow = li_key_row(p, ri, btab, key);
      const float* kp = (const float*)p.k + (krow * p.n2 + kh) * dstride + lg * 4;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        if (!PAD || c * 16 + lg * 4 < p.d) kf[c] = *(const f32x4*)(kp + c * 16);
        else kf[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
      }
    };
    constexpr int NP = 2;
    f32x4 kf[NP][KC];
#pragma unroll
    for (int i = 0; i < NP; ++i) kload(min(wave + 4 * i, ngroups - 1), kf[i]);
    for (int grp = wave; grp < ngroups; grp += 4 * NP) {
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int gi = grp + 4 * i;
        if (gi < ngroups) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < KC; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[c][t], kf[i][c][t], acc, 0, 0, 0);
          float s = 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) s += relu_bits(acc[r]) * wv[r];
          s = xgroup_sum(s);
          const int key = c0 + gi * 16 + li;
          // the same lane owns this key in every pass: no barrier needed
          if (lg == 0 && key < c1) {
            const int j = gi * 16 + li;
            const float prev = pass ? s_sc[j] : 0.f;
            s_sc[j] = pass + 1 < npass ? prev + s : (key < ri.lim ? prev + s : -INFINITY);
          }
        }
        kload(min(gi + 4 * NP, ngroups - 1), kf[i]);
      }
    }
  }
  __syncthreads();
  li_store_chunk(p, ri, btab, s_sc, srow, c0, c1);
}

// ---------------------------------------------------------------------------
// top-k kernel
// ---------------------------------------------------------------------------
constexpr int kTopkThreads = 1024;
// 128-entry blocks of the selection sort held in registers per wave: 16
// waves x 8 blocks x 128 = 16384 entries, the largest K
constexpr int kSortBlocksPerWave = 8;
constexpr int kTopkLdsBudget = 160 * 1024;  // LDS per workgroup on gfx950

// order-preserving map fp32 -> uint32 (larger score -> larger key); -0.0
// maps to the key of +0.0, so the two tie as they compare equal
__device__ __forceinline__ unsigned sort_key(float f) {
  const unsigned u = __float_as_uint(f == 0.f ? 0.f : f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
constexpr unsigned kNegInfKey = 0x007fffffu;  // sort_key(-inf)

struct TopkParams {
  const float* scores;  // [rows, s2]
  int32_t* indices;     // [rows, k]
  void* values;         // [rows, k] in val_dtype, or null
  int64_t rows;
  int32_t s2, k, val_dtype;
  int32_t val_zero;     // values get zeros (not requested, buffer given)
  int32_t sel_cap;      // power of two >= k: entries of the LDS sort buffer
};

// General selection of one row (any score distribution): radix select of
// the K-th largest key over the whole row, ordered selection, bitonic sort.
// The fast kernel below falls back to it for rows whose keys crowd into one
// histogram bin.
template <bool IN_LDS>
__device__ void topk_row_generic(const TopkParams& p, const int64_t row, unsigned char* tk_smem) {
  unsigned long long* sel = (unsigned long long*)tk_smem;   // p.sel_cap entries
  unsigned* hist = (unsigned*)(sel + p.sel_cap);             // 256
  int* s_wsum = (int*)(hist + 256);                          // 16
  unsigned* s_misc = (unsigned*)(s_wsum + 16);               // 4
  unsigned* s_keys = s_misc + 4;                             // s2 (IN_LDS)

  const int tid = threadIdx.x;
  const float* srow = p.scores + row * (int64_t)p.s2;
  const int S = p.s2;
  auto key_at = [&](int j) -> unsigned {
    if constexpr (IN_LDS) return s_keys[j];
    return sort_key(srow[j]);
  };
  if constexpr (IN_LDS) {
    // 16-byte loads, all independent, then the scalar tail
    const int S4 = (((uintptr_t)srow & 15) == 0) ? (S >> 2) : 0;
    for (int j = tid; j < S4; j += kTopkThreads) {
      const float4 v = ((const float4*)srow)[j];
      s_keys[4 * j] = sort_key(v.x);
      s_keys[4 * j + 1] = sort_key(v.y);
      s_keys[4 * j + 2] = sort_key(v.z);
      s_keys[4 * j + 3] = sort_key(v.w);
    }
    for (int j = 4 * S4 + tid; j < S; j += kTopkThreads) s_keys[j] = sort_key(srow[j]);
    __syncthreads();
  }

  const int lane = tid & 63, wave = tid >> 6;
  constexpr int NW = kTopkThreads / 64;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;

  // number of finite (visible) entries, and their smallest and largest key
  int nv = 0;
  unsigned kmin = 0xffffffffu, kmax = 0u;
  constexpr int UN = 4;  // keys read ahead per thread (independent LDS reads in flight)
  for (int base = 0; base < S; base += UN * kTopkThreads) {
    unsigned kq[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int j = base + u * kTopkThreads + tid;
      kq[u] = j < S ? key_at(j) : 0u;
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      if (kq[u] > kNegInfKey) {
        ++nv;
        kmin = min(kmin, kq[u]);
        kmax = max(kmax, kq[u]);
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    nv += __shfl_xor(nv, o);
    kmin = min(kmin, (unsigned)__shfl_xor((int)kmin, o));
    kmax = max(kmax, (unsigned)__shfl_xor((int)kmax, o));
  }
  unsigned* s_red = s_misc + 4 + (IN_LDS ? S : 0);  // 3 * NW words after the keys
  if (lane == 0) {
    s_red[wave] = (unsigned)nv;
    s_red[NW + wave] = kmin;
    s_red[2 * NW + wave] = kmax;
  }
  __syncthreads();
  int n_valid = 0;
  kmin = 0xffffffffu;
  kmax = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    n_valid += (int)s_red[w];
    kmin = min(kmin, s_red[NW + w]);
    kmax = max(kmax, s_red[2 * NW + w]);
  }
  const int K = p.k;
  const int take = min(K, n_valid);

  // radix select: thr = take-th largest valid key; need = entries == thr to
  // take.  The bits above the highest bit in which the finite keys differ
  // are common to all of them and skipped, so the digits of the first pass
  // are spread over the bins (the sign and exponent bits of real scores are
  // nearly constant, and one hot bin would serialise the LDS atomics).
  unsigned thr = kNegInfKey;  // with take == n_valid every valid entry (> -inf) is taken
  int need = 0;
  if (take > 0 && take < n_valid) {
    const unsigned diff = kmin ^ kmax;
    int bits = diff ? 32 - __clz((int)diff) : 0;
    unsigned pmask = bits >= 32 ? 0u : ~((1u << bits) - 1u);
    unsigned prefix = kmin & pmask;
    int remaining = take;
    while (bits > 0) {
      const int width = bits < 8 ? bits : 8;
      const int shift = bits - width;
      const unsigned dmask = (1u << width) - 1u;
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      for (int base = 0; base < S; base += UN * kTopkThreads) {
        unsigned kq[UN];
#pragma unroll
        for (int u = 0; u < UN; ++u) {
          const int j = base + u * kTopkThreads + tid;
          kq[u] = j < S ? key_at(j) : 0u;
        }
#pragma unroll
        for (int u = 0; u < UN; ++u) {
          const unsigned kk = kq[u];
          const bool act = kk > kNegInfKey && (kk & pmask) == prefix;
          const unsigned d = (kk >> shift) & dmask;
          // a wave whose active lanes share one digit adds once
          const unsigned long long am = __ballot(act);
          if (am) {
            const int first = __ffsll((long long)am) - 1;
            const unsigned d0 = (unsigned)__builtin_amdgcn_readlane((int)d, first);
            const unsigned long long same = __ballot(act && d == d0);
            if (same == am) {
              if (lane == first) atomicAdd(&hist[d0], (unsigned)__popcll(am));
            } else if (act) {
              atomicAdd(&hist[d], 1u);
            }
          }
        }
      }
      __syncthreads();
      if (tid < 64) {
        // bins 255..0 in descending order: lane l owns bins 255-4l .. 252-4l
        // (bins at or above 2^width stay zero)
        unsigned c[4];
        unsigned loc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { c[i] = hist[255 - 4 * tid - i]; loc += c[i]; }
        unsigned incl = loc;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const unsigned y = __shfl_up(incl, o);
          if (tid >= o) incl += y;
        }
        unsigned run = incl - loc;  // count in bins above this lane's
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (run < (unsigned)remaining && run + c[i] >= (unsigned)remaining) {
            s_misc[0] = 255u - 4u * tid - i;  // digit of the take-th largest
            s_misc[1] = run;                  // entries in higher bins
          }
          run += c[i];
        }
      }
      __syncthreads();
      remaining -= (int)s_misc[1];
      prefix |= s_misc[0] << shift;
      pmask |= dmask << shift;
      bits -= width;
      __syncthreads();
    }
    thr = prefix;
    need = remaining;
  }

  // ordered selection, one contiguous index range per wave, 64 consecutive
  // entries per step (conflict-free LDS reads); ballots give each entry its
  // rank in index order.  Entries > thr are all taken; entries == thr only
  // while their rank among them is < need (the lowest indices).
  const int per_wave = (((S + NW - 1) / NW) + 63) / 64 * 64;
  const int w0 = min(S, wave * per_wave), w1 = min(S, w0 + per_wave);
  int cgt = 0, ceq = 0;
  for (int base = w0; base < w1; base += UN * 64) {
    unsigned kq[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int j = base + u * 64 + lane;
      kq[u] = j < w1 ? key_at(j) : 0u;
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int j = base + u * 64 + lane;
      cgt += __popcll(__ballot(j < w1 && kq[u] > thr));
      ceq += __popcll(__ballot(j < w1 && need > 0 && kq[u] == thr));
    }
  }
  int* s_cnt = (int*)(s_red + 3 * NW);  // 2 * NW words
  if (lane == 0) {
    s_cnt[wave] = cgt;
    s_cnt[NW + wave] = ceq;
  }
  __syncthreads();
  int off_gt = 0, off_eq = 0, tot_gt = 0, tot_eq = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    off_gt += w < wave ? s_cnt[w] : 0;
    off_eq += w < wave ? s_cnt[NW + w] : 0;
    tot_gt += s_cnt[w];
    tot_eq += s_cnt[NW + w];
  }
  for (int base0 = w0; base0 < w1; base0 += UN * 64) {
   unsigned kq[UN];
#pragma unroll
   for (int u = 0; u < UN; ++u) {
     const int j = base0 + u * 64 + lane;
     kq[u] = j < w1 ? key_at(j) : 0u;
   }
#pragma unroll
   for (int u = 0; u < UN; ++u) {
    const int j = base0 + u * 64 + lane;
    const unsigned kk = kq[u];
    const bool gt = j < w1 && kk > thr;
    const bool eq = j < w1 && need > 0 && kk == thr;
    const unsigned long long mg = __ballot(gt), me = __ballot(eq);
    const unsigned long long ck = ((unsigned long long)(~kk) << 32) | (unsigned)j;
    if (gt) {
      const int pos = off_gt + __popcll(mg & lt_mask);
      if (pos < take) sel[pos] = ck;
    }
    if (eq) {
      const int rank = off_eq + __popcll(me & lt_mask);
      if (rank < need && tot_gt + rank < take) sel[tot_gt + rank] = ck;
    }
    off_gt += __popcll(mg);
    off_eq += __popcll(me);
   }
  }
  const int nsel = min(take, tot_gt + min(tot_eq, need));  // == take
  int npow = 1;
  while (npow < max(nsel, 1)) npow <<= 1;
  for (int i = nsel + tid; i < npow; i += kTopkThreads) sel[i] = ~0ull;  // npow <= p.sel_cap
  __syncthreads();

  // bitonic sort ascending of sel[0, npow).  Stages with stride >= 128 go
  // through LDS (one barrier each); the stages with stride < 128 run in
  // registers: wave w holds 128-entry blocks w, w + 16, w + 32, ... (two
  // entries per lane, index base + lane and base + 64 + lane; up to
  // kSortBlocksPerWave blocks, 16384 entries) and exchanges partners with
  // lane shuffles, so most of the 66 stages of a 2048-entry sort need no
  // barrier.
  auto lds_stage = [&](int size, int stride) {
    for (int t = tid; t < (npow >> 1); t += kTopkThreads) {
      const int i = 2 * t - (t & (stride - 1));
      const int jj = i + stride;
      const bool up = (i & size) == 0;
      const unsigned long long a = sel[i], bq = sel[jj];
      if ((a > bq) == up) { sel[i] = bq; sel[jj] = a; }
    }
    __syncthreads();
  };
  if (npow < 256) {
    for (int size = 2; size <= npow; size <<= 1)
      for (int stride = size >> 1; stride > 0; stride >>= 1) lds_stage(size, stride);
  } else {
    const int nblk = npow >> 7;  // <= 16 * kSortBlocksPerWave
    unsigned long long x[kSortBlocksPerWave][2];
    auto load_blocks = [&]() {
#pragma unroll
      for (int h = 0; h < kSortBlocksPerWave; ++h) {
        const int blk = wave + 16 * h;
        if (blk < nblk) {
          x[h][0] = sel[blk * 128 + lane];
          x[h][1] = sel[blk * 128 + 64 + lane];
        }
      }
    };
    auto store_blocks = [&]() {
#pragma unroll
      for (int h = 0; h < kSortBlocksPerWave; ++h) {
        const int blk = wave + 16 * h;
        if (blk < nblk) {
          sel[blk * 128 + lane] = x[h][0];
          sel[blk * 128 + 64 + lane] = x[h][1];
        }
      }
    };
    auto reg_stages = [&](int size, int smax) {
#pragma unroll
      for (int h = 0; h < kSortBlocksPerWave; ++h) {
        const int blk = wave + 16 * h;
        if (blk >= nblk) continue;
        const int base = blk * 128;
        for (int stride = smax; stride > 0; stride >>= 1) {
          if (stride == 64) {
            const bool up = ((base + lane) & size) == 0;
            const unsigned long long a = x[h][0], bq = x[h][1];
            if ((a > bq) == up) { x[h][0] = bq; x[h][1] = a; }
          } else {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const int idx = base + 64 * e + lane;
              const unsigned long long v = x[h][e];
              const unsigned long long y = __shfl_xor(v, stride);
              const bool lower = (lane & stride) == 0;
              const bool up = (idx & size) == 0;
              x[h][e] = (lower == up) ? (v < y ? v : y) : (v > y ? v : y);
            }
          }
        }
      }
    };
    load_blocks();
    for (int size = 2; size <= 128; size <<= 1) reg_stages(size, size >> 1);
    for (int size = 256; size <= npow; size <<= 1) {
      store_blocks();
      __syncthreads();
      for (int stride = size >> 1; stride >= 128; stride >>= 1) lds_stage(size, stride);
      load_blocks();
      reg_stages(size, 64);
    }
    store_blocks();
    __syncthreads();
  }

  // outputs
  int32_t* irow = p.indices + row * (int64_t)K;
  for (int i = tid; i < K; i += kTopkThreads) {
    int idx = -1;
    float v = -INFINITY;
    if (i < nsel) {
      idx = (int)(unsigned)(sel[i] & 0xffffffffu);
      v = srow[idx];  // the score itself (keeps the sign of a zero)
    }
    irow[i] = idx;
    if (p.values) {
      const int64_t o = row * (int64_t)K + i;
      const float w = p.val_zero ? 0.f : v;
      if (p.val_dtype == DSA_DTYPE_FP32) ((float*)p.values)[o] = w;
      else if (p.val_dtype == DSA_DTYPE_BF16) ((bf16*)p.values)[o] = (bf16)w;
      else ((f16*)p.values)[o] = (f16)w;
    }
  }
}

// ---------------------------------------------------------------------------
// Fast selection, one workgroup per row of up to kFastMaxS2 scores, each
// thread holding its kFastKpt keys in registers:
//  1. n_valid, kmin and kmax of the row's finite keys.  All of them share the
//     key bits above hb = bit length of (kmin ^ kmax).
//  2. A 4096-bin histogram of the 12 key bits right below that common prefix;
//     a scan from the top bin gives every bin's start in descending order
//     and the bin b* that holds the take-th largest key.  The answer lies
//     among the keys of bins >= b* (the candidates).
//  3. Counting sort of the candidates by bin: each takes a slot in its bin's
//     range (one LDS atomic per candidate).
//  4. Within its bin, a candidate's final position is its rank by
//     (~key << 32 | index) among the bin's candidates, i.e. score
//     descending, then index ascending.  The first `take` are the answer.
// Rows with more candidates than the buffer holds, or a bin above b* with
// more than kSegCap keys (crowded keys, e.g. many equal scores), take the
// general path above.
// ---------------------------------------------------------------------------
constexpr int kFastKpt = 32;                            // keys per thread
constexpr int kFastMaxS2 = kFastKpt * kTopkThreads;     // 32768
constexpr int kFastCap = 4096;                          // candidates (>= the largest K)
constexpr int kFastBins = 4096;                         // 12-bit digits
constexpr int kSegCap = 256;                            // keys per bin ranked directly
constexpr int kTopkWaves = kTopkThreads / 64;
// LDS of the fast path: bin counts, bin starts, bin cursors, candidate and
// output buffers, misc words
constexpr size_t kFastLds = 3 * (size_t)kFastBins * 4 + 2 * (size_t)kFastCap * 8 + 64 * 4;

// Wave-wide operations on DPP lane moves (no LDS round trips).  DPP controls
// of GFX9: row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 =
// 0x143, quad_perm = 0x00..0xff, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ unsigned dpp_u32(unsigned old, unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}
// inclusive prefix sum over the 64 lanes
__device__ __forceinline__ unsigned wave_incl_scan(unsigned v) {
  v += dpp_u32<0x111>(0u, v);
  v += dpp_u32<0x112>(0u, v);
  v += dpp_u32<0x114>(0u, v);
  v += dpp_u32<0x118>(0u, v);
  v += dpp_u32<0x142, 0xa>(0u, v);
  v += dpp_u32<0x143, 0xc>(0u, v);
  return v;
}
// reductions whose result is valid in lane 63
template <typename Op>
__device__ __forceinline__ unsigned wave_reduce_to63(unsigned v, unsigned ident, Op op) {
  v = op(v, dpp_u32<0xb1>(ident, v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_u32<0x4e>(ident, v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_u32<0x141>(ident, v));  // row_half_mirror
  v = op(v, dpp_u32<0x140>(ident, v));  // row_mirror
  v = op(v, dpp_u32<0x142, 0xa>(ident, v));
  v = op(v, dpp_u32<0x143, 0xc>(ident, v));
  return v;
}

// Exclusive scan of four values per thread over the workgroup, in (thread,
// value) order; wsum: kTopkWaves words of LDS.  Contains two barriers.
__device__ __forceinline__ void block_scan4(unsigned (&v)[4], unsigned* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const unsigned loc = v[0] + v[1] + v[2] + v[3];
  const unsigned incl = wave_incl_scan(loc);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  unsigned before = 0;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) before += w < wave ? wsum[w] : 0u;
  __syncthreads();  // wsum may be rewritten after this
  unsigned run = before + incl - loc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned c = v[i];
    v[i] = run;
    run += c;
  }
}

template <bool IN_LDS>
__global__ __launch_bounds__(kTopkThreads) void li_topk_kernel(TopkParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char tk_smem[];
  const int64_t row = blockIdx.x;
  const int S = p.s2;
  if (S > kFastMaxS2) {
    topk_row_generic<IN_LDS>(p, row, tk_smem);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* srow = p.scores + row * (int64_t)S;
  const int K = p.k;
  unsigned* const hcount = (unsigned*)tk_smem;         // kFastBins
  unsigned* const hbase = hcount + kFastBins;          // kFastBins
  unsigned* const cursor = hbase + kFastBins;          // kFastBins
  unsigned long long* const cand = (unsigned long long*)(cursor + kFastBins);  // kFastCap
  unsigned long long* const outb = cand + kFastCap;    // kFastCap
  unsigned* const misc = (unsigned*)(outb + kFastCap); // 48 words
  unsigned* const wsum = misc + 48;                    // kTopkWaves

  // the row in registers, all loads in flight: 16-byte loads where the row
  // is 16-byte aligned (key u = 4q + e is entry 4 * (q * 1024 + tid) + e),
  // else entry u * 1024 + tid
  const bool vec = (((uintptr_t)srow & 15) == 0);
  auto entry = [&](int u) { return vec ? 4 * ((u >> 2) * kTopkThreads + tid) + (u & 3) : u * kTopkThreads + tid; };
  unsigned kr[kFastKpt];
  if (vec) {
#pragma unroll
    for (int q = 0; q < kFastKpt / 4; ++q) {
      const int j = 4 * (q * kTopkThreads + tid);
      float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      if (j + 3 < S) {
        v = *(const float4*)(srow + j);
      } else {
        if (j < S) v.x = srow[j];
        if (j + 1 < S) v.y = srow[j + 1];
        if (j + 2 < S) v.z = srow[j + 2];
      }
      kr[4 * q] = sort_key(v.x);
      kr[4 * q + 1] = sort_key(v.y);
      kr[4 * q + 2] = sort_key(v.z);
      kr[4 * q + 3] = sort_key(v.w);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kFastKpt; ++u) {
      const int j = u * kTopkThreads + tid;
      kr[u] = j < S ? sort_key(srow[j]) : kNegInfKey;
    }
  }
  for (int i = tid; i < kFastBins; i += kTopkThreads) hcount[i] = 0u;

  // ---- 1. count and range of the finite keys ----
  int nv = 0;
  unsigned kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int u = 0; u < kFastKpt; ++u) {
    const bool v = kr[u] > kNegInfKey;
    nv += v;
    kmin = v ? min(kmin, kr[u]) : kmin;
    kmax = v ? max(kmax, kr[u]) : kmax;
  }
  {
    const unsigned tn = wave_reduce_to63((unsigned)nv, 0u, [](unsigned a, unsigned b) { return a + b; });
    const unsigned tmin = wave_reduce_to63(kmin, 0xffffffffu, [](unsigned a, unsigned b) { return min(a, b); });
    const unsigned tmax = wave_reduce_to63(kmax, 0u, [](unsigned a, unsigned b) { return max(a, b); });
    if (lane == 63) {
      misc[wave] = tn;
      misc[kTopkWaves + wave] = tmin;
      misc[2 * kTopkWaves + wave] = tmax;
    }
  }
  __syncthreads();
  int n_valid = 0;
  kmin = 0xffffffffu;
  kmax = 0u;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) {
    n_valid += (int)misc[w];
    kmin = min(kmin, misc[kTopkWaves + w]);
    kmax = max(kmax, misc[2 * kTopkWaves + w]);
  }
  const int take = min(K, n_valid);
  const unsigned diff = kmin ^ kmax;
  const int hb = diff ? 32 - __clz((int)diff) : 0;
  const int shift = hb > 12 ? hb - 12 : 0;
  auto digit = [&](unsigned kk) { return (kk >> shift) & (unsigned)(kFastBins - 1); };

  // ---- 2. histogram, bin starts (descending), threshold bin ----
  if (take > 0) {
#pragma unroll
    for (int u = 0; u < kFastKpt; ++u)
      if (kr[u] > kNegInfKey) atomicAdd(&hcount[digit(kr[u])], 1u);
  }
  __syncthreads();  // also: misc reads done before misc is rewritten
  int ncand = 0;
  unsigned bstar = 0;
  if (take > 0) {
    // thread t owns bins 4095 - 4t - i (descending), i = 0..3
    unsigned c[4], ex[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ex[i] = c[i] = hcount[kFastBins - 1 - 4 * tid - i];
    block_scan4(ex, wsum);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = kFastBins - 1 - 4 * tid - i;
      hbase[b] = ex[i];
      cursor[b] = ex[i];
      if (ex[i] < (unsigned)take && ex[i] + c[i] >= (unsigned)take) {
        misc[0] = (unsigned)b;    // b*
        misc[1] = ex[i] + c[i];   // keys in bins >= b*
      }
    }
    if (tid == 0) misc[2] = 0u;
    __syncthreads();
    bstar = misc[0];
    ncand = (int)misc[1];
    // largest bin among the candidates' bins
    unsigned cm = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) cm = (unsigned)(kFastBins - 1 - 4 * tid - i) >= bstar ? max(cm, c[i]) : cm;
    cm = wave_reduce_to63(cm, 0u, [](unsigned a, unsigned b) { return max(a, b); });
    if (lane == 63 && cm) atomicMax(&misc[2], cm);
    __syncthreads();
    if (ncand > kFastCap || misc[2] > (unsigned)kSegCap) {
      // crowded keys: the general selection (uniform branch)
      __syncthreads();
      topk_row_generic<IN_LDS>(p, row, tk_smem);
      return;
    }

    // ---- 3. counting sort of the candidates by bin ----
    // each candidate takes a slot of its bin's range in cand from the bin's
    // cursor (the order inside a bin is arbitrary: step 4 ranks by key)
#pragma unroll
    for (int u = 0; u < kFastKpt; ++u) {
      const unsigned d = digit(kr[u]);
      if (kr[u] > kNegInfKey && d >= bstar) {
        const unsigned slot = atomicAdd(&cursor[d], 1u);
        cand[slot] = ((unsigned long long)(~kr[u]) << 32) | (unsigned)entry(u);
      }
    }
    __syncthreads();

    // ---- 4. rank within the bin ----
    for (int q = tid; q < ncand; q += kTopkThreads) {
      const unsigned long long cv = cand[q];
      const unsigned d = digit(~(unsigned)(cv >> 32));
      const int s0 = (int)hbase[d], s1 = s0 + (int)hcount[d];
      int rank = 0;
      for (int r = s0; r < s1; ++r) rank += cand[r] < cv;
      outb[s0 + rank] = cv;
    }
    __syncthreads();
  }

  // ---- outputs ----
  int32_t* irow = p.indices + row * (int64_t)K;
  const bool want_val = p.values != nullptr && !p.val_zero;
  for (int i = tid; i < K; i += kTopkThreads) {
    int idx = -1;
    float val = -INFINITY;
    if (i < take) {
      idx = (int)(unsigned)(outb[i] & 0xffffffffull);
      // the score itself (keeps the sign of a zero), read only where values
      // are requested: the load would otherwise hold the next iteration
      if (want_val) val = srow[idx];
    }
    irow[i] = idx;
    if (p.values) {
      const int64_t o = row * (int64_t)K + i;
      const float w = p.val_zero ? 0.f : val;
      if (p.val_dtype == DSA_DTYPE_FP32) ((float*)p.values)[o] = w;
      else if (p.val_dtype == DSA_DTYPE_BF16) ((bf16*)p.values)[o] = (bf16)w;
      else ((f16*)p.values)[o] = (f16)w;
    }
  }
}

// ---------------------------------------------------------------------------
// Short rows (prefill): four rows per workgroup, one per 256-thread quarter,
// with the fast selection above scaled down (2048 bins, KPT keys per thread
// for rows of up to 256 * KPT scores, K <= kQuadMaxK).  A quarter needs
// about 36 KB of LDS where the one-row kernel needs 114 KB, so a CU holds
// four rows at a time instead of one, and their barrier waits and memory
// round trips overlap.  Each bin keeps one cursor word: it starts at the
// bin's first slot and ends one past its last, so the bin's start is the
// cursor minus the count.  A selected entry's value is recovered from its
// key (the map is invertible except that -0.0 shares +0.0's key, so zero
// keys read the score itself).  Every barrier is workgroup-wide and reached
// by every thread (the four rows advance in step).  A row whose candidates
// overflow the buffer or crowd into one bin is marked, and after the four
// fast rows the whole workgroup runs the general selection on each marked
// row.
// ---------------------------------------------------------------------------
constexpr int kQuadRows = 4;
constexpr int kQuadThr = kTopkThreads / kQuadRows;  // 256 per row
constexpr int kQuadBins = 2048;
constexpr int kQuadBinBits = 11;
constexpr int kQuadBpt = kQuadBins / kQuadThr;      // bins per thread in the scan
constexpr int kQuadCap = 2560;                      // candidates per row
constexpr int kQuadCpt = kQuadCap / kQuadThr;       // candidates per thread in the rank pass
constexpr int kQuadMaxK = 2048;
constexpr int kQuadWaves = kQuadThr / 64;
constexpr size_t kQuadRowLds = 2 * (size_t)kQuadBins * 4 + (size_t)kQuadCap * 8 + 16 * 4;
constexpr size_t kQuadLds = kQuadRows * kQuadRowLds + 64;
static_assert(kQuadCap % kQuadThr == 0 && kQuadBins % kQuadThr == 0 && (1 << kQuadBinBits) == kQuadBins, "quad");

// the score of a key (inverse of sort_key; +0.0 for the zero key)
__device__ __forceinline__ float unsort_key(unsigned k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
constexpr unsigned kZeroKey = 0x80000000u;  // sort_key(+0.0) == sort_key(-0.0)

// Marked rows of a four-row workgroup: the general selection with the whole
// workgroup, one row at a time (the LDS of the fast rows is dead by then).
// Not inlined: inside the fast kernel the general path's registers would be
// allocated for the whole kernel (128 VGPRs with spills against 60); it runs
// only for rows with crowded keys.
// The parameters go by value: taking the address of the kernel's copy would
// put it in scratch and turn every pointer of the fast path into a generic
// (flat) one, whose stores also count on the LDS counter, so each LDS wait
// of the output loop would wait for the stores to complete.
__device__ __attribute__((noinline)) void topk_quad_fallback(TopkParams p, unsigned marked, unsigned char* smem) {
  for (int r = 0; r < kQuadRows; ++r) {
    if (!((marked >> r) & 1u)) continue;
    __syncthreads();
    topk_row_generic<true>(p, (int64_t)blockIdx.x * kQuadRows + r, smem);
  }
}

// The fast selection of one row by 256 threads (tq = 0 .. 255), with the
// row's buffers at qb (kQuadRowLds bytes of LDS).  Every thread of the
// workgroup calls it in step: its barriers are workgroup-wide.  Returns true
// (uniform) for a live row whose candidates overflow the buffer or crowd
// into one bin; such a row's outputs are left to the general selection.
template <int KPT>
__device__ __forceinline__ bool topk_row256(const TopkParams& p, const int64_t row, const bool live, const int tq,
                                            unsigned char* qb) {
  const int lane = tq & 63, wq = tq >> 6;
  const int S = p.s2, K = p.k;
  unsigned* const hcount = (unsigned*)qb;                          // kQuadBins
  unsigned* const cursor = hcount + kQuadBins;                     // kQuadBins
  unsigned long long* const cand = (unsigned long long*)(cursor + kQuadBins);  // kQuadCap
  unsigned* const misc = (unsigned*)(cand + kQuadCap);             // 16 words
  const float* srow = p.scores + (live ? row : 0) * (int64_t)S;

  // keys in registers: entry u * 256 + tq (coalesced over the quarter).  The
  // loads are unconditional (index clamped into the row), so all of them are
  // in flight together: under a lane condition each one was issued in its
  // own branch and waited for there.
  unsigned kr[KPT];
  {
    float kv[KPT];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int j = u * kQuadThr + tq;
      kv[u] = srow[j < S ? j : S - 1];
    }
#pragma unroll
    for (int u = 0; u < KPT; ++u) kr[u] = (live && u * kQuadThr + tq < S) ? sort_key(kv[u]) : kNegInfKey;
  }
  for (int i = tq; i < kQuadBins; i += kQuadThr) hcount[i] = 0u;

  // ---- 1. count and range of the finite keys ----
  int nv = 0;
  unsigned kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int u = 0; u < KPT; ++u) {
    const bool v = kr[u] > kNegInfKey;
    nv += v;
    kmin = v ? min(kmin, kr[u]) : kmin;
    kmax = v ? max(kmax, kr[u]) : kmax;
  }
  {
    const unsigned tn = wave_reduce_to63((unsigned)nv, 0u, [](unsigned a, unsigned b) { return a + b; });
    const unsigned tmin = wave_reduce_to63(kmin, 0xffffffffu, [](unsigned a, unsigned b) { return min(a, b); });
    const unsigned tmax = wave_reduce_to63(kmax, 0u, [](unsigned a, unsigned b) { return max(a, b); });
    if (lane == 63) {
      misc[wq] = tn;
      misc[4 + wq] = tmin;
      misc[8 + wq] = tmax;
    }
  }
  __syncthreads();
  int n_valid = 0;
  kmin = 0xffffffffu;
  kmax = 0u;
#pragma unroll
  for (int w = 0; w < kQuadWaves; ++w) {
    n_valid += (int)misc[w];
    kmin = min(kmin, misc[4 + w]);
    kmax = max(kmax, misc[8 + w]);
  }
  const int take = min(K, n_valid);
  const unsigned diff = kmin ^ kmax;
  const int hb = diff ? 32 - __clz((int)diff) : 0;
  const int shift = hb > kQuadBinBits ? hb - kQuadBinBits : 0;
  auto digit = [&](unsigned kk) { return (kk >> shift) & (unsigned)(kQuadBins - 1); };

  // ---- 2. histogram, bin starts (descending), threshold bin ----
  if (take > 0) {
#pragma unroll
    for (int u = 0; u < KPT; ++u)
      if (kr[u] > kNegInfKey) atomicAdd(&hcount[digit(kr[u])], 1u);
  }
  __syncthreads();  // also: the misc reads are done before misc is rewritten
  // thread tq owns bins kQuadBins - 1 - kQuadBpt * tq - i (descending)
  unsigned c[kQuadBpt], ex[kQuadBpt];
  unsigned loc = 0;
#pragma unroll
  for (int i = 0; i < kQuadBpt; ++i) {
    c[i] = hcount[kQuadBins - 1 - kQuadBpt * tq - i];
    loc += c[i];
  }
  const unsigned incl = wave_incl_scan(loc);
  if (lane == 63) misc[12 + wq] = incl;
  __syncthreads();
  {
    unsigned run = incl - loc;
#pragma unroll
    for (int w = 0; w < kQuadWaves; ++w) run += w < wq ? misc[12 + w] : 0u;
#pragma unroll
    for (int i = 0; i < kQuadBpt; ++i) {
      ex[i] = run;
      run += c[i];
    }
  }
  __syncthreads();  // the wave totals are read before misc is rewritten
#pragma unroll
  for (int i = 0; i < kQuadBpt; ++i) {
    const int b = kQuadBins - 1 - kQuadBpt * tq - i;
    cursor[b] = ex[i];
    if (take > 0 && ex[i] < (unsigned)take && ex[i] + c[i] >= (unsigned)take) {
      misc[0] = (unsigned)b;    // b*
      misc[1] = ex[i] + c[i];   // keys in bins >= b*
    }
  }
  if (tq == 0) misc[2] = 0u;
  __syncthreads();
  const unsigned bstar = take > 0 ? misc[0] : 0u;
  const int ncand = take > 0 ? (int)misc[1] : 0;
  {
    unsigned cm = 0;
#pragma unroll
    for (int i = 0; i < kQuadBpt; ++i) cm = (unsigned)(kQuadBins - 1 - kQuadBpt * tq - i) >= bstar ? max(cm, c[i]) : cm;
    cm = wave_reduce_to63(cm, 0u, [](unsigned a, unsigned b) { return max(a, b); });
    if (lane == 63 && cm && take > 0) atomicMax(&misc[2], cm);
  }
  __syncthreads();
  const bool fallback = live && take > 0 && (ncand > kQuadCap || misc[2] > (unsigned)kSegCap);
  const bool fast = live && !fallback;

  // ---- 3. counting sort of the candidates by bin: every cursor atomic of a
  // thread first, then its candidate writes ----
  if (fast && take > 0) {
    unsigned slot[KPT];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const bool is_c = kr[u] > kNegInfKey && digit(kr[u]) >= bstar;
      slot[u] = is_c ? atomicAdd(&cursor[digit(kr[u])], 1u) : 0xffffffffu;
    }
#pragma unroll
    for (int u = 0; u < KPT; ++u)
      if (slot[u] != 0xffffffffu) cand[slot[u]] = ((unsigned long long)(~kr[u]) << 32) | (unsigned)(u * kQuadThr + tq);
  }
  __syncthreads();

  // ---- 4. rank within the bin (bin start = cursor - count), then outputs ----
  int32_t* irow = p.indices + (live ? row : 0) * (int64_t)K;
  auto put = [&](int i, int idx, float val) {
    irow[i] = idx;
    if (p.values) {
      const int64_t o = row * (int64_t)K + i;
      const float w = p.val_zero ? 0.f : val;
      if (p.val_dtype == DSA_DTYPE_FP32) ((float*)p.values)[o] = w;
      else if (p.val_dtype == DSA_DTYPE_BF16) ((bf16*)p.values)[o] = (bf16)w;
      else ((f16*)p.values)[o] = (f16)w;
    }
  };
  if (fast) {
    // the thread's candidates q = i * 256 + tq; each is ranked against its
    // bin's entries, four reads in flight per step (the reads of a step past
    // the bin's end are clamped into it and not counted)
    unsigned long long cv_r[kQuadCpt];
    int s0_r[kQuadCpt], rank_r[kQuadCpt];
#pragma unroll
    for (int i = 0; i < kQuadCpt; ++i) cv_r[i] = cand[min(i * kQuadThr + tq, kQuadCap - 1)];
#pragma unroll
    for (int i = 0; i < kQuadCpt; ++i) {
      rank_r[i] = 0;
      s0_r[i] = 0;
      if (i * kQuadThr + tq < ncand) {
        const unsigned long long cv = cv_r[i];
        const unsigned d = digit(~(unsigned)(cv >> 32));
        const int nb = (int)hcount[d];
        const int s0 = (int)cursor[d] - nb;
        int rank = 0;
        for (int r = 0; r < nb; r += 4) {
          unsigned long long e[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) e[j] = cand[s0 + min(r + j, nb - 1)];
#pragma unroll
          for (int j = 0; j < 4; ++j) rank += (r + j < nb && e[j] < cv) ? 1 : 0;
        }
        s0_r[i] = s0;
        rank_r[i] = rank;
      }
    }
    int pos_r[kQuadCpt];
#pragma unroll
    for (int i = 0; i < kQuadCpt; ++i) pos_r[i] = i * kQuadThr + tq < ncand ? s0_r[i] + rank_r[i] : -1;
#pragma unroll
    for (int i = 0; i < kQuadCpt; ++i) {
      if (pos_r[i] >= 0 && pos_r[i] < take) {
        const unsigned key = ~(unsigned)(cv_r[i] >> 32);
        const int idx = (int)(unsigned)(cv_r[i] & 0xffffffffull);
        put(pos_r[i], idx, key == kZeroKey ? srow[idx] : unsort_key(key));
      }
    }
    for (int i = take + tq; i < K; i += kQuadThr) put(i, -1, -INFINITY);
  }
  return fallback;
}

template <int KPT>
__global__ __launch_bounds__(kTopkThreads) void li_topk_quad_kernel(TopkParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char tk_smem[];
  const int tid = threadIdx.x;
  const int q = tid / kQuadThr, tq = tid - q * kQuadThr;  // quarter, thread in it
  const int64_t row = (int64_t)blockIdx.x * kQuadRows + q;
  unsigned* const flags = (unsigned*)(tk_smem + kQuadRows * kQuadRowLds);  // kQuadRows
  if (tid < kQuadRows) flags[tid] = 0u;  // ordered before the writes below by the row's barriers
  const bool fallback = topk_row256<KPT>(p, row, row < p.rows, tq, tk_smem + q * kQuadRowLds);
  if (fallback && tq == 0) flags[q] = 1u;
  __syncthreads();
  const unsigned marked = flags[0] | (flags[1] << 1) | (flags[2] << 2) | (flags[3] << 3);
  if (marked) topk_quad_fallback(p, marked, tk_smem);  // uniform
}

// ---------------------------------------------------------------------------
// Scores and top-k in one launch (BSND rows sharing key tiles, many rows):
// after its score rows, the workgroup selects their top-k itself, one row at
// a time with all 256 threads and the fast selection above, its buffers in
// the idle key-tile ring.  The rows' scores were written by this workgroup
// (through its CU's L2) just before, and the selection of one workgroup
// overlaps the score products of the CU's other workgroups, where the two
// launches ran the products and the selections one after the other with
// the score rows going through memory in between.  A row that needs the
// general selection gets kTopkMark as its first index, and
// li_topk_marked_kernel finishes it.
// ---------------------------------------------------------------------------
constexpr int32_t kTopkMark = -2147483647 - 1;  // below every index (-1 pads)

template <int D, typename T, int GT, int KPT, bool PG>
__global__ __launch_bounds__(kLiRows * 64) void li_score_rows_topk_kernel(LiParams p, TopkParams tp) {
  constexpr int TB = li_row_tile_bytes<D>();
  static_assert(kLiRowBufs * TB >= (int)kQuadRowLds, "one row's selection buffers fit the tile ring");
  __shared__ __attribute__((aligned(1024))) unsigned char s_k[kLiRowBufs][TB];
  __shared__ int s_lim[kLiRows];
  __shared__ int s_bt[kLiBtRows];
  li_rows_scores<D, T, GT, PG>(p, s_k, s_lim, s_bt);
  // the workgroup's rows, as li_rows_scores maps them
  const int nbk = p.batch * p.n2;
  const int ngroups = (p.s1 + kLiRows - 1) / kLiRows;
  const int bk = blockIdx.x % nbk;
  const int grp = ngroups - 1 - (int)(blockIdx.x / nbk);
  const int b = bk / p.n2, kh = bk - b * p.n2;
  // every score store of the workgroup is complete and visible before any
  // thread reads a row back (workgroup-scope release / acquire)
  __syncthreads();
  for (int r = 0; r < kLiRows; ++r) {
    const int s1r = grp * kLiRows + r;
    const bool live = s1r < p.s1;
    const int64_t srn = (int64_t)(b * p.s1 + (live ? s1r : 0)) * p.n2 + kh;
    if (r > 0) __syncthreads();  // the previous row's buffers are read
    const bool fb = topk_row256<KPT>(tp, srn, live, (int)threadIdx.x, &s_k[0][0]);
    if (fb && threadIdx.x == 0) tp.indices[srn * tp.k] = kTopkMark;
  }
}

// Rows the fused launch left to the general selection: a workgroup checks
// 64 rows' first indices and runs the general selection (whole workgroup,
// the row in LDS) on each marked one.
__global__ __launch_bounds__(kTopkThreads) void li_topk_marked_kernel(TopkParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char tk_smem[];
  __shared__ unsigned s_mark[2];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  if (threadIdx.x < 64) {
    const int64_t row = r0 + threadIdx.x;
    const bool m = row < p.rows && p.indices[row * p.k] == kTopkMark;
    const unsigned long long bal = __ballot(m);
    if (threadIdx.x == 0) {
      s_mark[0] = (unsigned)bal;
      s_mark[1] = (unsigned)(bal >> 32);
    }
  }
  __syncthreads();
  unsigned long long marked = (unsigned long long)s_mark[0] | ((unsigned long long)s_mark[1] << 32);
  while (marked) {  // uniform
    const int i = __builtin_ctzll(marked);
    marked &= marked - 1ull;
    __syncthreads();
    topk_row_generic<true>(p, r0 + i, tk_smem);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int64_t pow2_at_least(int64_t x) {
  int64_t n = 1;
  while (n < x) n <<= 1;
  return n;
}

// LDS bytes of li_topk_kernel: sort buffer, histogram, scan and misc words,
// and (rows kept in LDS) the row's keys
static size_t li_topk_fixed_bytes(int64_t k) {
  // sort buffer, histogram, scan words, misc words, reduction + count words
  return (size_t)pow2_at_least(k) * 8 + 256 * 4 + 16 * 4 + 4 * 4 + 5 * (kTopkThreads / 64) * 4;
}
static bool li_topk_row_in_lds(int64_t s2, int64_t k) {
  return li_topk_fixed_bytes(k) + (size_t)s2 * 4 <= (size_t)kTopkLdsBudget;
}

static TopkParams topk_params(const float* scores, int64_t rows, int64_t s2, int64_t k, int32_t* indices,
                              void* values, int32_t val_dtype, bool values_zero) {
  TopkParams p;
  p.scores = scores;
  p.indices = indices;
  p.values = values;
  p.val_zero = values_zero ? 1 : 0;
  p.rows = rows;
  p.s2 = (int32_t)s2;
  p.k = (int32_t)k;
  p.val_dtype = val_dtype;
  p.sel_cap = (int32_t)pow2_at_least(k);
  return p;
}

// Many short rows go four to a workgroup (li_topk_quad_kernel); the general
// path of a marked row then runs in the same LDS, so it must fit there with
// the row kept in LDS.
static bool li_topk_quad_fits(int64_t rows, int64_t s2, int64_t k) {
  return rows > (int64_t)device_cu_count() && s2 <= 32 * kQuadThr && k <= kQuadMaxK &&
         li_topk_fixed_bytes(k) + (size_t)s2 * 4 <= (size_t)kQuadRows * kQuadRowLds;
}

int li_topk_run(const float* scores, int64_t rows, int64_t s2, int64_t k, int32_t* indices,
                void* values, int32_t val_dtype, hipStream_t stream, bool values_zero) {
  if (rows <= 0) return DSA_OK;
  TopkParams p = topk_params(scores, rows, s2, k, indices, values, val_dtype, values_zero);
  // dynamic LDS above 64 KB needs the per-function limit raised (to the
  // full budget; set on every call, which also covers every device and
  // concurrent callers: a host-side setting, cheap next to the launch)
  // many short rows: four per workgroup
  if (li_topk_quad_fits(rows, s2, k)) {
    const void* fq = s2 <= 8 * kQuadThr    ? (const void*)li_topk_quad_kernel<8>
                     : s2 <= 16 * kQuadThr ? (const void*)li_topk_quad_kernel<16>
                                           : (const void*)li_topk_quad_kernel<32>;
    DSA_HIP(hipFuncSetAttribute(fq, hipFuncAttributeMaxDynamicSharedMemorySize, kTopkLdsBudget));
    void* args[] = {&p};
    DSA_HIP(hipLaunchKernel(fq, dim3((unsigned)((rows + kQuadRows - 1) / kQuadRows)), dim3(kTopkThreads), args,
                            kQuadLds, stream));
    return DSA_OK;
  }
  const bool in_lds = li_topk_row_in_lds(s2, k);
  size_t lds = li_topk_fixed_bytes(k) + (in_lds ? (size_t)s2 * 4 : 0);  // general path
  if (lds < kFastLds) lds = kFastLds;
  const void* fn = in_lds ? (const void*)li_topk_kernel<true> : (const void*)li_topk_kernel<false>;
  DSA_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kTopkLdsBudget));
  if (in_lds)
    hipLaunchKernelGGL(li_topk_kernel<true>, dim3((unsigned)rows), dim3(kTopkThreads), lds, stream, p);
  else
    hipLaunchKernelGGL(li_topk_kernel<false>, dim3((unsigned)rows), dim3(kTopkThreads), lds, stream, p);
  DSA_HIP(hipGetLastError());
  return DSA_OK;
}

// Keys per workgroup: enough chunks per row that the grid puts one
// workgroup on every CU, in one round.  Two resident workgroups per CU
// measured slower: they start together, but one streams ahead while the
// other waits behind it, so the grid ran as two serial rounds with a long
// tail (decode step 72.5 -> 66.6 us with one per CU).
// Largest chunk (a multiple of 64 keys) whose key loads, 16-key groups
// included, stay within the kLiBtStage staged table entries.
static int64_t li_paged_chunk_cap(int64_t page) {
  const int64_t cap = ((kLiBtStage - 3) * page / 64) * 64;
  return cap < 64 ? 64 : cap;
}

static hipError_t launch_score_kernel(const void* fn, LiParams p, hipStream_t stream) {
  const int64_t rows = p.q_rows * p.n2;
  const int64_t target = (int64_t)device_cu_count();
  const int64_t per_row = rows >= target ? 1 : (target + rows - 1) / rows;
  int64_t chunk = (p.s2 + per_row - 1) / per_row;
  chunk = ((chunk + 63) / 64) * 64;
  chunk = chunk < 64 ? 64 : chunk;
  p.chunk = (int32_t)(chunk > kLiMaxChunk ? kLiMaxChunk : chunk);
  if (p.layout_k == DSA_LAYOUT_PA_BSND) p.chunk = (int32_t)std::min<int64_t>(p.chunk, li_paged_chunk_cap(p.page_size));
  const unsigned chunks = (unsigned)((p.s2 + p.chunk - 1) / p.chunk);
  void* args[] = {&p};
  return hipLaunchKernel(fn, dim3((unsigned)rows, chunks), dim3(kLiThreads), args, 0, stream);
}

template <int D, typename T, int GT, bool PAD>
static hipError_t launch_score(const LiParams& p, hipStream_t stream) {
  // one query row per batch: no key is read twice (exact head dims only)
  if (!PAD && p.q_rows == p.batch)
    return launch_score_kernel((const void*)li_score_kernel<D, T, GT, false, true>, p, stream);
  // three or more query rows per batch (BSND): rows share key tiles through
  // LDS, while the row's Q fragments fit the registers (GT * D / 32 <= 16);
  // at three rows one of the four waves idles (multi-token decode S1 = 3 at
  // B = 32: 140 us with the one-row kernel, 84 us here)
  if constexpr (!PAD && GT * (D / 32) <= 16) {
    // packed (TND) queries with one key head and three or more rows per
    // sequence on average: groups of four consecutive rows, a group that
    // spans sequences running once per sequence
    const bool tnd_rows = p.layout_q == DSA_LAYOUT_TND && p.n2 == 1 && p.q_rows >= 3 * (int64_t)p.batch;
    if ((p.layout_q == DSA_LAYOUT_BSND && p.s1 >= 3) || tnd_rows) {
      LiParams q = p;
      const unsigned grid = tnd_rows ? (unsigned)((p.q_rows + kLiRows - 1) / kLiRows)
                                     : (unsigned)((int64_t)p.batch * p.n2 * ((p.s1 + kLiRows - 1) / kLiRows));
      // few query rows per batch (multi-token decode): the rows' keys split
      // into chunks of at least 8 tiles, so that about two workgroups per CU
      // run (one workgroup per row group left most CUs idle)
      const int64_t want = 2 * (int64_t)device_cu_count();
      const int tiles = (p.s2 + kLiRowTile - 1) / kLiRowTile;
      unsigned chunks = 1;
      if ((int64_t)grid < want) {
        const int64_t c = (want + grid - 1) / grid;
        q.row_tiles = (int32_t)std::max<int64_t>(8, (tiles + c - 1) / c);
        chunks = (unsigned)((tiles + q.row_tiles - 1) / q.row_tiles);
        if (chunks <= 1) q.row_tiles = 0;
      }
      void* args[] = {&q};
      const void* fn = p.layout_k == DSA_LAYOUT_PA_BSND ? (const void*)li_score_rows_kernel<D, T, GT, true>
                                                        : (const void*)li_score_rows_kernel<D, T, GT, false>;
      return hipLaunchKernel(fn, dim3(grid, chunks), dim3(kLiRows * 64),
                             args, 0, stream);
    }
  }
  // two query rows per batch (BSND, one key head): one workgroup per
  // batch and key chunk runs both rows on each loaded key fragment, the
  // chunk sized so that the grid puts one workgroup on every CU
  if constexpr (!PAD && GT * (D / 32) <= 16) {
    if (p.layout_q == DSA_LAYOUT_BSND && p.n2 == 1 && p.s1 == 2 && !(test_flags() & kTestLiNoPair)) {
      LiParams q = p;
      const int64_t pairs = p.q_rows / 2;
      const int64_t target = (int64_t)device_cu_count();
      const int64_t per = pairs >= target ? 1 : (target + pairs - 1) / pairs;
      int64_t chunk = (p.s2 + per - 1) / per;
      chunk = ((chunk + 63) / 64) * 64;
      chunk = chunk < 64 ? 64 : chunk;
      q.chunk = (int32_t)(chunk > kLiPairMaxChunk ? kLiPairMaxChunk : chunk);
      if (p.layout_k == DSA_LAYOUT_PA_BSND) q.chunk = (int32_t)std::min<int64_t>(q.chunk, li_paged_chunk_cap(p.page_size));
      const unsigned chunks = (unsigned)((p.s2 + q.chunk - 1) / q.chunk);
      void* args[] = {&q};
      return hipLaunchKernel((const void*)li_score_pair_kernel<D, T, GT, kLiPairRing>, dim3((unsigned)pairs, chunks),
                             dim3(kLiThreads), args, 0, stream);
    }
  }
  // a few query rows per batch (BSND, one key head): a batch's rows on one
  // XCD, where the second and later reads of its keys hit in L2
  LiParams q = p;
  if (p.layout_q == DSA_LAYOUT_BSND && p.n2 == 1 && p.s1 > 1 && p.q_rows % (8 * (int64_t)p.s1) == 0)
    q.xcd_group = p.s1;
  return launch_score_kernel((const void*)li_score_kernel<D, T, GT, PAD, false>, q, stream);
}

template <int D, typename T, bool PAD>
static hipError_t launch_score_g(const LiParams& p, hipStream_t stream) {
  if (p.g <= 16) return launch_score<D, T, 1, PAD>(p, stream);
  if (p.g <= 32) return launch_score<D, T, 2, PAD>(p, stream);
  if (p.g <= 64) return launch_score<D, T, 4, PAD>(p, stream);
  return launch_score<D, T, 8, PAD>(p, stream);
}

template <int D, bool PAD>
static hipError_t launch_score_f32(const LiParams& p, hipStream_t stream) {
  return launch_score_kernel((const void*)li_score_f32_kernel<D, PAD>, p, stream);
}

// Head dims 64 / 128 / 256 run exact kernels; any other supported head dim
// (a multiple of 8 up to 256; of 4 for fp32) runs the next larger one with
// zero-padded rows.
template <typename T>
static hipError_t launch_score_d(const LiParams& p, int64_t d, hipStream_t stream) {
  if constexpr (__is_same(T, float)) {
    if (d == 64) return launch_score_f32<64, false>(p, stream);
    if (d == 128) return launch_score_f32<128, false>(p, stream);
    if (d == 256) return launch_score_f32<256, false>(p, stream);
    if (d < 64) return launch_score_f32<64, true>(p, stream);
    if (d < 128) return launch_score_f32<128, true>(p, stream);
    return launch_score_f32<256, true>(p, stream);
  } else {
    if (d == 64) return launch_score_g<64, T, false>(p, stream);
    if (d == 128) return launch_score_g<128, T, false>(p, stream);
    if (d == 256) return launch_score_g<256, T, false>(p, stream);
    if (d < 64) return launch_score_g<64, T, true>(p, stream);
    if (d < 128) return launch_score_g<128, T, true>(p, stream);
    return launch_score_g<256, T, true>(p, stream);
  }
}

static LiParams li_params(const void* query, const void* key, const void* weights, const int32_t* act_q,
                          const int32_t* act_k, float* scores, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                          int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows, int32_t sparse_mode,
                          int32_t layout_q, int32_t layout_k, int32_t w_dtype, const int32_t* block_table,
                          int64_t max_blocks, int64_t page_size);

int li_scores_run(const void* query, const void* key, const void* weights, const int32_t* act_q,
                  const int32_t* act_k, float* scores, int64_t batch, int64_t s1, int64_t s2,
                  int64_t n1, int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows,
                  int32_t sparse_mode, int32_t layout_q, int32_t layout_k, int32_t dtype,
                  int32_t w_dtype, hipStream_t stream, const int32_t* block_table,
                  int64_t max_blocks, int64_t page_size) {
  if (q_rows <= 0 || s2 <= 0) return DSA_OK;
  const LiParams p = li_params(query, key, weights, act_q, act_k, scores, batch, s1, s2, n1, n2, d, q_rows, k_rows,
                               sparse_mode, layout_q, layout_k, w_dtype, block_table, max_blocks, page_size);
  hipError_t e = dtype == DSA_DTYPE_BF16   ? launch_score_d<bf16>(p, d, stream)
                 : dtype == DSA_DTYPE_FP16 ? launch_score_d<f16>(p, d, stream)
                                           : launch_score_d<float>(p, d, stream);
  DSA_HIP(e);
  return DSA_OK;
}

static LiParams li_params(const void* query, const void* key, const void* weights, const int32_t* act_q,
                          const int32_t* act_k, float* scores, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                          int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows, int32_t sparse_mode,
                          int32_t layout_q, int32_t layout_k, int32_t w_dtype, const int32_t* block_table,
                          int64_t max_blocks, int64_t page_size) {
  LiParams p;
  p.q = query;
  p.k = key;
  p.w = weights;
  p.act_q = act_q;
  p.act_k = act_k;
  p.scores = scores;
  p.q_rows = q_rows;
  p.k_rows = k_rows;
  p.batch = (int32_t)batch;
  p.s1 = (int32_t)s1;
  p.s2 = (int32_t)s2;
  p.n1 = (int32_t)n1;
  p.n2 = (int32_t)n2;
  p.g = (int32_t)(n1 / n2);
  p.mode = sparse_mode;
  p.layout_q = layout_q;
  p.layout_k = layout_k;
  p.w_dtype = w_dtype;
  p.block_table = block_table;
  p.max_blocks = (int32_t)max_blocks;
  p.page_size = (int32_t)(page_size > 0 ? page_size : 1);
  p.page_shift = (p.page_size & (p.page_size - 1)) == 0 ? __builtin_ctz((unsigned)p.page_size) : -1;
  p.chunk = kLiChunk;
  p.row_tiles = 0;
  p.xcd_group = 0;
  p.d = (int32_t)d;
  return p;
}

// The fused launch: exact head dim 128, 16-bit inputs, G = 33 .. 64 heads per
// key head (the DSA indexer's 64), BSND query rows sharing key tiles (as
// launch_score picks li_score_rows_kernel), rows that the top-k would give
// four to a workgroup and enough of them that the workgroups fill the CUs
// several times over.
template <typename T, int KPT>
static hipError_t launch_fused(const LiParams& p, const TopkParams& tp, hipStream_t stream) {
  LiParams q = p;
  TopkParams t = tp;
  const unsigned grid = (unsigned)((int64_t)p.batch * p.n2 * ((p.s1 + kLiRows - 1) / kLiRows));
  void* args[] = {&q, &t};
  const void* fn = p.layout_k == DSA_LAYOUT_PA_BSND ? (const void*)li_score_rows_topk_kernel<128, T, 4, KPT, true>
                                                    : (const void*)li_score_rows_topk_kernel<128, T, 4, KPT, false>;
  return hipLaunchKernel(fn, dim3(grid), dim3(kLiRows * 64), args, 0, stream);
}

int li_fwd_run(const void* query, const void* key, const void* weights, const int32_t* act_q,
               const int32_t* act_k, float* scores, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
               int64_t n2, int64_t d, int64_t q_rows, int64_t k_rows, int32_t sparse_mode, int32_t layout_q,
               int32_t layout_k, int32_t dtype, int32_t w_dtype, int64_t k, int32_t* indices, void* values,
               hipStream_t stream, const int32_t* block_table, int64_t max_blocks, int64_t page_size,
               bool values_zero) {
  const int64_t rows = q_rows * n2;
  const int64_t g = n2 > 0 ? n1 / n2 : 0;
  const bool fuse = q_rows > 0 && s2 > 0 && (dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_FP16) && d == 128 &&
                    g > 32 && g <= 64 && layout_q == DSA_LAYOUT_BSND && s1 >= 4 && q_rows != batch &&
                    rows >= 4 * (int64_t)device_cu_count() && s2 <= 16 * kQuadThr && li_topk_quad_fits(rows, s2, k) &&
                    !(test_flags() & kTestLiUnfused);
  if (!fuse) {
    int st = li_scores_run(query, key, weights, act_q, act_k, scores, batch, s1, s2, n1, n2, d, q_rows, k_rows,
                           sparse_mode, layout_q, layout_k, dtype, w_dtype, stream, block_table, max_blocks,
                           page_size);
    if (st != DSA_OK) return st;
    return li_topk_run(scores, rows, s2, k, indices, values, dtype, stream, values_zero);
  }
  const LiParams p = li_params(query, key, weights, act_q, act_k, scores, batch, s1, s2, n1, n2, d, q_rows, k_rows,
                               sparse_mode, layout_q, layout_k, w_dtype, block_table, max_blocks, page_size);
  const TopkParams tp = topk_params(scores, rows, s2, k, indices, values, dtype, values_zero);
  const bool bf = dtype == DSA_DTYPE_BF16;
  // rows of up to 4096 scores (16 per thread: 158 VGPRs, three workgroups per
  // CU as the score kernel alone; 32 per thread took 224 and two)
  hipError_t e = s2 <= 8 * kQuadThr ? (bf ? launch_fused<bf16, 8>(p, tp, stream) : launch_fused<f16, 8>(p, tp, stream))
                                    : (bf ? launch_fused<bf16, 16>(p, tp, stream) : launch_fused<f16, 16>(p, tp, stream));
  DSA_HIP(e);
  // the rows marked for the general selection (the row kept in LDS)
  const size_t lds = li_topk_fixed_bytes(k) + (size_t)s2 * 4;
  DSA_HIP(hipFuncSetAttribute((const void*)li_topk_marked_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds));
  hipLaunchKernelGGL(li_topk_marked_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(kTopkThreads), lds, stream, tp);
  DSA_HIP(hipGetLastError());
  return DSA_OK;
}

}  // namespace dsa
