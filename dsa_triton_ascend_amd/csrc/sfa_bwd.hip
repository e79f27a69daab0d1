// Sparse flash attention backward for gfx950 (MLA-absorb, MQA).
//
// Semantics follow the reference kernel `_sfa_grad_kernel`
// (sparse_flash_attention_grad_triton.py:158-308) and its golden
// (sparse_flash_attention_grad_numpy.py:34-143).  For every active query row
// and every attended token (the forward's masks), with v = key[:, :D]:
//   s     = (q_nope.k_nope + q_rope.k_rope) * scale
//   P     = exp(s - softmax_max) / softmax_sum   (sum <= 0 taken as 1, 233-234)
//   delta = sum_d dO * O                          (237)
//   dS    = P * (dP - delta) * scale, dP = dO.v   (262-267)
//   dq += dS k_nope,  dq_rope += dS k_rope        (271-272)
//   dk += dS^T q_nope, dk_rope += dS^T q_rope, dv += P^T dO   (277-300)
// The reference scatters dk / dk_rope / dv with fp32 atomics, so its results
// depend on the order of the additions (and it rejects deterministic=True).
// Here every output is deterministic and no floating-point atomics are used:
//
//  A. sfa_bwd_dq_kernel: one workgroup per (query row, 64 heads), 4 waves of
//     16 heads.  Tiles of 32 attended tokens are gathered into LDS by
//     LDS-DMA; S^T = K.Q^T and dP^T = V.dO^T share the K fragment reads; P
//     and dS are lane-local and go through an LDS tile; dq^T += K^T.dS^T is
//     split by column slice (each wave all 64 heads over a quarter of the
//     columns, both operands through the transposing LDS read).  dS and P
//     of the tile are stored ([row][slot][dS | P][head]) for
//     kernel B, and the row's compacted token list is recorded together with
//     each slot's rank in its token's bucket (an integer count).
//  B. sfa_bwd_rec_kernel: one workgroup per query row, all heads (8 waves).
//     Each wave owns a slice of the output columns [dK | dK_rope | dV] (or
//     [dK + dV | dK_rope] for the shared latent) and holds Q^T / dO^T for all
//     heads of its slice as MFMA A operands; per tile it reads dS / P from
//     LDS and produces, per attended token, the head-summed contribution
//     ("record") of its columns.  Records go to the token's bucket as fp16
//     scaled by a power of two per (record, slice), so the stored values
//     keep 11 bits relative to the slice's largest entry.
//  C. sfa_bwd_reduce_kernel: one wave per (key token, slice) sums the
//     token's records in fixed point (integer-valued doubles below 2^52:
//     exact and associative, so the bucket order does not matter) and
//     writes the key gradients.
// Rows are processed in chunks whose workspace stays within a budget; the
// chunks' sums are added in chunk order in fp32.
#include <atomic>
#include <type_traits>

#include "sfa_common.h"

namespace dsa {

struct SfaBwdParams {
  const void* q;
  const void* qr;
  const void* k;
  const void* kr;
  const int32_t* idx;
  const void* dout;
  const void* out;
  const float* smax;
  const float* ssum;
  const int32_t* act_q;
  const int32_t* act_k;
  const int32_t* block_table;  // unused (no paged layout in the backward)
  void* dq;
  void* dqr;
  // outputs of the key side (kernel C)
  void* dk;
  void* dkr;
  void* dv;  // nullptr: dk receives dk + dv
  int64_t rows, kv_rows;
  int64_t row0;    // first row of the chunk
  int32_t nrows;   // rows of the chunk
  int32_t batch, s1, s2, n1, K, bs, mode, layout_q, layout_kv, max_blocks, page_size;
  int64_t band_pre, band_next;  // pre_tokens / next_tokens clamped to +-kBandOpen
  int32_t hp;      // heads padded to a multiple of 32 (dS / P row stride)
  int32_t kposp;   // index positions per row, padded to a multiple of 32
  int32_t nc;      // record columns: 2D + 64, or D + 64 when merged
  float scale, scale_log2;
  // workspace
  int32_t* cnt;    // [kv_rows] slots per token in this chunk
  int32_t* offs;   // [kv_rows + 1] bucket offsets
  int32_t* list;   // [nrows, kposp] physical token of each compacted slot
  int32_t* rank;   // [nrows, kposp] the slot's place in its token's bucket
  int32_t* nval;   // [nrows] compacted slots per row
  void* dsp;       // [nrows, kposp, 2, hp] dS and P (T; fp16 scaled by 2^kF16Shift)
  _Float16* rec;   // [slots, nc] records in bucket order
  int16_t* rexp;   // [slots, kRecSlices] exponent of each record slice
  float* acc;      // [kv_rows, nc] running fp32 sums over chunks
};

constexpr int kBwdTile = 32;
constexpr int kBwdList = 2048;  // positions resolved per compaction round
constexpr int kBwdWaves = 4;    // kernel A
constexpr int kBwdHeads = 64;   // heads per kernel-A workgroup
constexpr int kRecSlices = 8;   // column slices (one per kernel-B wave)
// fp16 dS / P are stored scaled by 2^8: dS is typically ~1e-5, inside
// fp16's subnormal range, and P <= 1 stays below 256.  bf16 has fp32's
// exponent range and is stored as is.
constexpr int kF16Shift = 8;
// a slice exponent that marks non-finite contributions
constexpr int kRecNonFinite = 0x7fff;
// Smallest slice exponent: a slice whose largest magnitude is below
// 2^kRecMinExp (a bf16 product of tiny P and d_out, or an all-zero slice)
// is stored with this exponent, so its scale 2^-e stays finite (2^120) and
// its stored values stay below 1; an all-zero slice then cannot raise the
// token's largest exponent and cost the fixed-point sum its resolution.
constexpr int kRecMinExp = -120;

__device__ __forceinline__ void bwd_dma16(unsigned lds_base, int voff, __amdgpu_buffer_rsrc_t rsrc) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_base), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void bwd_dma16_glb(unsigned lds_base, const void* gaddr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_base), "v"(gaddr) : "memory");
}
__device__ __forceinline__ void bwd_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __attribute__((aligned(16))) unsigned char g_bwd_zero_row[1024];

// Column slices of a record.  Unmerged: slices 0-3 split the dK | dK_rope
// tiles ((D + 64) / 16), slices 4-7 the dV tiles (D / 16); merged: the
// eight slices split the (D + 64) / 16 tiles of dK + dV | dK_rope.
template <int D, bool MERGE>
struct RecSlices {
  static constexpr int NK = (D + 64) / 16, NV = D / 16;
  static constexpr int MT = MERGE ? (NK + 7) / 8 : (NK / 4 > NV / 4 ? NK / 4 : NV / 4);
  static_assert(MERGE || (NK % 4 == 0 && NV % 4 == 0), "slices");
  // first column tile of slice s and its tile count
  static __host__ __device__ constexpr int t0(int s) {
    return MERGE ? s * NK / 8 : (s < 4 ? s * (NK / 4) : NK + (s - 4) * (NV / 4));
  }
  static __host__ __device__ constexpr int n(int s) {
    return MERGE ? (s + 1) * NK / 8 - s * NK / 8 : (s < 4 ? NK / 4 : NV / 4);
  }
};

// ---------------------------------------------------------------------------
// A. dq, dq_rope; dS / P; token list and bucket ranks
// ---------------------------------------------------------------------------
template <int D, typename T, bool BUF>
__global__ __launch_bounds__(kBwdWaves * 64, 1) void sfa_bwd_dq_kernel(SfaBwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int DR = 64;
  constexpr int KS = (D + DR) / 32, KSN = D / 32;
  constexpr int NDT = D / 16;
  constexpr int TILE = kBwdTile;
  constexpr int NT = kBwdWaves * 64;
  constexpr int ROW = D * 2;
  constexpr int TPI = 1024 / ROW;                // nope rows per DMA (1 KB per DMA)
  constexpr int NDN = TILE / TPI / kBwdWaves;    // nope DMAs per wave per tile
  constexpr int TR = kBwdHeads + 8;              // padded [token][head] row
  constexpr float kDsMul = __is_same(T, f16) ? (float)(1 << kF16Shift) : 1.f;
  static_assert(TILE % (TPI * kBwdWaves) == 0, "layout");

  constexpr int NBUF = 3;  // tile ring: tile t+2 is in flight while tile t runs
  __shared__ __attribute__((aligned(1024))) unsigned char s_k[NBUF][TILE * ROW];
  __shared__ __attribute__((aligned(1024))) unsigned char s_kr[NBUF][TILE * DR * 2];
  __shared__ int s_list[kBwdList + TILE];
  // dS, P and (bf16, short ranges) the lo part of dS of the 64 heads
  __shared__ __attribute__((aligned(16))) T s_t[3][TILE][TR];
  __shared__ int s_wcnt[kBwdWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int rowl = blockIdx.x;
  const int row = (int)(p.row0 + rowl);
  const int hg = blockIdx.y;
  const int hbase = hg * kBwdHeads;
  const RowInfo ri = sfa_row_info(p, row);
  const int64_t total_pos = (int64_t)p.K * p.bs;
  const int32_t* idx_row = p.idx + (int64_t)row * p.K;
  const u32x4 z4 = {0u, 0u, 0u, 0u};

  // ---- per-lane head hbase + 16*wave + li: fragments and statistics ----
  const int head = hbase + wave * 16 + li;
  const bool hv = head < p.n1;
  const int64_t hrow = (int64_t)row * p.n1 + (hv ? head : 0);
  V8 qf[KS], dof[KSN];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    u32x4 v;
    if (ks < KSN) v = *(const u32x4*)((const T*)p.q + hrow * D + ks * 32 + lg * 8);
    else v = *(const u32x4*)((const T*)p.qr + hrow * DR + (ks - KSN) * 32 + lg * 8);
    qf[ks] = as_v8<V8>(hv ? v : z4);
  }
  // every dO and O load is issued before any is used (used one by one, the
  // loads had come back a few at a time, one memory round trip each)
  u32x4 ov[KSN];
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks) {
    dof[ks] = as_v8<V8>(*(const u32x4*)((const T*)p.dout + hrow * D + ks * 32 + lg * 8));
    ov[ks] = *(const u32x4*)((const T*)p.out + hrow * D + ks * 32 + lg * 8);
  }
  float delta = 0.f;
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks) {
    const V8 ov8 = as_v8<V8>(ov[ks]);
#pragma unroll
    for (int j = 0; j < 8; ++j) delta += E::to_f32(dof[ks][j]) * E::to_f32(ov8[j]);
    if (!hv) dof[ks] = as_v8<V8>(z4);
  }
  delta = xgroup_sum(delta);  // lanes li, li+16, li+32, li+48 cover all D columns
  float m2 = 0.f, inv = 0.f;
  if (hv) {
    m2 = p.smax[hrow] * kLog2e;
    const float ss = p.ssum[hrow];
    inv = 1.f / (ss > 0.f ? ss : 1.f);
  } else {
    delta = 0.f;
  }
  // dq^T of this wave's column slice (d-tiles dt0 .. dt0 + NQW - 1 of the
  // D + 64 columns, nope tiles then rope) for the workgroup's four head tiles
  constexpr int NQ = NDT + DR / 16, NQW = NQ / kBwdWaves;
  static_assert(NQ % kBwdWaves == 0, "column slices");
  const int dt0 = __builtin_amdgcn_readfirstlane(wave) * NQW;
  f32x4 acc_dq[NQW][4];
#pragma unroll
  for (int q = 0; q < NQW; ++q)
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) acc_dq[q][ht] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // ---- tile DMA: wave w loads nope rows (j*4 + w)*TPI .. +TPI (lane L ->
  // row + L/CPT, source chunk (L%CPT) ^ nope_swz) and rope rows 8w .. 8w+7.
  // BUF: 32-bit buffer offsets (key tensors under 2 GiB; the range check
  // yields zero rows), otherwise 64-bit addresses and an explicit zero row.
  constexpr int CPT = 64 / TPI;  // chunks per row covered by one DMA
  __amdgpu_buffer_rsrc_t rk, rr;
  if constexpr (BUF) {
    rk = __builtin_amdgcn_make_buffer_rsrc((void*)p.k, (short)0, (int)(p.kv_rows * D * 2), 0x00020000);
    rr = __builtin_amdgcn_make_buffer_rsrc((void*)p.kr, (short)0, (int)(p.kv_rows * DR * 2), 0x00020000);
  }
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto issue_tile = [&](int t, int b) {
    int ph[NDN + 1];
#pragma unroll
    for (int j = 0; j < NDN; ++j) ph[j] = s_list[t * TILE + (j * kBwdWaves + wave_s) * TPI + lane / CPT];
    ph[NDN] = s_list[t * TILE + wave_s * 8 + (lane >> 3)];
#pragma unroll
    for (int j = 0; j < NDN; ++j) {
      const int tk = (j * kBwdWaves + wave_s) * TPI + lane / CPT;
      const int ch = (lane % CPT) ^ nope_swz(tk);
      const unsigned dst = (unsigned)(uintptr_t)&s_k[b][(j * kBwdWaves + wave_s) * TPI * ROW];
      if constexpr (BUF) {
        bwd_dma16(dst, ph[j] >= 0 ? ph[j] * ROW + ch * 16 : (int)0x80000000, rk);
      } else {
        bwd_dma16_glb(dst, ph[j] >= 0 ? (const void*)((const unsigned char*)p.k + (int64_t)ph[j] * ROW + ch * 16)
                                      : (const void*)(g_bwd_zero_row + ch * 16));
      }
    }
    {
      const int tk = wave_s * 8 + (lane >> 3);
      const int ch = (lane & 7) ^ rope_swz(tk);
      const unsigned dst = (unsigned)(uintptr_t)&s_kr[b][wave_s * 8 * DR * 2];
      if constexpr (BUF) {
        bwd_dma16(dst, ph[NDN] >= 0 ? ph[NDN] * (DR * 2) + ch * 16 : (int)0x80000000, rr);
      } else {
        bwd_dma16_glb(dst, ph[NDN] >= 0
                               ? (const void*)((const unsigned char*)p.kr + (int64_t)ph[NDN] * (DR * 2) + ch * 16)
                               : (const void*)(g_bwd_zero_row + ch * 16));
      }
    }
  };

  // dS / P rows of this workgroup's heads in the slot's [dS | P] row
  const int nh = min(kBwdHeads, p.hp - hbase);  // 32 or 64 heads stored
  T* dsp_row = (T*)p.dsp + (int64_t)rowl * p.kposp * 2 * p.hp + hbase;
  int32_t* list_row = p.list + (int64_t)rowl * p.kposp;
  int32_t* rank_row = p.rank + (int64_t)rowl * p.kposp;

  int jbase = 0;  // slots compacted by earlier rounds
  for (int64_t c0 = 0; c0 < total_pos; c0 += kBwdList) {
    // ---- compact this range of positions into s_list (stable order) ----
    const int64_t c1 = min(total_pos, c0 + (int64_t)kBwdList);
    int n_valid = 0;
    // The range's index entries are all loaded first (unconditional, at
    // clamped positions), and the slots' bucket ranks are stored after the
    // whole range's atomics are in flight: a load or atomic whose value is
    // used right away is waited for on the spot, which had cost two memory
    // round trips per 256 positions.
    constexpr int RPT = kBwdList / NT;
    static_assert(RPT * NT == kBwdList, "positions per thread");
    int idv[RPT], rkv[RPT], jv[RPT];
#pragma unroll
    for (int u = 0; u < RPT; ++u) idv[u] = sfa_load_id(p, idx_row, (int)min(c0 + u * NT + tid, c1 - 1));
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const int64_t b0 = c0 + (int64_t)u * NT;
      jv[u] = -1;
      rkv[u] = 0;
      if (b0 >= c1) continue;  // uniform
      const int64_t pos = b0 + tid;
      int phys = 0;
      bool valid = false;
      if (ri.active && pos < c1) valid = sfa_resolve_id(p, ri, idv[u], (int)pos, &phys, (const int32_t*)nullptr);
      const unsigned long long m = __ballot(valid);
      if (lane == 0) s_wcnt[wave] = __popcll(m);
      lds_barrier();
      int off = n_valid, tot = 0;
#pragma unroll
      for (int w = 0; w < kBwdWaves; ++w) {
        const int c = s_wcnt[w];
        off += w < wave ? c : 0;
        tot += c;
      }
      if (valid) {
        const int j = off + __popcll(m & ((1ull << lane) - 1ull));
        s_list[j] = phys;
        if (hg == 0) {
          // the token list and, from the token's count, the slot's place in
          // its bucket (integer counts: their order does not matter)
          list_row[jbase + j] = phys;
          rkv[u] = atomicAdd(&p.cnt[phys], 1);
          jv[u] = jbase + j;
        }
      }
      n_valid += tot;
      lds_barrier();
    }
#pragma unroll
    for (int u = 0; u < RPT; ++u)
      if (jv[u] >= 0) rank_row[jv[u]] = rkv[u];
    if (tid < TILE) s_list[n_valid + tid] = -1;
    lds_barrier();
    const int n_tiles = (n_valid + TILE - 1) / TILE;
    if (n_tiles > 0) issue_tile(0, 0);
    if (n_tiles > 1) issue_tile(1, 1);
    // P.V-style split of dS into bf16 hi + lo for the dq product only while
    // the range has few tokens (as the forward splits P): over longer ranges
    // one rounding of dS averages out.
    const bool lo = n_valid < 256;

    for (int t = 0; t < n_tiles; ++t) {
      const int b = t % NBUF;
      // tile t's DMA has landed.  Issued per wave in the order DMA(t),
      // stores(t-1), DMA(t+1), and vector memory operations, loads and
      // stores alike, retire in order on this counter: with tile t+1's
      // NDN + 1 DMAs and (after a full tile t-1) its first dS / P row store
      // allowed in flight, DMA(t) is complete without waiting for the
      // stores' acknowledgements.
      if (t > 0 && t + 1 < n_tiles) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(NDN + 2) : "memory");
      else if (t + 1 < n_tiles) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(NDN + 1) : "memory");
      else bwd_wait_all();
      lds_barrier();
      const unsigned char* kt = s_k[b];
      const unsigned char* krt = s_kr[b];

      // ---- S^T = K.Q^T and dP^T = K_nope.dO^T (shared K fragments) ----
      f32x4 acc_s[2], acc_p[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        acc_s[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        acc_p[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      }
      // K fragments are read PF steps ahead of their MFMAs; the scheduling
      // barrier keeps the reads there (sunk next to their MFMAs, each MFMA
      // would wait out a full LDS round trip with no other wave to run)
      {
        constexpr int NS = 2 * KS, PF = 6;
        auto kread = [&](int st) -> u32x4 {
          const int ks = st >> 1, tk = (st & 1) * 16 + li;
          const unsigned char* a = ks < KSN ? kt + tk * ROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16)
                                            : krt + tk * (DR * 2) + ((((ks - KSN) * 4 + lg) ^ rope_swz(tk)) * 16);
          return *(const u32x4*)a;
        };
        u32x4 fa[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) fa[i] = kread(i);
#pragma unroll
        for (int st = 0; st < NS; ++st) {
          const int ks = st >> 1, tt = st & 1;
          const V8 av = as_v8<V8>(fa[st % PF]);
          if (st + PF < NS) fa[st % PF] = kread(st + PF);
          acc_s[tt] = E::mfma(av, qf[ks], acc_s[tt]);
          if (ks < KSN) acc_p[tt] = E::mfma(av, dof[ks], acc_p[tt]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }

      // ---- P^T, dS^T (token tt*16 + 4*lg + r, head li) ----
      constexpr bool kSplit = __is_same(T, bf16);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tt = j >> 2, r = j & 3;
        const int tk = tt * 16 + lg * 4 + r;
        const bool tv = t * TILE + tk < n_valid;
        const float pp = tv ? fast_exp2(acc_s[tt][r] * p.scale_log2 - m2) * inv : 0.f;
        const float ds = pp * (acc_p[tt][r] - delta) * p.scale;
        const T dh = E::from_f32(ds * kDsMul);
        s_t[0][tk][wave * 16 + li] = dh;
        s_t[1][tk][wave * 16 + li] = E::from_f32(pp * kDsMul);
        if (kSplit && lo) s_t[2][tk][wave * 16 + li] = E::from_f32(ds - E::to_f32(dh));
      }
      lds_barrier();  // dS / P of the 64 heads in LDS
      // ---- dS / P rows out (16 bytes per thread: 8 heads of one slot); all
      // of a thread's LDS reads go out before its stores ----
      {
        const int cpr = nh / 8;  // chunks per (slot, dS | P) row: 4 or 8
        constexpr int NE = (TILE * 2 * (kBwdHeads / 8) + NT - 1) / NT;
        u32x4 v[NE];
        int64_t off[NE];
        bool ok[NE];
#pragma unroll
        for (int i = 0; i < NE; ++i) {
          const int e = tid + i * NT;
          const bool in = e < TILE * 2 * cpr;
          const int ee = in ? e : 0;
          const int tk = ee / (2 * cpr), rem = ee - tk * 2 * cpr, which = rem / cpr, c = rem - which * cpr;
          const int j = t * TILE + tk;
          ok[i] = in && j < n_valid;
          off[i] = ((int64_t)(jbase + j) * 2 + which) * p.hp + c * 8;
          v[i] = *(const u32x4*)&s_t[which][tk][c * 8];
        }
#pragma unroll
        for (int i = 0; i < NE; ++i)
          if (ok[i]) *(u32x4*)(dsp_row + off[i]) = v[i];
      }
      // tile t+2 into the buffer tile t-1 used (every wave is past tile t's
      // first barrier, so past tile t-1)
      if (t + 2 < n_tiles) issue_tile(t + 2, (t + 2) % NBUF);

      // ---- dq^T += K^T.dS^T over this wave's column slice ----
      // Both operands through the transposing read: rows 4*lg + li/4 (+16),
      // 16-byte chunk 2*c + (li&3)/2 (+8 bytes for odd li) of a [token][col]
      // tile give k-index 8*lg + j as token 16*(j>>2) + 4*lg + (j&3), column
      // 16*c + li.  dS^T of all four head tiles is read once per tile, so
      // each K^T fragment feeds four MFMAs (the wave's 16 heads alone read
      // the whole K tile transposed for one MFMA per fragment).  fp16 dS is
      // carried as dS * 2^8 (the workspace value); dq is scaled back at the end.
      {
        const int r1 = lg * 4 + (li >> 2);
        const int hb = (li & 3) >> 1;
        auto tr8 = [&](const unsigned char* p1, const unsigned char* p2) -> V8 {
          const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
          const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
          const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
          return __builtin_bit_cast(V8, w);
        };
        // K^T fragment of d-tile dt (nope tiles, then the rope tiles)
        auto tread = [&](int dt) -> V8 {
          const bool nope = dt < NDT;
          const int ch = 2 * (nope ? dt : dt - NDT) + hb;
          const unsigned char* p1 = nope ? kt + r1 * ROW + ((ch ^ nope_swz(r1)) * 16)
                                         : krt + r1 * (DR * 2) + ((ch ^ rope_swz(r1)) * 16);
          const unsigned char* p2 = nope ? kt + (r1 + 16) * ROW + ((ch ^ nope_swz(r1 + 16)) * 16)
                                         : krt + (r1 + 16) * (DR * 2) + ((ch ^ rope_swz(r1 + 16)) * 16);
          return tr8(p1 + (li & 1) * 8, p2 + (li & 1) * 8);
        };
        auto sread = [&](int plane, int ht) -> V8 {
          const unsigned char* b0 = (const unsigned char*)&s_t[plane][0][0] + (2 * ht + hb) * 16 + (li & 1) * 8;
          return tr8(b0 + r1 * (TR * 2), b0 + (r1 + 16) * (TR * 2));
        };
        constexpr int PF = 4;
        V8 fk[PF], dsb[4];
#pragma unroll
        for (int i = 0; i < PF; ++i) fk[i] = tread(dt0 + i);
#pragma unroll
        for (int ht = 0; ht < 4; ++ht) dsb[ht] = sread(0, ht);
#pragma unroll
        for (int q = 0; q < NQW; ++q) {
          const V8 w = fk[q % PF];
          if (q + PF < NQW) fk[q % PF] = tread(dt0 + q + PF);
#pragma unroll
          for (int ht = 0; ht < 4; ++ht) acc_dq[q][ht] = E::mfma(w, dsb[ht], acc_dq[q][ht]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (kSplit && lo) {
          // the lo part of dS (short ranges), a second pass over the slice
#pragma unroll
          for (int ht = 0; ht < 4; ++ht) dsb[ht] = sread(2, ht);
#pragma unroll
          for (int i = 0; i < PF; ++i) fk[i] = tread(dt0 + i);
#pragma unroll
          for (int q = 0; q < NQW; ++q) {
            const V8 w = fk[q % PF];
            if (q + PF < NQW) fk[q % PF] = tread(dt0 + q + PF);
#pragma unroll
            for (int ht = 0; ht < 4; ++ht) acc_dq[q][ht] = E::mfma(w, dsb[ht], acc_dq[q][ht]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      // s_t is rewritten by the next tile only after its first barrier
    }
    bwd_wait_all();
    lds_barrier();  // s_list is rebuilt for the next range
    jbase += n_valid;
  }
  if (hg == 0 && tid == 0) p.nval[rowl] = jbase;

  // ---- dq, dq_rope: C register r of (q, ht) is column 16*(dt0 + q) +
  // 4*lg + r of head hbase + 16*ht + li ----
  {
    typedef T T4 __attribute__((ext_vector_type(4)));
    const float mul = 1.f / kDsMul;
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) {
      const int hh = hbase + ht * 16 + li;
      if (hh < p.n1) {
        const int64_t hr = (int64_t)row * p.n1 + hh;
#pragma unroll
        for (int q = 0; q < NQW; ++q) {
          const int dt = dt0 + q;
          const f32x4 a = acc_dq[q][ht] * mul;
          const T4 o = {E::from_f32(a[0]), E::from_f32(a[1]), E::from_f32(a[2]), E::from_f32(a[3])};
          T* dst = dt < NDT ? (T*)p.dq + hr * D + dt * 16 : (T*)p.dqr + hr * DR + (dt - NDT) * 16;
          *(T4*)(dst + lg * 4) = o;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// B. records: per attended token, the head-summed dK | dK_rope | dV columns
// ---------------------------------------------------------------------------
// rec^T[col][token] = sum_h X[h][col] * Y[h][token] on v_mfma_f32_16x16x32:
// A = X^T (lane: column li, heads 8*lg..) resident for the row, B = dS or P
// (lane: token li, heads 8*lg..) from LDS; C register r = column 4*lg + r of
// token li, so a lane stores 4 consecutive fp16 values of one record.
// Waves of the record kernel: eight (two per SIMD, 256 registers each), or
// four when a wave's resident operands need more (D = 512 with 128 heads:
// each wave then takes two slices, one after the other, with 512 registers).
template <int D, typename T, bool MERGE, int HP>
__global__ __launch_bounds__(8 * 64, 1) void sfa_bwd_rec_kernel(SfaBwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  using SL = RecSlices<D, MERGE>;
  constexpr int DR = 64;
  constexpr int MT = SL::MT;
  constexpr int NW = 8;
  constexpr int KH = HP / 32;          // k-steps over heads
  constexpr int TILE = kBwdTile;
  constexpr int ROWB = 2 * HP * 2;     // bytes of a slot's [dS | P] row
  constexpr int CH = ROWB / 16;        // 16-byte chunks per slot row
  constexpr int TB = TILE * ROWB;      // tile bytes
  constexpr int NDMA = TB / 1024;      // 1 KB DMAs per tile
  constexpr int SPD = 1024 / ROWB;     // slots per DMA
  constexpr int SWM = CH < 16 ? CH - 1 : 15;  // chunk swizzle mask
  constexpr int XC = 2 * D + DR;       // staged columns: Q nope | Q rope | dO
  constexpr int XROW = XC + 16;        // padded staged row (elements)
  static_assert(NDMA >= 1 && NDMA <= 2 * NW && kRecSlices == NW, "tile DMAs / slices");
  constexpr int NBUF = 3;              // tile ring: tile t+2 is in flight while tile t runs
  constexpr int NPOS = 2048;           // record positions resolved per refill (64 tiles)
  __shared__ __attribute__((aligned(1024))) unsigned char s_ds[NBUF][TB];
  __shared__ __attribute__((aligned(16))) T s_x[32 * XROW];  // 32 heads of [Q | Q rope | dO]
  __shared__ int s_pos[NPOS];          // bucket position of each slot of 64 tiles

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int rowl = blockIdx.x;
  const int64_t row = p.row0 + rowl;
  const int nv = p.nval[rowl];
  const int n_tiles = (nv + TILE - 1) / TILE;

  // ---- this wave's column slice and its A operands X^T (X = [Q | Q rope |
  // dO] of all heads): 32 heads at a time are staged row-major in LDS and
  // read back transposed (ds_read_b64_tr_b16: lane li gets column li of a
  // 4-row block).  Operand slot j of lane group lg holds head
  // 32*ks + 16*(j >> 2) + 4*lg + (j & 3); the dS / P reads below use the
  // same order. ----
  const int sl = wave_s;
  const int ct0 = SL::t0(sl), nct = SL::n(sl);
  const bool vslice = !MERGE && sl >= 4;  // dV columns (P^T . dO)
  V8 xa[MT][KH];                          // Q nope / Q rope / dO columns
  V8 xo[MERGE ? MT : 1][KH];              // merged nope columns: dO
  constexpr int CPR = XC / 8;             // 16-byte chunks per staged row
  // A thread's chunks of the 32 heads are all loaded before any is written:
  // a load under a condition, or written to LDS right away, is waited for
  // on the spot, and the staging then took one memory round trip per chunk
  // (per-row timeline: 120 k cycles before the tile loop, against about
  // 8.5 k per tile).  Heads >= N1 load head 0 and are zeroed at the write.
  constexpr int XPT = (32 * CPR + NW * 64 - 1) / (NW * 64);  // chunks per thread
  for (int ks = 0; ks < KH; ++ks) {
    u32x4 xv[XPT];
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int e = u * NW * 64 + tid;
      const int ec = e < 32 * CPR ? e : 0;
      const int hh = ec / CPR, c = (ec - hh * CPR) * 8;
      const int h = ks * 32 + hh;
      const int64_t r = row * p.n1 + (h < p.n1 ? h : 0);
      const T* src = c < D ? (const T*)p.q + r * D + c
                   : c < D + DR ? (const T*)p.qr + r * DR + (c - D)
                                : (const T*)p.dout + r * D + (c - D - DR);
      xv[u] = *(const u32x4*)src;
    }
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int e = u * NW * 64 + tid;
      const int hh = e / CPR, c = (e - hh * CPR) * 8;
      if (e < 32 * CPR) *(u32x4*)&s_x[hh * XROW + c] = ks * 32 + hh < p.n1 ? xv[u] : (u32x4){0u, 0u, 0u, 0u};
    }
    lds_barrier();
    const int r1 = lg * 4 + (li >> 2);
    auto xread = [&](int col0) -> V8 {
      const T* a1 = &s_x[r1 * XROW + col0 + 4 * (li & 3)];
      const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)a1));
      const i16x4 w2 =
          __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(a1 + 16 * XROW)));
      const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
      return __builtin_bit_cast(V8, w);
    };
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int ct = ct0 + (i < nct ? i : 0);
      xa[i][ks] = xread(ct * 16);
      if constexpr (MERGE) xo[i][ks] = xread(D + DR + (ct * 16 < D ? ct * 16 : 0));
    }
    lds_barrier();  // s_x is restaged for the next 32 heads
  }

  // ---- tile DMA: the tile's slot rows are contiguous in dS / P; slot s of
  // the tile lands with its 16-byte chunk c at chunk c ^ (s & SWM) ----
  const unsigned char* src_row = (const unsigned char*)p.dsp + (int64_t)rowl * p.kposp * ROWB;
  auto issue_tile = [&](int t, int b) {
    for (int d = wave_s; d < NDMA; d += NW) {
      const int s = d * SPD + lane / CH;       // slot within the tile
      const int c = (lane % CH) ^ (s & SWM);   // source chunk for this LDS chunk
      const unsigned dst = (unsigned)(uintptr_t)&s_ds[b][d * 1024];
      bwd_dma16_glb(dst, src_row + ((int64_t)t * TILE + s) * ROWB + c * 16);
    }
  };
  // B operand of token tt*16 + li for k-step ks of dS (which 0) or P (1):
  // heads 32*ks + 4*lg .. +3 and 32*ks + 16 + 4*lg .. +3 (8 bytes each)
  auto b_read = [&](int b, int tt, int ks, int which) -> V8 {
    const int s = tt * 16 + li;
    const int c = which * (HP / 8) + ks * 4 + (lg >> 1);
    const unsigned char* rb = &s_ds[b][s * ROWB + (lg & 1) * 8];
    const i16x4 w1 = *(const i16x4*)(rb + ((c ^ (s & SWM)) * 16));
    const i16x4 w2 = *(const i16x4*)(rb + (((c + 2) ^ (s & SWM)) * 16));
    const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
    return __builtin_bit_cast(V8, w);
  };

  const int32_t* list_row = p.list + (int64_t)rowl * p.kposp;
  const int32_t* rank_row = p.rank + (int64_t)rowl * p.kposp;
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  // record staging: 16 rows (tokens) of the slice per wave, in s_x (free
  // after the operands are read)
  constexpr int SROW = MT * 16 + 8;
  static_assert(NW * 16 * SROW <= 32 * XROW, "staging fits");
  _Float16* stg = (_Float16*)s_x + wave_s * 16 * SROW;
  // DMAs this wave issues per tile (0, 1 or 2)
  const int ndw = wave_s < NDMA ? (NDMA - wave_s + NW - 1) / NW : 0;
  if (n_tiles > 0) issue_tile(0, 0);
  if (n_tiles > 1) issue_tile(1, 1);
  // Vector-memory stores a wave issues per 16-token half of a full tile
  // (every token of the half valid): the whole-record loop below, one
  // 16-byte store per iteration it < kRecIters (two records per wave, 32
  // lanes each; lane 0 is active in every iteration, so none is skipped),
  // then the one exponent store (lanes of group 0).  The tile wait below
  // counts on exactly these: a store fewer per half would let it pass
  // before the tile's DMA has landed.
  constexpr int kRecPieces = 2 * (MERGE ? SL::NK : SL::NK + SL::NV);  // 16-byte pieces per record
  constexpr int kRecIters = (kRecPieces + 31) / 32;
  static_assert(kRecPieces > (kRecIters - 1) * 32, "lane 0 stores in every record iteration");
  constexpr int kHalfStores = kRecIters + 1;
  for (int t = 0; t < n_tiles; ++t) {
    const int b = t % NBUF;
    // tile t's DMA has landed: per wave the issue order is DMA(t),
    // stores(t-1) (two halves), DMA(t+1), and vector memory operations,
    // loads and stores alike, retire in order on this counter, so the
    // previous (full) tile's stores and DMA(t+1) may stay in flight (waiting
    // for them too held every tile behind the previous tile's store
    // acknowledgements)
    if (t > 0 && t + 1 < n_tiles && ndw >= 2) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kHalfStores + 2) : "memory");
    else if (t > 0 && t + 1 < n_tiles && ndw == 1) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kHalfStores + 1) : "memory");
    else if (t > 0 && t + 1 < n_tiles) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kHalfStores) : "memory");
    else if (t + 1 < n_tiles && ndw >= 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else if (t + 1 < n_tiles && ndw == 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
    else bwd_wait_all();
    lds_barrier();
    if ((t % (NPOS / TILE)) == 0) {
      // bucket positions of the next 64 tiles' slots (every wave is past
      // the reads of the previous ones); every load of a round is issued
      // before its values are used (two memory round trips, not two per
      // slot)
      constexpr int PPT = NPOS / (NW * 64);
      int lt[PPT], lr[PPT];
#pragma unroll
      for (int u = 0; u < PPT; ++u) {
        const int j = t * TILE + u * NW * 64 + tid;
        const int jc = j < nv ? j : 0;
        lt[u] = list_row[jc];
        lr[u] = rank_row[jc];
      }
#pragma unroll
      for (int u = 0; u < PPT; ++u) lt[u] = p.offs[lt[u]];
#pragma unroll
      for (int u = 0; u < PPT; ++u) {
        const int j = t * TILE + u * NW * 64 + tid;
        s_pos[u * NW * 64 + tid] = j < nv ? lt[u] + lr[u] : 0;
      }
      lds_barrier();
    }
    // one 16-token half at a time: the two halves' accumulators are not
    // live together
#pragma unroll 1
    for (int tt = 0; tt < 2; ++tt) {
      const int j = t * TILE + tt * 16 + li;
      const int64_t pos = s_pos[(j - (t / (NPOS / TILE)) * NPOS)];
      f32x4 acc[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
      // k-steps outer: each B fragment (dS or P of 32 heads) is read right
      // before the MT products that use it
#pragma unroll
      for (int ks = 0; ks < KH; ++ks) {
        const V8 bf = b_read(b, tt, ks, vslice ? 1 : 0);
        V8 bq;
        if constexpr (MERGE) bq = b_read(b, tt, ks, 1);
#pragma unroll
        for (int i = 0; i < MT; ++i)
          if (i < nct) {
            acc[i] = E::mfma(xa[i][ks], bf, acc[i]);
            if constexpr (MERGE)
              if ((ct0 + i) * 16 < D) acc[i] = E::mfma(xo[i][ks], bq, acc[i]);
          }
      }
      // the slice's largest magnitude for token li (lanes li, li+16, li+32, li+48)
      // (a NaN-propagating maximum, so that a NaN value is flagged too; a
      // non-finite lane reads as infinite in the cross-lane reduction)
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = __builtin_elementwise_maximum(mx, fabsf(acc[i][r]));
      mx = mx < INFINITY ? mx : INFINITY;
      mx = xgroup_max(mx);
      // stored value = acc * 2^-e with 2^e > max |acc| (|stored| < 1); e is
      // at least kRecMinExp (an all-zero slice gets it too)
      int e = kRecMinExp;
      if (!(mx < INFINITY)) e = kRecNonFinite;
      else if (mx > 0.f) (void)frexpf(mx, &e);
      if (e < kRecMinExp) e = kRecMinExp;
      const float sc = e == kRecNonFinite ? 1.f : ldexpf(1.f, -e);
      // the 16 tokens' slices go to this wave's LDS staging rows; the
      // records are stored whole from there, below
      _Float16* srow = stg + li * SROW;
#pragma unroll
      for (int i = 0; i < MT; ++i)
        if (i < nct) {
          const h4 v = {(_Float16)(acc[i][0] * sc), (_Float16)(acc[i][1] * sc), (_Float16)(acc[i][2] * sc),
                        (_Float16)(acc[i][3] * sc)};
          *(h4*)(srow + i * 16 + lg * 4) = v;
        }
      lds_barrier();  // every slice of the half's 16 tokens is staged
      // whole records: wave w stores tokens 2w (lanes 0-31) and 2w + 1
      // (lanes 32-63) of the half.  A record is its slices' column tiles in
      // order; 16-byte piece gp is half gp & 1 of column tile gp / 2, read
      // from that tile's slice staging.  A record row (17 or 9 whole 128-byte
      // lines) goes out as full-line writes, where per-slice pieces wrote 64
      // bytes of 16 different records per instruction.
      {
        constexpr int PPR = kRecPieces;
        constexpr int NIT = kRecIters;  // the store count kHalfStores is derived from
        const int tk = wave_s * 2 + (lane >> 5);
        const int j2 = t * TILE + tt * 16 + tk;
        const int64_t pos2 = s_pos[j2 - (t / (NPOS / TILE)) * NPOS];
        u32x4 pv[NIT];
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int gp = it * 32 + (lane & 31);
          const int ct = (gp < PPR ? gp : 0) >> 1;
          int s2 = 0;
#pragma unroll
          for (int u = 1; u < NW; ++u) s2 += ct >= SL::t0(u) ? 1 : 0;
          pv[it] = *(const u32x4*)((const _Float16*)s_x + (s2 * 16 + tk) * SROW + (ct - SL::t0(s2)) * 16 +
                                   (gp & 1) * 8);
        }
        if (j2 < nv) {
#pragma unroll
          for (int it = 0; it < NIT; ++it) {
            const int gp = it * 32 + (lane & 31);
            // non-temporal: the records are read back only by the reduction
            // kernel, gigabytes later
            if (gp < PPR) __builtin_nontemporal_store(pv[it], (u32x4*)(p.rec + pos2 * p.nc + gp * 8));
          }
        }
      }
      lds_barrier();  // the staging is rewritten by the next half
      // the exponent of the true value (fp16 dS / P carry 2^kF16Shift)
      if (j < nv && lg == 0)
        p.rexp[pos * kRecSlices + sl] =
            (int16_t)(e == kRecNonFinite ? e : e - (__is_same(T, f16) ? kF16Shift : 0));
    }
    // tile t+2 into the buffer tile t-1 used (every wave is past tile t's
    // barrier), after this tile's stores
    if (t + 2 < n_tiles) issue_tile(t + 2, (t + 2) % NBUF);
  }
}

// ---------------------------------------------------------------------------
// C. per key token: the sum of its records, one wave per column slice
// ---------------------------------------------------------------------------
// Records of token t are rec[offs[t] .. offs[t+1]); a slice value is
// fp16 * 2^e.  They are summed in fixed point with 2^-F resolution: each
// term rounded to the grid (scaled and rounded in fp32, where the fp16
// value times a power of two is exact, then widened to a double), F chosen
// from the largest slice exponent and the record count so that every
// partial sum is an integer below 2^52, so the double additions are exact
// and associative (a conversion to int64 per element measured slower).  A lane
// reads 16 bytes (8 columns) of a record, so one load instruction covers
// 64 / (width / 8) records of the slice; the lanes holding the same columns
// are summed through LDS at the end.  The chunk's sum is added to the
// running fp32 sum (FIRST: none yet); FINAL writes the key gradients in the
// key dtype.
template <typename T, int D, bool MERGE, bool FIRST, bool FINAL>
__global__ __launch_bounds__(kRecSlices * 64) void sfa_bwd_reduce_kernel(SfaBwdParams p) {
  using SL = RecSlices<D, MERGE>;
  constexpr int DR = 64;
  constexpr int U = 4;  // loads in flight per lane
  __shared__ double s_red[kRecSlices][64][8];
  const int lane = threadIdx.x & 63;
  const int s = threadIdx.x >> 6;  // slice
  const int64_t t = blockIdx.x;
  const int c0 = SL::t0(s) * 16, width = SL::n(s) * 16;  // <= 160 columns
  const int cps = width / 8;                 // 16-byte chunks per record slice
  const int rpi = 64 / cps;                  // records per load instruction
  const int u = lane / cps, ch = lane - u * cps;
  const bool act = u < rpi;
  const int o0 = __builtin_amdgcn_readfirstlane(p.offs[t]);
  const int len = __builtin_amdgcn_readfirstlane(p.offs[t + 1]) - o0;
  // pass 1: the largest slice exponent
  int emax = -100000;
  for (int i = lane; i < len; i += 64) emax = max(emax, (int)p.rexp[(int64_t)(o0 + i) * kRecSlices + s]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) emax = max(emax, __shfl_xor(emax, o));
  const bool nonfinite = emax == kRecNonFinite;
  int lb = 0;
  while ((1 << lb) < len) ++lb;
  // every term is rounded to the grid 2^-F and the sums of such integers,
  // |sum| < len * 2^emax * 2^F <= 2^52, are exact in a double: the
  // additions do not depend on their order (the records' order in the
  // bucket, the lanes' split of them)
  const int F = 52 - emax - lb;
  // pass 2
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  double a[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  if (len > 0 && !nonfinite && act) {
    const _Float16* src = p.rec + (int64_t)o0 * p.nc + c0 + ch * 8;
    const int16_t* ex = p.rexp + (int64_t)o0 * kRecSlices + s;
    for (int base = 0; base < len; base += rpi * U) {
      h8 v[U];
      int ev[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int r = base + k * rpi + u;
        const bool ok = r < len;
        v[k] = ok ? *(const h8*)(src + (int64_t)r * p.nc) : (h8){0, 0, 0, 0, 0, 0, 0, 0};
        ev[k] = ok ? (int)ex[(int64_t)r * kRecSlices] : 0;
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        // ev + F <= 52 for every record of the token; idle lanes (ev = 0)
        // hold zeros, and 2^F can exceed fp32's range (0 * inf is NaN)
        const float sc = ldexpf(1.f, min(ev[k] + F, 60));
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] += (double)__builtin_rintf((float)v[k][e] * sc);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_red[s][lane][e] = a[e];
  __syncthreads();
  if (lane >= cps) return;
  double sum[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  for (int k = 0; k < rpi; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) sum[e] += s_red[s][k * cps + ch][e];
  const double us = ldexp(1.0, -F);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = c0 + ch * 8 + e;  // record column
    float v = len == 0 ? 0.f : (nonfinite ? NAN : (float)(sum[e] * us));
    float* ap = p.acc + t * p.nc + c;
    if (!FIRST) v += *ap;
    if (!FINAL) {
      *ap = v;
      continue;
    }
    const T o = Elem<T>::from_f32(v);
    if (c < D) ((T*)p.dk)[t * D + c] = o;
    else if (c < D + DR) ((T*)p.dkr)[t * DR + (c - D)] = o;
    else ((T*)p.dv)[t * D + (c - D - DR)] = o;
  }
}

__global__ __launch_bounds__(256) void bwd_zero_kernel(int32_t* a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] = 0;
}

// exclusive scan of cnt[0..n) into offs[0..n] (one workgroup)
__global__ __launch_bounds__(1024) void bwd_scan_kernel(const int32_t* cnt, int32_t* offs, int64_t n) {
  __shared__ int32_t s_sum[1024];
  const int tid = threadIdx.x;
  const int64_t per = (n + 1023) / 1024;
  const int64_t lo = min(n, tid * per), hi = min(n, lo + per);
  int32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += cnt[i];
  s_sum[tid] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int32_t v = tid >= o ? s_sum[tid - o] : 0;
    __syncthreads();
    s_sum[tid] += v;
    __syncthreads();
  }
  int32_t run = tid > 0 ? s_sum[tid - 1] : 0;
  for (int64_t i = lo; i < hi; ++i) {
    offs[i] = run;
    run += cnt[i];
  }
  if (tid == 1023) offs[n] = s_sum[1023];
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Rows per chunk: the per-row workspace of a chunk stays within this budget
// (a whole S = 4096, topK = 2048, N1 = 128, D = 512 problem fits one chunk).
constexpr size_t kBwdChunkBudget = 24ull << 30;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct BwdPlan {
  int64_t hp, kposp, nc, chunk_rows, nchunks;
  size_t cnt, offs, acc, list, rank, nval, dsp, rec, rexp, total;
};

static BwdPlan bwd_plan(int64_t q_rows, int64_t kv_rows, int64_t n1, int64_t d, int64_t total_pos, bool merge,
                        int esz) {
  BwdPlan L;
  L.hp = ((n1 + 31) / 32) * 32;
  L.kposp = ((total_pos + 31) / 32) * 32;
  L.nc = merge ? d + 64 : 2 * d + 64;
  const size_t per_row = (size_t)L.kposp * (2 * sizeof(int32_t) + 2 * L.hp * esz + L.nc * sizeof(_Float16) +
                                            kRecSlices * sizeof(int16_t)) + sizeof(int32_t);
  const size_t budget = (test_flags() & kTestSmallBwdChunks) ? ((size_t)1 << 16) : kBwdChunkBudget;
  int64_t cr = (int64_t)(budget / per_row);
  if (cr < 1) cr = 1;
  // equal chunks
  L.nchunks = q_rows > 0 ? (q_rows + cr - 1) / cr : 1;
  L.chunk_rows = q_rows > 0 ? (q_rows + L.nchunks - 1) / L.nchunks : 1;
  size_t o = 0;
  L.cnt = o;
  o += align256((size_t)kv_rows * sizeof(int32_t));
  L.offs = o;
  o += align256((size_t)(kv_rows + 1) * sizeof(int32_t));
  L.acc = o;
  if (L.nchunks > 1) o += align256((size_t)kv_rows * L.nc * sizeof(float));
  L.nval = o;
  o += align256((size_t)L.chunk_rows * sizeof(int32_t));
  L.list = o;
  o += align256((size_t)L.chunk_rows * L.kposp * sizeof(int32_t));
  L.rank = o;
  o += align256((size_t)L.chunk_rows * L.kposp * sizeof(int32_t));
  L.dsp = o;
  o += align256((size_t)L.chunk_rows * L.kposp * 2 * L.hp * esz);
  L.rec = o;
  o += align256((size_t)L.chunk_rows * L.kposp * L.nc * sizeof(_Float16));
  L.rexp = o;
  o += align256((size_t)L.chunk_rows * L.kposp * kRecSlices * sizeof(int16_t));
  L.total = o;
  return L;
}

size_t sfa_bwd_workspace_bytes(int64_t q_rows, int64_t kv_rows, int64_t n1, int64_t d, int64_t total_pos,
                               bool merge) {
  return bwd_plan(q_rows, kv_rows, n1, d, total_pos, merge, 2).total;
}

template <int D, typename T, bool MERGE>
static hipError_t run_bwd_chunks(SfaBwdParams p, const BwdPlan& L, hipStream_t stream) {
  const bool buf = (int64_t)p.kv_rows * D * 2 < (1ll << 31) && !(test_flags() & kTestForceGlobalGather);
  const int64_t zb = (p.kv_rows + 255) / 256;
  for (int64_t c = 0; c < L.nchunks; ++c) {
    p.row0 = c * L.chunk_rows;
    const int64_t nr = min(L.chunk_rows, p.rows - p.row0);
    if (nr <= 0) break;
    p.nrows = (int32_t)nr;
    hipLaunchKernelGGL(bwd_zero_kernel, dim3((unsigned)zb), dim3(256), 0, stream, p.cnt, p.kv_rows);
    const dim3 ga((unsigned)nr, (unsigned)((p.n1 + kBwdHeads - 1) / kBwdHeads));
    if (buf) hipLaunchKernelGGL((sfa_bwd_dq_kernel<D, T, true>), ga, dim3(kBwdWaves * 64), 0, stream, p);
    else hipLaunchKernelGGL((sfa_bwd_dq_kernel<D, T, false>), ga, dim3(kBwdWaves * 64), 0, stream, p);
    hipLaunchKernelGGL(bwd_scan_kernel, dim3(1), dim3(1024), 0, stream, p.cnt, p.offs, p.kv_rows);
    const dim3 gb((unsigned)nr);
    if (p.hp == 32) hipLaunchKernelGGL((sfa_bwd_rec_kernel<D, T, MERGE, 32>), gb, dim3(512), 0, stream, p);
    else if (p.hp == 64) hipLaunchKernelGGL((sfa_bwd_rec_kernel<D, T, MERGE, 64>), gb, dim3(512), 0, stream, p);
    else hipLaunchKernelGGL((sfa_bwd_rec_kernel<D, T, MERGE, 128>), gb, dim3(512), 0, stream, p);
    const dim3 gc((unsigned)p.kv_rows);
    const bool first = c == 0, final = c == L.nchunks - 1;
    if (first && final) hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, D, MERGE, true, true>), gc, dim3(512), 0, stream, p);
    else if (first) hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, D, MERGE, true, false>), gc, dim3(512), 0, stream, p);
    else if (final) hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, D, MERGE, false, true>), gc, dim3(512), 0, stream, p);
    else hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, D, MERGE, false, false>), gc, dim3(512), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int D, typename T>
static hipError_t run_bwd_d(const SfaBwdParams& p, const BwdPlan& L, bool merge, hipStream_t stream) {
  return merge ? run_bwd_chunks<D, T, true>(p, L, stream) : run_bwd_chunks<D, T, false>(p, L, stream);
}

int sfa_bwd_run(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, const void* d_out, const void* out, const float* softmax_max,
                const float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                void* d_query, void* d_query_rope, void* d_key, void* d_key_rope, void* d_value,
                int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t sparse_count,
                int64_t q_rows, int64_t kv_rows, int32_t sparse_block_size, int32_t sparse_mode,
                int64_t pre_tokens, int64_t next_tokens, int32_t layout, int32_t dtype, float scale_value,
                void* workspace, hipStream_t stream) {
  const bool merge = d_value == nullptr;
  const BwdPlan L = bwd_plan(q_rows, kv_rows, n1, d, sparse_count * (int64_t)sparse_block_size, merge, 2);
  unsigned char* ws = (unsigned char*)workspace;
  SfaBwdParams p;
  p.q = query;
  p.qr = query_rope;
  p.k = key;
  p.kr = key_rope;
  p.idx = sparse_indices;
  p.dout = d_out;
  p.out = out;
  p.smax = softmax_max;
  p.ssum = softmax_sum;
  p.act_q = actual_seq_q;
  p.act_k = actual_seq_kv;
  p.block_table = nullptr;
  p.dq = d_query;
  p.dqr = d_query_rope;
  p.dk = d_key;
  p.dkr = d_key_rope;
  p.dv = d_value;
  p.rows = q_rows;
  p.kv_rows = kv_rows;
  p.row0 = 0;
  p.nrows = 0;
  p.batch = (int32_t)batch;
  p.s1 = (int32_t)s1;
  p.s2 = (int32_t)s2;
  p.n1 = (int32_t)n1;
  p.K = (int32_t)sparse_count;
  p.bs = sparse_block_size;
  p.mode = sparse_mode;
  p.band_pre = band_clamp(pre_tokens);
  p.band_next = band_clamp(next_tokens);
  p.layout_q = layout;
  p.layout_kv = layout;
  p.max_blocks = 0;
  p.page_size = 1;
  p.hp = (int32_t)L.hp;
  p.kposp = (int32_t)L.kposp;
  p.nc = (int32_t)L.nc;
  p.scale = scale_value;
  p.scale_log2 = scale_value * kLog2e;
  p.cnt = (int32_t*)(ws + L.cnt);
  p.offs = (int32_t*)(ws + L.offs);
  p.acc = (float*)(ws + L.acc);
  p.nval = (int32_t*)(ws + L.nval);
  p.list = (int32_t*)(ws + L.list);
  p.rank = (int32_t*)(ws + L.rank);
  p.dsp = (void*)(ws + L.dsp);
  p.rec = (_Float16*)(ws + L.rec);
  p.rexp = (int16_t*)(ws + L.rexp);
  if (q_rows == 0) {
    // no query rows: every key gradient is zero (the reduce kernel writes
    // zeros for tokens without records)
    const int64_t zb = (kv_rows + 1 + 255) / 256;
    hipLaunchKernelGGL(bwd_zero_kernel, dim3((unsigned)zb), dim3(256), 0, stream, p.offs, kv_rows + 1);
    DSA_HIP(hipGetLastError());
  }
  hipError_t e;
  const bool bf = dtype == DSA_DTYPE_BF16;
  if (q_rows == 0) {
    const dim3 gc((unsigned)kv_rows);
    auto zero_out = [&](auto tag) {
      using T = decltype(tag);
      if (d == 128) {
        if (merge) hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, 128, true, true, true>), gc, dim3(512), 0, stream, p);
        else hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, 128, false, true, true>), gc, dim3(512), 0, stream, p);
      } else if (d == 256) {
        if (merge) hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, 256, true, true, true>), gc, dim3(512), 0, stream, p);
        else hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, 256, false, true, true>), gc, dim3(512), 0, stream, p);
      } else {
        if (merge) hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, 512, true, true, true>), gc, dim3(512), 0, stream, p);
        else hipLaunchKernelGGL((sfa_bwd_reduce_kernel<T, 512, false, true, true>), gc, dim3(512), 0, stream, p);
      }
      return hipGetLastError();
    };
    e = bf ? zero_out(bf16{}) : zero_out(f16{});
  } else if (d == 128) {
    e = bf ? run_bwd_d<128, bf16>(p, L, merge, stream) : run_bwd_d<128, f16>(p, L, merge, stream);
  } else if (d == 256) {
    e = bf ? run_bwd_d<256, bf16>(p, L, merge, stream) : run_bwd_d<256, f16>(p, L, merge, stream);
  } else {
    e = bf ? run_bwd_d<512, bf16>(p, L, merge, stream) : run_bwd_d<512, f16>(p, L, merge, stream);
  }
  DSA_HIP(e);
  return DSA_OK;
}

}  // namespace dsa
