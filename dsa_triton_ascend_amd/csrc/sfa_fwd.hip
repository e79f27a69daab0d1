// Sparse flash attention forward for gfx950 (MLA-absorb, MQA).
//
// Semantics follow the reference kernel `_sfa_kernel`
// (sparse_flash_attention_triton.py:150-332): a token of query row (b, s1) is
// attended iff its id is not -1, id < threshold and id < act_k, where
// threshold = act_k (mode 0) or act_k - act_q + s1 + 1 (mode 3), and the row
// is active iff s1 < act_q and threshold > 0 (247-254, 270-272); scores are
// (q_nope.k_nope + q_rope.k_rope) * scale in fp32; value = key[:, :D];
// softmax_max / softmax_sum are the row max and sum of exp(score - max)
// (326-332).  Paged KV (block_table), TND rows and block-wise ids are
// resolved in the kernel instead of on the host
// (sparse_flash_attention_triton.py:345-421).
//
// Design (one workgroup = one query row, all heads; 4 waves x 32 heads):
//  * The row's index range is compacted into an LDS list of physical KV rows
//    (invalid ids dropped), so ragged / -1 padded rows cost nothing.
//  * Tiles of 32 tokens are gathered HBM -> registers -> LDS (16-byte loads,
//    double-buffered: the next tile's loads are in flight during the current
//    tile's MFMAs).  Token rows are stored with an XOR chunk swizzle.
//  * Each wave keeps its 32 heads of Q (D + 64 columns, bf16) in registers
//    as MFMA B operands and its O^T accumulator [D x 32] in fp32 registers.
//  * S^T = K . Q^T on v_mfma_f32_16x16x32 (K rows from LDS, ds_read_b128):
//    the result layout puts one head per lane column, so the online softmax
//    (exp2 domain) is lane-local plus a 4-lane butterfly, and P^T is already
//    in B-operand layout for the second product.
//  * O^T += V^T . P^T with V^T fragments read straight from the row-major K
//    tile by ds_read_b64_tr_b16 (the transposing LDS read of gfx950).
//  * When there are fewer rows than CUs the row's tokens are split across
//    workgroups (all on one XCD) and a combine kernel merges the partial
//    (O, max, sum) triples.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "sfa_common.h"

namespace dsa {

struct SfaFwdParams {
  const void* q;
  const void* qr;
  const void* k;
  const void* kr;
  const int32_t* idx;
  const int32_t* act_q;
  const int32_t* act_k;
  const int32_t* block_table;
  void* out;
  float* smax;
  float* ssum;
  // split partials (splits > 1): part_o[s, r, h, :] = O_s / (l_s * scale_s)
  // in fp16, scale_s = 2^e >= max |O_s / l_s| (so |values| < 1: fp16 keeps
  // 11 bits for the largest ones); part_ml[s, r, h] = {reference max (log2
  // units), l_s, exact max (log2 units), scale_s}
  _Float16* part_o;
  float* part_ml;
  int64_t rows;
  int64_t kv_rows;
  int32_t batch, s1, s2, n1, K;
  int32_t bs;  // sparse_block_size
  int32_t mode, layout_q, layout_kv;
  int64_t band_pre, band_next;  // pre_tokens / next_tokens clamped to +-kBandOpen
  int32_t max_blocks, page_size;
  int32_t splits, rows_per_xcd, pos_per_split;
  float scale_log2;
  int32_t return_lse;  // 0: no statistics, 1: the statistics, 2: zeros
};

constexpr int kSfaTile = 32;
constexpr int kSfaMaxList = 2048;
// P carries a bf16 lo part (the P.V product then has ~16 bits of P) only
// while a workgroup attends fewer tokens than this; from here on P is
// rounded once to bf16, as the reference kernel rounds it
// (sparse_flash_attention_triton.py:313-323).  The rounding error of O is
// then ~2^-9 |v| / sqrt(3 n_eff) with n_eff the effective number of tokens
// of the softmax, far below the fp32-golden tolerance (atol 2e-3) at these
// lengths, while for a handful of tokens it is not.
constexpr int kLoSplitMinTokens = 256;
constexpr float kRefSlack = 64.f;  // log2 units
// Smallest exponent of a split partial's scale 2^e: a partial whose largest
// |O / l| is below 2^kPartMinExp (tiny values) keeps the scale 2^-120, so
// the stored multiplier inv * 2^-e (inv <= 1: l counts the reference-max
// token) stays finite and the stored values stay below 1.
constexpr int kPartMinExp = -120;

// Zero row for padding slots of the 64-bit gather path (the buffer path
// gets zeros from the hardware range check instead).
__device__ __attribute__((aligned(16))) unsigned char g_sfa_zero_row[1024];

// One 16-byte-per-lane DMA from global memory straight into LDS: lane L's
// 16 bytes land at lds_base + 16*L (LDS address taken from M0).  Issued via
// inline asm so that the compiler does not drain all outstanding DMA before
// every LDS read; the tile loop waits with explicit vmcnt counts instead.
__device__ __forceinline__ void dma_buf16(unsigned lds_base, int voff, __amdgpu_buffer_rsrc_t rsrc) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_base), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void dma_glb16(unsigned lds_base, const void* gaddr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_base), "v"(gaddr) : "memory");
}
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// HT = head tiles (of 16 heads) per wave, NW = waves; a workgroup covers
// NW*HT*16 heads.
// BUF: gather with buffer loads (32-bit offsets, key tensors under 2 GiB;
// the hardware range check yields the zero rows); otherwise 64-bit global
// addresses with an explicit zero row.
// CH: the split's position range may exceed kSfaMaxList and is compacted
// and run in chunks.  A separate instantiation: the chunk loop around the
// tile loop costs the D = 512 kernel registers it does not have (it spills),
// so ranges that fit one list run the kernel without it.
template <int D, typename T, int HT, int NW, bool BUF, bool CH>
__global__ __launch_bounds__(NW * 64, 1) void sfa_fwd_kernel(SfaFwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr bool kSplitP = __is_same(T, bf16);
  constexpr int DR = 64;
  constexpr int KS = (D + DR) / 32;  // GEMM1 k-steps
  constexpr int KSN = D / 32;        // of which from the nope part
  constexpr int NDT = D / 16;        // GEMM2 d-tiles
  constexpr int TILE = kSfaTile;
  constexpr int NOPE_BYTES = TILE * D * 2;
  constexpr int BUF_BYTES = NOPE_BYTES + TILE * DR * 2;
  constexpr int NBUF = 3;                    // DMA ring: tiles t+1, t+2 in flight during t
  constexpr int CPT = D / 8;                 // 16-byte chunks per nope row
  constexpr int TPI = 64 / CPT;              // nope tokens per wave-wide DMA (1 KB)
  // Every wave issues NI nope DMAs (1 KB each) per tile, and waves 0..3
  // one rope DMA (8 tokens x 128 B) each.  An LDS-DMA holds its wave at
  // issue while the CU's gather path is busy; spread over all waves, the
  // SIMD's other wave runs MFMAs meanwhile.
  constexpr int NI = TILE / TPI / NW;
  constexpr int NTHR = NW * 64;
  // LDS layout: the NBUF tile buffers are interleaved in 1 KB blocks (one
  // DMA each) so that a buffer index only adds a small immediate to a read
  // address: nope block k (tokens k*TPI..) of buffer b at (k*NBUF + b) KB,
  // rope block k (tokens 8k..8k+7) of buffer b at ROPE0 + (k*NBUF + b) KB.
  constexpr int ROPE0 = NBUF * NOPE_BYTES;
  auto nope_off = [](int tk, int b) { return ((tk / TPI) * NBUF + b) * 1024 + (tk % TPI) * (D * 2); };
  auto rope_off = [](int tk, int b) { return ROPE0 + ((tk >> 3) * NBUF + b) * 1024 + (tk & 7) * (DR * 2); };
  static_assert(TILE == 32 && (NW == 4 || NW == 8) && NI >= 1, "tile/wave layout");
  constexpr int HEADS_PER_WG = NW * HT * 16;
  constexpr int QL = 4;        // Q k-steps staged in LDS
  constexpr int KQR = KS - QL; // Q k-steps held in registers
  static_assert(KQR >= 0 && KS - KSN <= QL, "Q staging covers the rope part");

  __shared__ __attribute__((aligned(16))) unsigned char smem[NBUF * BUF_BYTES];
  __shared__ int s_list[kSfaMaxList + kSfaTile];
  // The last QL k-steps of Q (the rope part and the end of the nope part)
  // of the workgroup's heads, QL * 64 bytes per head (nope swizzle): read
  // from LDS by GEMM1's last k-steps instead of held in registers
  __shared__ __attribute__((aligned(16))) unsigned char s_q[HEADS_PER_WG * QL * 64];
  __shared__ int s_wcnt[NW];
  __shared__ RowInfo s_ri;  // the row's lengths, for compacting chunks after the first

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;  // lane within 16-lane group
  const int lg = lane >> 4;  // 16-lane group

  // ---- block -> (row, split, head group); a row's blocks share an XCD ----
  const int hgroups = (p.n1 + HEADS_PER_WG - 1) / HEADS_PER_WG;
  const int bid = blockIdx.x;
  const int jj = bid >> 3;
  const int hg = jj % hgroups;
  const int jr = jj / hgroups;
  const int64_t row = (int64_t)(bid & 7) * p.rows_per_xcd + jr / p.splits;
  const int split = jr % p.splits;
  if (row >= p.rows) return;

  const RowInfo ri = sfa_row_info(p, (int)row);
  if (tid == 0) s_ri = ri;
  const int32_t* idx_row = p.idx + row * p.K;
  const int total_pos = p.K * p.bs;
  const int p0 = split * p.pos_per_split;
  const int p1 = min(total_pos, p0 + p.pos_per_split);

  const int head0 = hg * HEADS_PER_WG + wave * HT * 16;
  const bool wave_active = head0 < p.n1;

  // ---- Q fragments (B operand of S^T = K.Q^T): lane -> head li, k = 8*lg.. ----
  // Q fragments: k-steps < KQR in registers, the last QL in LDS (loaded
  // first, stored to LDS once the register part's loads are out)
  V8 qf[HT][KQR > 0 ? KQR : 1];
  u32x4 qlv[HT][QL];
  const u32x4 z4 = {0u, 0u, 0u, 0u};
  auto q_chunk = [&](int64_t hsafe, int ks) -> u32x4 {
    if (ks < KSN) return *(const u32x4*)((const T*)p.q + hsafe * D + ks * 32 + lg * 8);
    return *(const u32x4*)((const T*)p.qr + hsafe * DR + (ks - KSN) * 32 + lg * 8);
  };
  auto load_q = [&]() {
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      const int head = head0 + ht * 16 + li;
      const bool hv = head < p.n1;
      const int64_t hsafe = row * p.n1 + (hv ? head : 0);
#pragma unroll
      for (int m = 0; m < QL; ++m) qlv[ht][m] = hv ? q_chunk(hsafe, KQR + m) : z4;
    }
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      const int head = head0 + ht * 16 + li;
      const bool hv = head < p.n1;
      const int64_t hsafe = row * p.n1 + (hv ? head : 0);
#pragma unroll
      for (int ks = 0; ks < KQR; ++ks) qf[ht][ks] = as_v8<V8>(hv ? q_chunk(hsafe, ks) : z4);
    }
  };
  // A wave with no index positions to resolve (the split has fewer than
  // 64 * wave positions) loads its Q before the compaction: a wave's loads
  // complete in issue order, so Q loads issued ahead of the index loads
  // would make the index chain wait for them, and those issued after it
  // start late.
  const bool q_early = wave_active && (int64_t)wave * 64 >= (int64_t)(p1 - p0);
  if (q_early) load_q();

  // ---- compact attended positions into s_list (stable order) ----
  // The split's positions are taken in chunks of at most kSfaMaxList: a
  // chunk is compacted into s_list and its tiles are run before the next
  // chunk is compacted; the online-softmax state and the O accumulators
  // carry over in registers, so a long range needs no extra split.
  // The first round's index entries are loaded first.  A PA_BSND row's
  // block table is then staged in the unused tail of s_list (loaded while
  // the index loads are in flight), so that resolving a page costs an LDS
  // read instead of a second dependent global load.  Only the waves that
  // resolve positions load it: the others have their Q loads in flight,
  // ahead of anything they would issue now.
  const int n_chunks = p1 > p0 ? (CH ? (p1 - p0 + kSfaMaxList - 1) / kSfaMaxList : 1) : 0;
  const int first_id = p0 + tid < p1 ? sfa_load_id(p, idx_row, p0 + tid) : -1;
  const int32_t* tab = nullptr;
  if (p.layout_kv == DSA_LAYOUT_PA_BSND) {
    const int32_t* gtab = p.block_table + (int64_t)ri.b * p.max_blocks;
    tab = gtab;
    if ((p1 - p0) + p.max_blocks <= kSfaMaxList) {
      int* s_tab = s_list + (kSfaMaxList + TILE - p.max_blocks);
      const int nct = min(NTHR, ((p1 - p0 + 63) / 64) * 64);
      if (tid < nct)
        for (int i = tid; i < p.max_blocks; i += nct) s_tab[i] = gtab[i];
      lds_barrier();
      tab = s_tab;
    }
  }
  int n_valid = 0, n_tiles = 0;
  // Compacts chunk c (every wave takes part; the barriers also order the
  // list's reuse after the previous chunk's tiles).  Chunk 0 resolves with
  // the values at hand; later chunks (CH kernels only) re-derive the row's
  // position, lengths and index pointer from blockIdx, the kernel arguments
  // and s_ri instead of holding them in registers across the tile loop.
  auto compact_range = [&](int cb, int ce, const RowInfo& rc, const int32_t* irow, const int32_t* tb,
                           bool first) {
    n_valid = 0;
    for (int c0 = cb; c0 < ce; c0 += NTHR) {
      int pos = c0 + tid;
      int phys = 0;
      bool valid = false;
      // the index load does not wait for the row's lengths (act_q / act_k)
      const int id = (first && c0 == cb) ? first_id : (pos < ce ? sfa_load_id(p, irow, pos) : -1);
      if (rc.active && pos < ce) valid = sfa_resolve_id(p, rc, id, pos, &phys, tb);
      unsigned long long m = __ballot(valid);
      if (lane == 0) s_wcnt[wave] = __popcll(m);
      lds_barrier();
      int off = n_valid;
      int tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const int cw = s_wcnt[w];
        off += (w < wave) ? cw : 0;
        tot += cw;
      }
      if (valid) s_list[off + __popcll(m & ((1ull << lane) - 1ull))] = phys;
      n_valid += tot;
      lds_barrier();
    }
    // pad the list to a whole tile with -1 so tile loads index it unconditionally
    if (tid < TILE) s_list[n_valid + tid] = -1;
    lds_barrier();
    n_tiles = (n_valid + TILE - 1) / TILE;
  };
  auto compact = [&](int c) {
    if (c == 0) {
      compact_range(p0, min(p1, p0 + kSfaMaxList), ri, idx_row, tab, true);
      return;
    }
    int bl = blockIdx.x;
    asm volatile("" : "+s"(bl));
    const int jr2 = (bl >> 3) / hgroups;
    const int64_t row2 = (int64_t)(bl & 7) * p.rows_per_xcd + jr2 / p.splits;
    const int q0 = (jr2 % p.splits) * p.pos_per_split;
    const int q1 = min(p.K * p.bs, q0 + p.pos_per_split);
    const RowInfo rc = s_ri;
    const int32_t* tb = p.layout_kv == DSA_LAYOUT_PA_BSND ? p.block_table + (int64_t)rc.b * p.max_blocks : nullptr;
    const int cb = q0 + c * kSfaMaxList;
    compact_range(cb, min(q1, cb + kSfaMaxList), rc, p.idx + row2 * p.K, tb, false);
  };
  if (n_chunks > 0) compact(0);

  // ---- tile gather: global -> LDS by DMA, swizzled rows ----
  // nope: DMA i of wave w covers tokens (i*NW + w)*TPI .. +TPI, lane L holds
  // chunk L % CPT of token tk0 + L / CPT and loads source chunk
  // (L % CPT) ^ nope_swz(tk), so that LDS chunk c holds chunk c ^ nope_swz.
  // rope: wave w < 4 covers tokens 8w .. 8w+7, lane L -> token 8w + L/8.
  const unsigned smem_base = (unsigned)(uintptr_t)smem;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const bool rope_wave = wave_s < 4;
  const int wiss = wave_s & 3;  // rope block of waves 0..3
  // wave-uniform DMA destinations: nope block (j*NW + wave), rope block wiss
  const unsigned smem_wave = smem_base + nope_off(wave_s * TPI, 0);
  const unsigned smem_rope_wave = smem_base + rope_off(wiss * 8, 0) - rope_off(0, 0);
  __amdgpu_buffer_rsrc_t rsrc_k, rsrc_r;
  if constexpr (BUF) {
    rsrc_k = __builtin_amdgcn_make_buffer_rsrc((void*)p.k, (short)0, (int)(p.kv_rows * D * 2), 0x00020000);
    rsrc_r = __builtin_amdgcn_make_buffer_rsrc((void*)p.kr, (short)0, (int)(p.kv_rows * DR * 2), 0x00020000);
  }
  // DMA j < NI of a wave loads nope block (j*NW + wave); DMA NI (waves
  // 0..3) loads rope block wiss.  A tile past the end (phys = -1
  // everywhere) loads zeros and touches no memory.  With one token per nope
  // DMA (D = 512) the row id is wave-uniform and kept in a scalar register.
  constexpr int NDMA = NI + 1;  // DMA slots per wave (the last: rope, waves 0..3)
  auto dma_phys = [&](int t, bool live, int j) -> int {
    const int tk = j < NI ? (j * NW + wave_s) * TPI + lane / CPT : wiss * 8 + (lane >> 3);
    int v = s_list[t * TILE + tk];  // -1 past n_valid / for -1 pages
    if (TPI == 1 && j < NI) v = __builtin_amdgcn_readfirstlane(v);
    return live && (j < NI || rope_wave) ? v : -1;
  };
  auto dma_issue = [&](int j, int phys, int b) {
    if (j < NI) {
      const int tk = (j * NW + wave_s) * TPI + lane / CPT;
      const int ch = (lane % CPT) ^ nope_swz(tk);
      const unsigned dst = smem_wave + nope_off(j * NW * TPI, b);
      if constexpr (BUF) {
        dma_buf16(dst, phys >= 0 ? phys * (D * 2) + ch * 16 : (int)0x80000000, rsrc_k);
      } else {
        const void* src = phys >= 0 ? (const void*)((const unsigned char*)p.k + (int64_t)phys * (D * 2) + ch * 16)
                                    : (const void*)(g_sfa_zero_row + ch * 16);
        dma_glb16(dst, src);
      }
    } else if (rope_wave) {
      const int tk = wiss * 8 + (lane >> 3);
      const int ch = (lane & 7) ^ rope_swz(tk);
      const unsigned dst = smem_rope_wave + rope_off(0, b);
      if constexpr (BUF) {
        dma_buf16(dst, phys >= 0 ? phys * (DR * 2) + ch * 16 : (int)0x80000000, rsrc_r);
      } else {
        const void* src = phys >= 0 ? (const void*)((const unsigned char*)p.kr + (int64_t)phys * (DR * 2) + ch * 16)
                                    : (const void*)(g_sfa_zero_row + ch * 16);
        dma_glb16(dst, src);
      }
    }
  };
  // whole tile at once (prologue and gather-only waves); the s_list reads
  // all go first: the DMA asm is a compiler memory barrier, so a read placed
  // between two DMAs would wait for its own LDS round trip
  auto issue_tile = [&](int t, int b) {
    int ph[NDMA];
#pragma unroll
    for (int j = 0; j < NDMA; ++j) ph[j] = dma_phys(t, true, j);
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dma_issue(j, ph[j], b);
  };
  // the same for any t: a tile past the end loads zeros
  auto issue_tile_or_zero = [&](int t, int b) {
    const bool live = t < n_tiles;
    int ph[NDMA];
#pragma unroll
    for (int j = 0; j < NDMA; ++j) ph[j] = dma_phys(live ? t : 0, live, j);
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dma_issue(j, ph[j], b);
  };
  // Barrier sequence, identical for every wave: per tile one barrier, then
  // one vote barrier, and (only if the vote is set) a second pass of tiles.
  // Tile t is waited for (vmcnt) before its barrier and tile t+2 is issued
  // after it, into the buffer tile t-1 used (all waves are past it).  Each
  // wave issues its NI (+1) loads per tile (zeros past the end), so the
  // vmcnt counts hold.
  auto gather_loop_prologue = [&]() {
    if (n_tiles > 0) issue_tile(0, 0);
    if (n_tiles > 1) issue_tile(1, 1);
  };
  auto tile_sync = [&](int t) {
    if (t + 1 >= n_tiles) wait_vmcnt<0>();
    else if (rope_wave) wait_vmcnt<NI + 1>();
    else wait_vmcnt<NI>();
    lds_barrier();
  };
  auto next_buf = [](int b) { return b == 0 ? NBUF - 1 : b - 1; };

  // The first two tiles go out before the Q loads, so that their gather
  // and the Q traffic are in flight together (the Q loads' own waits then
  // also cover these older DMAs, which only makes them earlier).
  gather_loop_prologue();

  if (!wave_active) {
    // waves without heads (N1 < HEADS_PER_WG) only take their share of the
    // gather, with the same barrier and load sequence as the other waves
    auto gather_only = [&](bool prologue) {
      if (prologue) gather_loop_prologue();
      for (int t0 = 0; t0 < n_tiles; t0 += NBUF)
#pragma unroll
        for (int b = 0; b < NBUF; ++b) {
          const int t = t0 + b;
          if (t >= n_tiles) break;
          tile_sync(t);
          issue_tile_or_zero(t + 2, next_buf(b));
        }
      wait_vmcnt<0>();
    };
    gather_only(false);
    if constexpr (CH)
      for (int c = 1; c < n_chunks; ++c) {
        compact(c);
        gather_only(true);
      }
    if (__syncthreads_or(0)) {
      if constexpr (CH) {
        for (int c = 0; c < (n_chunks > 0 ? n_chunks : 1); ++c) {
          if (n_chunks > 1) compact(c);
          gather_only(true);
        }
      } else {
        gather_only(true);
      }
    }
    return;
  }

  if (!q_early) load_q();

  // staged Q fragment (head li of head tile ht, chunk 4m + lg) at
  // ql_base ^ (m << 6) + ht * (16 * QL * 64)
  auto ql_base = [&](int ln) {
    const int l = ln & 15, g = ln >> 4;
    return (wave_s * HT * 16 + l) * (QL * 64) + ((g ^ nope_swz(l)) * 16);
  };
  {
    const int qb = ql_base(lane);
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int m = 0; m < QL; ++m) *(u32x4*)(s_q + ((qb ^ (m << 6)) + ht * (16 * QL * 64))) = qlv[ht][m];
  }

  f32x4 acc_o[NDT][HT];
  float m_ref[HT], m_true[HT], l_run[HT];
  // m_ref: reference max (log2 units) that P and O are taken relative to.
  // It is fixed by the first tile with a visible token and never raised
  // inside the tile loop (raising it would rescale O, which the register
  // allocator can only do by cycling the accumulator through VGPRs every
  // tile).  P = 2^(s - m_ref) may therefore exceed 1; up to 2^kRefSlack is
  // exact in fp32/bf16.  A head whose max exceeds m_ref + kRefSlack sets
  // `overflow`, and the row is recomputed once with m_ref = exact max.
  // m_true tracks the exact max for the returned statistics.
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    m_ref[ht] = -INFINITY;
    m_true[ht] = -INFINITY;
    l_run[ht] = 0.f;  // lane-partial sum of 2^(s - m_ref)
  }
  bool overflow = false;

  // ---- per-lane LDS byte offsets ----
  // GEMM1 A fragment: token tk = tt*16 + li, chunk ks*4 + lg.  Row starts
  // are multiples of 256 bytes and the swizzle only XORs the low four chunk
  // bits, so chunk (4m + lg) ^ swz lies at g1 ^ (m << 6) (m = ks mod 4) plus
  // 256 bytes per further group of four k-steps; rope chunks (4m + lg) ^ swz
  // at g1r ^ (m << 6).  Tokens 16..31 share the swizzle of tokens 0..15 and
  // sit a constant distance further on.  The XORs are recomputed per tile
  // from one base each (the bases are re-derived through an empty asm so the
  // compiler cannot hoist fourteen loop-invariant addresses into registers).
  // The per-lane bases are recomputed from the lane id at every use (a few
  // VALU ops): kept live across the tile loop they would be spilled, and a
  // spill reload waits for all outstanding loads, the tile DMAs included.
  auto fresh_lane = []() {
    int ln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(ln));
    return ln;
  };
  auto g1_base = [&](int ln) { const int l = ln & 15, g = ln >> 4; return nope_off(l, 0) + ((g ^ nope_swz(l)) * 16); };
  auto g1r_base = [&](int ln) { const int l = ln & 15, g = ln >> 4; return rope_off(l, 0) + ((g ^ rope_swz(l)) * 16); };
  constexpr int G1_TT = nope_off(16, 0) - nope_off(0, 0);
  constexpr int G1R_TT = rope_off(16, 0) - rope_off(0, 0);
  // GEMM2 transposed reads: row r1 = 4*lg + li/4 (and r1 + 16, same swizzle),
  // chunk dt*2 + (li&3)/2, 8-byte half (li&1): chunk (2m | h) ^ swz is at
  // g2 ^ (m << 5) for m = dt mod 8, plus 256 bytes per further eight d-tiles.
  auto g2_base = [&](int ln) {
    const int l = ln & 15, g = ln >> 4;
    const int r1 = g * 4 + (l >> 2);
    const int h = (l & 3) >> 1;
    return nope_off(r1, 0) + ((h ^ nope_swz(r1)) * 16) + (l & 1) * 8;
  };
  constexpr int G2_ROW16 = (16 / TPI) * NBUF * 1024;  // row r1 -> r1 + 16
  constexpr int NS1 = KS * 2;  // GEMM1 steps (k-step x token tile)
  // fragments in flight: with two waves per SIMD the other wave covers LDS
  // latency, and the registers are needed for the accumulators
  constexpr int PF1 = NW == 8 ? 4 : (HT == 1 ? 8 : 4);  // GEMM1
  constexpr int PF2 = NW == 8 ? 4 : (HT == 1 ? 8 : (D >= 512 ? 2 : 4));  // GEMM2

  // LDS fragment readers for buffer b
  auto a1 = [&](int g1b, int g1rb, int b, int st) -> u32x4 {
    const int ks = st >> 1, tt = st & 1;
    if (ks < KSN) return *(const u32x4*)(smem + ((g1b ^ ((ks & 3) << 6)) + tt * G1_TT + b * 1024 + (ks >> 2) * 256));
    return *(const u32x4*)(smem + ((g1rb ^ ((ks - KSN) << 6)) + tt * G1R_TT + b * 1024));
  };
  auto a2 = [&](int g2b, int b, int dt) -> V8 {
    const unsigned char* p1 = smem + ((g2b ^ ((dt & 7) << 5)) + b * 1024 + (dt >> 3) * 256);
    const bf16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1);
    const bf16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p1 + G2_ROW16));
    const i16x4 w1 = __builtin_bit_cast(i16x4, v1);
    const i16x4 w2 = __builtin_bit_cast(i16x4, v2);
    const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
    return __builtin_bit_cast(V8, w);
  };
  // s_list entries of tile tn (zeros past the end) for this wave's DMAs
  auto dma_plan = [&](int tn, int (&dph)[NDMA]) {
    const bool live = tn < n_tiles;
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dph[j] = dma_phys(live ? tn : 0, live, j);
  };

  // ---- GEMM1 of tile t (buffer b): S^T[32 tok x HT*16 heads] ----
  // With DMA, this wave's loads of tile tn into buffer bn go out evenly
  // spaced over the steps, so that the address unit drains while the MFMAs
  // run.
  auto gemm1 = [&](int t, int b, f32x4 (&acc_s)[2][HT], auto with_dma, int tn, int bn) {
    const int ln = fresh_lane();
    const int g1b = g1_base(ln), g1rb = g1r_base(ln), qlb = ql_base(ln);
    // staged Q fragments, read two k-steps ahead of use
    V8 ql[HT][QL];
    auto ql_read = [&](int m) {
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
        ql[ht][m] = as_v8<V8>(*(const u32x4*)(s_q + ((qlb ^ (m << 6)) + ht * (16 * QL * 64))));
    };
    constexpr bool kDma = decltype(with_dma)::value;
    int dph[NDMA];
    if constexpr (kDma) dma_plan(tn, dph);
    constexpr int DSTEP = NS1 / NDMA;  // GEMM1 steps per DMA slot
    static_assert(DSTEP >= 2, "DMA slots inside GEMM1");
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) acc_s[tt][ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
    u32x4 fa[PF1];
#pragma unroll
    for (int i = 0; i < PF1; ++i) fa[i] = a1(g1b, g1rb, b, i);
#pragma unroll
    for (int m = 0; m < QL && KQR + m < 2; ++m) ql_read(m);
#pragma unroll
    for (int st = 0; st < NS1; ++st) {
      const int ks = st >> 1, tt = st & 1;
      if (tt == 0 && ks + 2 >= KQR && ks + 2 < KS && ks + 2 - KQR >= 0) ql_read(ks + 2 - KQR);
      const V8 av = as_v8<V8>(fa[st % PF1]);
      if (st + PF1 < NS1) fa[st % PF1] = a1(g1b, g1rb, b, st + PF1);
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
        acc_s[tt][ht] = E::mfma(av, ks < KQR ? qf[ht][ks < KQR ? ks : 0] : ql[ht][ks < KQR ? 0 : ks - KQR], acc_s[tt][ht]);
      if constexpr (kDma)
        if (st % DSTEP == 2 && st / DSTEP < NDMA) dma_issue(st / DSTEP, dph[st / DSTEP], bn);
      // keeps the prefetched fragment reads where they are: without it the
      // scheduler sinks each read next to its MFMA to save registers, and
      // every MFMA then waits out a full LDS round trip
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- softmax numerators of tile t and O^T += V^T . P^T (buffer b) ----
  auto sm_gemm2 = [&](int t, int b, f32x4 (&acc_s)[2][HT], auto with_lo) {
    constexpr bool kLo = kSplitP && decltype(with_lo)::value;
    const int g2b = g2_base(fresh_lane());
    // first V^T fragments go out before the softmax arithmetic
    V8 fv[PF2];
#pragma unroll
    for (int i = 0; i < PF2; ++i) fv[i] = a2(g2b, b, i);

    // P^T is split into bf16 hi + lo parts for bf16 I/O (fp16 keeps 11 bits
    // in one part) while the workgroup attends few tokens: the P.V product
    // then carries ~16 bits of P (see kLoSplitMinTokens).
    V8 pf[HT], pf_lo[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      float tmax = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = t * TILE + tt * 16 + lg * 4 + r;
          float v = acc_s[tt][ht][r] * p.scale_log2;
          v = tok < n_valid ? v : -INFINITY;
          acc_s[tt][ht][r] = v;
          tmax = fmaxf(tmax, v);
        }
      }
      tmax = xgroup_max(tmax);
      m_true[ht] = fmaxf(m_true[ht], tmax);
      if (m_ref[ht] == -INFINITY) m_ref[ht] = tmax;
      overflow |= tmax > m_ref[ht] + kRefSlack;
      V8 hi, lo;
      float lsum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // m_ref == -inf only while no token is visible: all s are -inf too
        const float e = m_ref[ht] == -INFINITY ? 0.f : fast_exp2(acc_s[j >> 2][ht][j & 3] - m_ref[ht]);
        lsum += e;
        const T h = E::from_f32(e);
        hi[j] = h;
        lo[j] = E::from_f32(e - E::to_f32(h));
      }
      l_run[ht] += lsum;
      pf[ht] = hi;
      pf_lo[ht] = lo;
    }

#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const V8 av = fv[dt % PF2];
      if (dt + PF2 < NDT) fv[dt % PF2] = a2(g2b, b, dt + PF2);
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
        acc_o[dt][ht] = E::mfma(av, pf[ht], acc_o[dt][ht]);
        if constexpr (kLo) acc_o[dt][ht] = E::mfma(av, pf_lo[ht], acc_o[dt][ht]);
      }
      __builtin_amdgcn_sched_barrier(0);  // PF2 fragments stay in flight
    }
  };

  using DmaSpread = std::integral_constant<bool, true>;

  // Tile t: wait for its loads, barrier, GEMM1 (every wave loads its share
  // of tile t+2 into the buffer tile t-1 used, spaced over the steps: every
  // workgroup runs the same schedule, and bursts would queue at the memory
  // system), softmax, GEMM2.  (A two-group ping-pong schedule, GEMM1 of one
  // group beside softmax + GEMM2 of the other, measured slower here: the
  // per-wave LDS read rate, not MFMA issue, bounds each phase.)
  auto run_tiles = [&](bool prologue, auto with_lo) {
    if (prologue) gather_loop_prologue();
    for (int t0 = 0; t0 < n_tiles; t0 += NBUF)
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        const int t = t0 + b;
        if (t >= n_tiles) break;
        tile_sync(t);
        f32x4 sc[2][HT];
        gemm1(t, b, sc, DmaSpread{}, t + 2, next_buf(b));
        sm_gemm2(t, b, sc, with_lo);
      }
    wait_vmcnt<0>();  // tail loads of tiles past the end
  };
  using LoOn = std::integral_constant<bool, true>;
  using LoOff = std::integral_constant<bool, false>;

#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) acc_o[dt][ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // chunk 0 is compacted and its first tiles are in flight; later chunks
  // are compacted here and issue their own first tiles
  for (int c = 0; c < (CH && n_chunks > 0 ? n_chunks : 1); ++c) {
    if (CH && c > 0) compact(c);
    if (kSplitP && n_valid >= kLoSplitMinTokens) run_tiles(c > 0, LoOff{});
    else run_tiles(c > 0, LoOn{});
  }
  if (__syncthreads_or(overflow ? 1 : 0)) {
    // rare: some head's score exceeded the reference by 2^kRefSlack; redo
    // the row with the exact maxima found by the first pass
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      m_ref[ht] = m_true[ht];
      l_run[ht] = 0.f;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) acc_o[dt][ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // rare second pass: always with the lo part
    for (int c = 0; c < (CH && n_chunks > 0 ? n_chunks : 1); ++c) {
      if (CH && n_chunks > 1) compact(c);
      run_tiles(true, LoOn{});
    }
  }

  // ---- epilogue ----
  // per head tile: total sum, statistics, and for split partials the fp16
  // scale 2^ex >= max |O / l| of the head
  float mul[HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    const int head = head0 + ht * 16 + li;
    const float l_tot = xgroup_sum(l_run[ht]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    int ex = 0;
    if (p.splits > 1) {
      float a = 0.f;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) a = fmaxf(a, fabsf(acc_o[dt][ht][r]));
      a = xgroup_max(a) * inv;
      if (a > 0.f) (void)frexpf(a, &ex);  // a < 2^ex
      ex = ex < kPartMinExp ? kPartMinExp : ex;
    }
    mul[ht] = ldexpf(inv, -ex);
    if (head < p.n1 && lg == 0) {
      const int64_t orow = row * p.n1 + head;
      if (p.splits == 1) {
        if (p.return_lse) {
          const bool any = p.return_lse == 1 && l_tot > 0.f;
          p.smax[orow] = any ? m_true[ht] * kLn2 : 0.f;
          p.ssum[orow] = any ? l_tot * fast_exp2(m_ref[ht] - m_true[ht]) : 0.f;
        }
      } else {
        const int64_t prow = (int64_t)split * p.rows * p.n1 + orow;
        const f32x4 ml = {m_ref[ht], l_tot, m_true[ht], ldexpf(1.f, ex)};
        *(f32x4*)(p.part_ml + prow * 4) = ml;
      }
    }
  }
  // O rows (output in T, or split partials in fp16) are staged through this
  // wave's own LDS region, half of D at a time (the tile ring is idle now),
  // so that global stores are whole 16-byte-per-lane row segments rather
  // than 8-byte pieces of 16 different rows.
  constexpr int HALF = D / 2;
  constexpr int SROW = HALF * 2 + 16;  // padded staging row (bytes)
  constexpr int ROWS = HT * 16;
  constexpr int CPR = HALF * 2 / 16;   // 16-byte chunks per staged row
  constexpr int ITER = ROWS * CPR / 64;
  static_assert(NW * ROWS * SROW <= NBUF * BUF_BYTES && ITER * 64 == ROWS * CPR, "epilogue staging");
  typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
  typedef T T4 __attribute__((ext_vector_type(4)));
  unsigned char* stg = smem + wave * (ROWS * SROW);
  const bool to_out = p.splits == 1;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int dq = 0; dq < NDT / 2; ++dq) {
        const f32x4 v = acc_o[hh * (NDT / 2) + dq][ht] * mul[ht];
        u16x4 w;
        if (to_out) {
          const T4 o = {E::from_f32(v[0]), E::from_f32(v[1]), E::from_f32(v[2]), E::from_f32(v[3])};
          w = __builtin_bit_cast(u16x4, o);
        } else {
          const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
          w = __builtin_bit_cast(u16x4, o);
        }
        *(u16x4*)(stg + (ht * 16 + li) * SROW + (dq * 16 + lg * 4) * 2) = w;
      }
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int c = i * 64 + lane;
      const int r = c / CPR, col = c % CPR;
      const u32x4 val = *(const u32x4*)(stg + r * SROW + col * 16);
      const int head = head0 + r;
      if (head < p.n1) {
        const int64_t orow = row * p.n1 + head;
        unsigned char* dst = to_out ? (unsigned char*)p.out + orow * (D * 2)
                                    : (unsigned char*)(p.part_o + ((int64_t)split * p.rows * p.n1 + orow) * D);
        *(u32x4*)(dst + hh * (HALF * 2) + col * 16) = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// D = 512 kernel with O^T split by column slice: HG (64 or 128) heads per
// workgroup, 8 waves, and the two products divided among the waves in
// different ways, so that each LDS fragment is read by fewer waves.
//  * S^T = K . Q^T: wave w takes head tile w % (HG/16) (16 heads); with 64
//    heads also token half w / 4 (16 of the tile's 32 tokens, 18 MFMAs per
//    tile; each K fragment read by two waves instead of eight), with 128
//    heads all 32 tokens (36 MFMAs, as in sfa_fwd_kernel).
//  * The softmax numerators P^T of the HG heads go through LDS, 64 bytes
//    per head (bf16 hi and, for short ranges, lo parts: at 64 heads in a
//    second buffer, at 128 heads through the same buffer after the hi part).
//  * O^T += V^T . P^T: wave w owns columns 64w .. 64w + 63 of all HG heads
//    (HG accumulator registers); each V^T fragment is read by one wave and
//    serves HG/16 head tiles (sfa_fwd_kernel reads every V^T fragment in
//    each of its 8 waves).
// 64 heads is the decode (token-split) configuration: per token and head
// the LDS reads drop by about 25 % against sfa_fwd_kernel, and the split
// partials halve (4 splits of 64 heads instead of 8 of 128 at B = 32: 17
// instead of 34 MB written and read back).  The price is a second gather of
// every KV row, by the row's other head group: both run on one XCD, so HBM
// reads stay the same (L2 serves the second), but each CU's gather path,
// whose DMA issue is the loop's limiter, carries twice the bytes.  The
// token halves of a head share one reference max, taken from the first
// tile's two half maxima through one LDS exchange.  128 heads is the
// configuration of every other D = 512 launch (prefill).
// ---------------------------------------------------------------------------
constexpr int kSfaDsHeads = 64;

template <int D, typename T, int HG, bool BUF, bool CH>
__global__ __launch_bounds__(512, 1) void sfa_fwd_ds_kernel(SfaFwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr bool kSplitP = __is_same(T, bf16);
  constexpr int NW = 8;
  constexpr int NTHR = NW * 64;
  constexpr int HGT = HG / 16;       // head tiles of the workgroup
  constexpr int TG = NW / HGT;       // token groups of GEMM1 (2 or 1)
  constexpr int NTT = 2 / TG;        // 16-token sub-tiles per GEMM1 wave
  constexpr int DR = 64;
  constexpr int KS = (D + DR) / 32;  // GEMM1 k-steps
  constexpr int KSN = D / 32;
  constexpr int NDW = D / NW / 16;   // GEMM2 d-tiles per wave
  constexpr int TILE = kSfaTile;
  constexpr int NOPE_BYTES = TILE * D * 2;
  constexpr int BUF_BYTES = NOPE_BYTES + TILE * DR * 2;
  constexpr int NBUF = 3;
  constexpr int CPT = D / 8;
  constexpr int TPI = 64 / CPT;
  constexpr int NI = TILE / TPI / 4;
  constexpr int ROPE0 = NBUF * NOPE_BYTES;
  auto nope_off = [](int tk, int b) { return ((tk / TPI) * NBUF + b) * 1024 + (tk % TPI) * (D * 2); };
  auto rope_off = [](int tk, int b) { return ROPE0 + ((tk >> 3) * NBUF + b) * 1024 + (tk & 7) * (DR * 2); };
  static_assert(D == 512 && TPI == 1 && NI == 8 && NDW == 4 && (HG == 64 || HG == 128), "D = 512 layout");
  constexpr int QL = 4;
  constexpr int KQR = KS - QL;
  constexpr int PROW = TILE * 2;  // bytes of one head's P^T row
  // P buffers: hi and lo at 64 heads; at 128 heads one (the LDS is full),
  // the lo part goes through it after the hi part
  constexpr int NPB = (kSplitP && HG == 64) ? 2 : 1;

  __shared__ __attribute__((aligned(16))) unsigned char smem[NBUF * BUF_BYTES];
  __shared__ int s_list[kSfaMaxList + kSfaTile];
  __shared__ __attribute__((aligned(16))) unsigned char s_q[HG * QL * 64];
  // P^T of the tile: row h (64 bytes) holds head h's 32 numerators, token
  // 16*tt + 4*g + r in slot 8*g + 4*tt + r, 16-byte chunk g stored at
  // g ^ ((h >> 2) & 3); the lo parts follow the hi parts
  __shared__ __attribute__((aligned(16))) unsigned char s_p[NPB * HG * PROW];
  // per-head statistics: token groups' maxima (at 64 heads: first tile,
  // then exact) and sums, reference maxima, each wave's max |O|, output
  // scales.  At 128 heads they live in s_p, which is idle after the tiles
  // (and no maxima are exchanged during them).
  constexpr int NSTAT = 2 * TG * HG + HG + NW * HG + HG;
  static_assert(HG == 64 || NSTAT * 4 <= NPB * HG * PROW, "statistics in the P buffer");
  __shared__ float s_stat_own[HG == 64 ? NSTAT : 1];
  float* const s_mx = HG == 64 ? s_stat_own : (float*)s_p;  // [TG][HG]
  float* const s_lsum = s_mx + TG * HG;                      // [TG][HG]
  float* const s_mref = s_lsum + TG * HG;                    // [HG]
  float* const s_am = s_mref + HG;                           // [NW][HG]
  float* const s_mul = s_am + NW * HG;                       // [HG]
  __shared__ int s_wcnt[NW];
  __shared__ RowInfo s_ri;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;

  const int hgroups = (p.n1 + HG - 1) / HG;
  const int bid = blockIdx.x;
  const int jj = bid >> 3;
  const int hg = jj % hgroups;
  const int jr = jj / hgroups;
  const int64_t row = (int64_t)(bid & 7) * p.rows_per_xcd + jr / p.splits;
  const int split = jr % p.splits;
  if (row >= p.rows) return;

  const RowInfo ri = sfa_row_info(p, (int)row);
  if (tid == 0) s_ri = ri;
  const int32_t* idx_row = p.idx + row * p.K;
  const int total_pos = p.K * p.bs;
  const int p0 = split * p.pos_per_split;
  const int p1 = min(total_pos, p0 + p.pos_per_split);

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int hq = wave_s % HGT;  // GEMM1 head tile
  const int th = wave_s / HGT;  // GEMM1 token half (64 heads), 0 (128 heads)
  const int head1 = hg * HG + hq * 16;

  // ---- Q fragments of the GEMM1 head tile (both token halves hold them) ----
  V8 qf[KQR];
  u32x4 qlv[QL];
  const u32x4 z4 = {0u, 0u, 0u, 0u};
  auto q_chunk = [&](int64_t hsafe, int ks) -> u32x4 {
    if (ks < KSN) return *(const u32x4*)((const T*)p.q + hsafe * D + ks * 32 + lg * 8);
    return *(const u32x4*)((const T*)p.qr + hsafe * DR + (ks - KSN) * 32 + lg * 8);
  };
  auto load_q = [&]() {
    const int head = head1 + li;
    const bool hv = head < p.n1;
    const int64_t hsafe = row * p.n1 + (hv ? head : 0);
    if (th == 0) {
#pragma unroll
      for (int m = 0; m < QL; ++m) qlv[m] = hv ? q_chunk(hsafe, KQR + m) : z4;
    }
#pragma unroll
    for (int ks = 0; ks < KQR; ++ks) qf[ks] = as_v8<V8>(hv ? q_chunk(hsafe, ks) : z4);
  };
  // ---- compaction of the split's positions (as in sfa_fwd_kernel) ----
  const int n_chunks = p1 > p0 ? (CH ? (p1 - p0 + kSfaMaxList - 1) / kSfaMaxList : 1) : 0;
  // the index entries of the first chunk, all loaded up front (one memory
  // round trip instead of one per compaction step)
  constexpr int kIdPre = kSfaMaxList / NTHR;
  int first_ids[kIdPre];
  {
    const int ce0 = min(p1, p0 + kSfaMaxList);
#pragma unroll
    for (int u = 0; u < kIdPre; ++u) {
      const int pos = p0 + u * NTHR + tid;
      first_ids[u] = pos < ce0 ? sfa_load_id(p, idx_row, pos) : -1;
    }
  }
  const int32_t* tab = nullptr;
  const bool paged = p.layout_kv == DSA_LAYOUT_PA_BSND;
  const int32_t* gtab = paged ? p.block_table + (int64_t)ri.b * p.max_blocks : nullptr;
  const bool stage_tab = paged && (p1 - p0) + p.max_blocks <= kSfaMaxList;
  const int nct = min(NTHR, ((p1 - p0 + 63) / 64) * 64);
  const int tab0 = stage_tab && tid < nct && tid < p.max_blocks ? gtab[tid] : 0;
  // Q is issued after the compaction's inputs (row lengths, index entries,
  // the first block-table entries): vector memory operations complete in
  // order, so the compaction waits for those alone, and Q's latency overlaps
  // the compaction and the first tiles' DMA issue (decode 40.1 -> 39.9 us
  // against Q after the DMA issue)
  asm volatile("" ::: "memory");
  load_q();
  if (paged) {
    tab = gtab;
    if (stage_tab) {
      int* s_tab = s_list + (kSfaMaxList + TILE - p.max_blocks);
      if (tid < nct) {
        if (tid < p.max_blocks) s_tab[tid] = tab0;
        for (int i = tid + nct; i < p.max_blocks; i += nct) s_tab[i] = gtab[i];
      }
      lds_barrier();
      tab = s_tab;
    }
  }
  int n_valid = 0, n_tiles = 0;
  auto compact_range = [&](int cb, int ce, const RowInfo& rc, const int32_t* irow, const int32_t* tb,
                           bool first) {
    n_valid = 0;
    for (int c0 = cb; c0 < ce; c0 += NTHR) {
      int pos = c0 + tid;
      int phys = 0;
      bool valid = false;
      int id;
      if (first) {
        const int it = (c0 - cb) / NTHR;
        id = first_ids[0];
#pragma unroll
        for (int u = 1; u < kIdPre; ++u) id = it == u ? first_ids[u] : id;
      } else {
        id = pos < ce ? sfa_load_id(p, irow, pos) : -1;
      }
      if (rc.active && pos < ce) valid = sfa_resolve_id(p, rc, id, pos, &phys, tb);
      unsigned long long m = __ballot(valid);
      if (lane == 0) s_wcnt[wave] = __popcll(m);
      lds_barrier();
      int off = n_valid;
      int tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const int cw = s_wcnt[w];
        off += (w < wave) ? cw : 0;
        tot += cw;
      }
      if (valid) s_list[off + __popcll(m & ((1ull << lane) - 1ull))] = phys;
      n_valid += tot;
      lds_barrier();
    }
    if (tid < TILE) s_list[n_valid + tid] = -1;
    lds_barrier();
    n_tiles = (n_valid + TILE - 1) / TILE;
  };
  auto compact = [&](int c) {
    if (c == 0) {
      compact_range(p0, min(p1, p0 + kSfaMaxList), ri, idx_row, tab, true);
      return;
    }
    int bl = blockIdx.x;
    asm volatile("" : "+s"(bl));
    const int jr2 = (bl >> 3) / hgroups;
    const int64_t row2 = (int64_t)(bl & 7) * p.rows_per_xcd + jr2 / p.splits;
    const int q0 = (jr2 % p.splits) * p.pos_per_split;
    const int q1 = min(p.K * p.bs, q0 + p.pos_per_split);
    const RowInfo rc = s_ri;
    const int32_t* tb = p.layout_kv == DSA_LAYOUT_PA_BSND ? p.block_table + (int64_t)rc.b * p.max_blocks : nullptr;
    const int cb = q0 + c * kSfaMaxList;
    compact_range(cb, min(q1, cb + kSfaMaxList), rc, p.idx + row2 * p.K, tb, false);
  };
  if (n_chunks > 0) compact(0);

  // ---- tile gather by LDS-DMA, spread over all eight waves ----
  // Nope DMA j < NIW of wave w loads the 1 KB row of token j*8 + w; waves
  // 0..3 also load the rope rows of tokens 8w .. 8w+7 (one DMA).  An LDS-DMA
  // of 1 KB occupies the CU's address unit for about 16 cycles, and a wave
  // that issues into a full queue stalls: issued by four waves, the tile's 36
  // DMAs held those waves back in every tile.
  constexpr int NIW = TILE / NW;
  const unsigned smem_base = (unsigned)(uintptr_t)smem;
  const bool rope_wave = wave_s < 4;
  __amdgpu_buffer_rsrc_t rsrc_k, rsrc_r;
  if constexpr (BUF) {
    rsrc_k = __builtin_amdgcn_make_buffer_rsrc((void*)p.k, (short)0, (int)(p.kv_rows * D * 2), 0x00020000);
    rsrc_r = __builtin_amdgcn_make_buffer_rsrc((void*)p.kr, (short)0, (int)(p.kv_rows * DR * 2), 0x00020000);
  }
  constexpr int NDMA = NIW + 1;  // DMA slots per wave (the last one: rope, waves 0..3)
  // The DMAs of tile t+2 go out during tile t: slots 0 .. G1D-1 between
  // the GEMM1 MFMAs, the rest between the GEMM2 MFMAs.  Issued in GEMM2
  // alone, the LDS-DMA issue stalls lengthened that phase (decode 41.0 ->
  // 40.3 us with two slots in GEMM1; prefill unchanged).
  constexpr int G1D = 2;
  static_assert(G1D >= 0 && G1D < NDMA, "DMA slots issued during GEMM1");
  auto dma_phys = [&](int t, bool live, int j) -> int {
    int v;
    if (j < NIW) v = __builtin_amdgcn_readfirstlane(s_list[t * TILE + j * NW + wave_s]);
    else v = rope_wave ? s_list[t * TILE + wave_s * 8 + (lane >> 3)] : -1;
    return live ? v : -1;
  };
  auto dma_issue = [&](int j, int phys, int b) {
    if (j < NIW) {
      const int tk = j * NW + wave_s;
      const int ch = lane ^ nope_swz(tk);
      const unsigned dst = smem_base + nope_off(tk, b);
      if constexpr (BUF) {
        dma_buf16(dst, phys >= 0 ? phys * (D * 2) + ch * 16 : (int)0x80000000, rsrc_k);
      } else {
        const void* src = phys >= 0 ? (const void*)((const unsigned char*)p.k + (int64_t)phys * (D * 2) + ch * 16)
                                    : (const void*)(g_sfa_zero_row + ch * 16);
        dma_glb16(dst, src);
      }
    } else if (rope_wave) {
      const int tk = wave_s * 8 + (lane >> 3);
      const int ch = (lane & 7) ^ rope_swz(tk);
      const unsigned dst = smem_base + rope_off(wave_s * 8, b);
      if constexpr (BUF) {
        dma_buf16(dst, phys >= 0 ? phys * (DR * 2) + ch * 16 : (int)0x80000000, rsrc_r);
      } else {
        const void* src = phys >= 0 ? (const void*)((const unsigned char*)p.kr + (int64_t)phys * (DR * 2) + ch * 16)
                                    : (const void*)(g_sfa_zero_row + ch * 16);
        dma_glb16(dst, src);
      }
    }
  };
  auto issue_tile = [&](int t, int b) {
    int ph[NDMA];
#pragma unroll
    for (int j = 0; j < NDMA; ++j) ph[j] = dma_phys(t, true, j);
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dma_issue(j, ph[j], b);
  };
  auto gather_loop_prologue = [&]() {
    if (n_tiles > 0) issue_tile(0, 0);
    if (n_tiles > 1) issue_tile(1, 1);
  };
  // a wave's DMAs of tile t+1 are its last NIW (+1) loads
  auto tile_sync = [&](int t) {
    if (t + 1 >= n_tiles) wait_vmcnt<0>();
    else if (rope_wave) wait_vmcnt<NIW + 1>();
    else wait_vmcnt<NIW>();
    lds_barrier();
  };
  auto next_buf = [](int b) { return b == 0 ? NBUF - 1 : b - 1; };
  gather_loop_prologue();

  auto ql_base = [&](int ln) {
    const int l = ln & 15, g = ln >> 4;
    return (hq * 16 + l) * (QL * 64) + ((g ^ nope_swz(l)) * 16);
  };
  if (th == 0) {
    const int qb = ql_base(lane);
#pragma unroll
    for (int m = 0; m < QL; ++m) *(u32x4*)(s_q + (qb ^ (m << 6))) = qlv[m];
  }

  f32x4 acc_o[NDW][HGT];
  // reference max (log2 units) shared by the token halves, fixed by the
  // first tile; exact max of this half; lane-partial sum of 2^(s - m_ref)
  float m_ref = -INFINITY, m_true = -INFINITY, l_run = 0.f;
  bool overflow = false;
  bool need_ref = true;

  auto fresh_lane = []() {
    int ln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(ln));
    return ln;
  };
  auto g1_base = [&](int ln) { const int l = ln & 15, g = ln >> 4; return nope_off(l, 0) + ((g ^ nope_swz(l)) * 16); };
  auto g1r_base = [&](int ln) { const int l = ln & 15, g = ln >> 4; return rope_off(l, 0) + ((g ^ rope_swz(l)) * 16); };
  constexpr int G1_TT = nope_off(16, 0) - nope_off(0, 0);
  constexpr int G1R_TT = rope_off(16, 0) - rope_off(0, 0);
  auto g2_base = [&](int ln) {
    const int l = ln & 15, g = ln >> 4;
    const int r1 = g * 4 + (l >> 2);
    const int h = (l & 3) >> 1;
    return nope_off(r1, 0) + ((h ^ nope_swz(r1)) * 16) + (l & 1) * 8;
  };
  constexpr int G2_ROW16 = (16 / TPI) * NBUF * 1024;
  // P^T chunk of lane ln in head tile 0 (B operand of GEMM2)
  auto p_base = [&](int ln) {
    const int l = ln & 15, g = ln >> 4;
    return l * PROW + ((g ^ ((l >> 2) & 3)) * 16);
  };
  auto a1 = [&](int g1b, int g1rb, int b, int ks, int tt) -> u32x4 {
    if (ks < KSN) return *(const u32x4*)(smem + ((g1b ^ ((ks & 3) << 6)) + tt * G1_TT + b * 1024 + (ks >> 2) * 256));
    return *(const u32x4*)(smem + ((g1rb ^ ((ks - KSN) << 6)) + tt * G1R_TT + b * 1024));
  };
  auto a2 = [&](int g2b, int b, int dt) -> V8 {
    const unsigned char* pp = smem + ((g2b ^ ((dt & 7) << 5)) + b * 1024 + (dt >> 3) * 256);
    const bf16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)pp);
    const bf16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(pp + G2_ROW16));
    const i16x4 w1 = __builtin_bit_cast(i16x4, v1);
    const i16x4 w2 = __builtin_bit_cast(i16x4, v2);
    const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
    return __builtin_bit_cast(V8, w);
  };
  auto dma_plan = [&](int tn, int (&dph)[NDMA]) {
    const bool live = tn < n_tiles;
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dph[j] = dma_phys(live ? tn : 0, live, j);
  };

  // ---- GEMM1: S^T [16 NTT tokens x 16 heads] of this wave's head tile ----
  // Two accumulators so consecutive MFMAs are independent: the two token
  // sub-tiles (128 heads) or even / odd k-steps (64 heads).  Step st is
  // k-step st / NTT of sub-tile st % NTT.  No scheduling barriers (the
  // compiler's interleaving of the fragment reads measured faster than the
  // fixed prefetch order at 64 heads).
  auto gemm1 = [&](int b, f32x4 (&s_out)[NTT], const int (&dph)[NDMA], int bn) {
    const int ln = fresh_lane();
    const int g1b = g1_base(ln), g1rb = g1r_base(ln), qlb = ql_base(ln);
    V8 ql[QL];
    auto ql_read = [&](int m) { ql[m] = as_v8<V8>(*(const u32x4*)(s_q + (qlb ^ (m << 6)))); };
    constexpr int NS = KS * NTT;
    constexpr int PF = NTT == 1 ? 6 : 4;
    auto a1s = [&](int st) { return a1(g1b, g1rb, b, st / NTT, NTT == 1 ? th : st % NTT); };
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    u32x4 fa[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) fa[i] = a1s(i);
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const int ks = st / NTT;
      if (st % NTT == 0 && ks + 2 >= KQR && ks + 2 < KS) ql_read(ks + 2 - KQR);
      const V8 av = as_v8<V8>(fa[st % PF]);
      if (st + PF < NS) fa[st % PF] = a1s(st + PF);
      acc[st & 1] = E::mfma(av, ks < KQR ? qf[ks < KQR ? ks : 0] : ql[ks < KQR ? 0 : ks - KQR], acc[st & 1]);
      if constexpr (G1D > 0) {
        constexpr int kStep1 = NS / G1D;
        if (st % kStep1 == kStep1 / 2 && st / kStep1 < G1D) dma_issue(st / kStep1, dph[st / kStep1], bn);
      }
      if constexpr (NTT == 2) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NTT == 1) s_out[0] = acc[0] + acc[1];
    else { s_out[0] = acc[0]; s_out[1] = acc[1]; }
  };

  // ---- softmax numerators of this wave's 16 NTT tokens x 16 heads -> s_p ----
  // token 16*tt + 4*lg + r of head 16*hq + li goes to slot 8*lg + 4*tt + r
  typedef T T4 __attribute__((ext_vector_type(4)));
  const int pw_off = (hq * 16 + li) * PROW + ((lg ^ ((li >> 2) & 3)) * 16);
  auto softmax_p = [&](int t, const f32x4 (&s)[NTT], auto with_lo, T4 (&lo_out)[NTT]) {
    constexpr bool kLo = kSplitP && decltype(with_lo)::value;
    float v[NTT][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < NTT; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tt = NTT == 1 ? th : u;
        const int tok = t * TILE + tt * 16 + lg * 4 + r;
        const float x = tok < n_valid ? s[u][r] * p.scale_log2 : -INFINITY;
        v[u][r] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = xgroup_max(tmax);
    m_true = fmaxf(m_true, tmax);
    if constexpr (TG == 2) {
      if (need_ref) {
        // the first tile of the pass: both halves take the max of the two
        if (lg == 0) s_mx[th * HG + hq * 16 + li] = tmax;
        lds_barrier();
        m_ref = fmaxf(s_mx[hq * 16 + li], s_mx[HG + hq * 16 + li]);
        // no finite score in the first tile (non-finite inputs): the first
        // pass contributes nothing and the row is redone with the exact max
        overflow |= m_ref == -INFINITY;
        need_ref = false;
      }
    } else {
      // the wave sees all of its heads' tokens: the reference max is the
      // first tile's with a visible score
      if (m_ref == -INFINITY) m_ref = tmax;
    }
    overflow |= tmax > m_ref + kRefSlack;
    float lsum = 0.f;
#pragma unroll
    for (int u = 0; u < NTT; ++u) {
      T4 hi, lo;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = m_ref == -INFINITY ? 0.f : fast_exp2(v[u][r] - m_ref);
        lsum += e;
        hi[r] = E::from_f32(e);
        lo[r] = E::from_f32(e - E::to_f32(hi[r]));
      }
      const int tt = NTT == 1 ? th : u;
      *(T4*)(s_p + pw_off + tt * 8) = hi;
      if constexpr (kLo) {
        if constexpr (NPB == 2) *(T4*)(s_p + HG * PROW + pw_off + tt * 8) = lo;
        else lo_out[u] = lo;
      }
    }
    l_run += lsum;
  };
  auto write_lo = [&](const T4 (&lo)[NTT]) {
#pragma unroll
    for (int u = 0; u < NTT; ++u) *(T4*)(s_p + pw_off + (NTT == 1 ? th : u) * 8) = lo[u];
  };

  // ---- GEMM2: O^T [64 columns x HG heads] += V^T . P^T ----
  // With DMA, this wave's remaining DMAs of tile t+2 (slots G1D.., into
  // buffer bn) go out between the MFMAs: every wave stalls on its DMA issue
  // for a while (the CU's gather path is shared), and here the other wave
  // of the SIMD has MFMAs to run meanwhile.  TWO: the lo part of P sits in
  // the second buffer and is multiplied in the same pass.
  V8 va[NDW];
  auto gemm2 = [&](int b, auto two, auto with_dma, const int (&dph)[NDMA], int bn) {
    constexpr bool kTwo = decltype(two)::value;
    constexpr bool kDma = decltype(with_dma)::value;
    const int ln = fresh_lane();
    const int pb = p_base(ln);
    if constexpr (kDma) {
      // the hi pass reads the wave's V^T fragments (kept for a lo pass)
      const int g2b = g2_base(ln);
#pragma unroll
      for (int j = 0; j < NDW; ++j) va[j] = a2(g2b, b, wave_s * NDW + j);
    }
    auto pread = [&](int ht, int part) { return as_v8<V8>(*(const u32x4*)(s_p + part * HG * PROW + pb + ht * 16 * PROW)); };
    V8 ph = pread(0, 0), pl = kTwo ? pread(0, 1) : ph;
#pragma unroll
    for (int ht = 0; ht < HGT; ++ht) {
      const V8 ch = ph, cl = pl;
      if (ht + 1 < HGT) {
        ph = pread(ht + 1, 0);
        if constexpr (kTwo) pl = pread(ht + 1, 1);
      }
#pragma unroll
      for (int j = 0; j < NDW; ++j) {
        acc_o[j][ht] = E::mfma(va[j], ch, acc_o[j][ht]);
        if constexpr (kTwo) acc_o[j][ht] = E::mfma(va[j], cl, acc_o[j][ht]);
        if constexpr (kDma) {
          constexpr int NR = NDMA - G1D;
          constexpr int kStep = HGT * NDW / NR;
          const int st = ht * NDW + j;
          if (st % kStep == 0 && st / kStep < NR) dma_issue(G1D + st / kStep, dph[G1D + st / kStep], bn);
        }
      }
    }
  };

  // Tile t: wait for its loads, barrier, GEMM1, softmax numerators to LDS,
  // barrier, GEMM2 (with the DMAs of tile t+2 into the buffer tile t-1
  // used); with one P buffer and the lo part, a barrier, the lo part into
  // the buffer, a barrier and its GEMM2.  The next tile's first barrier
  // orders the P^T reads before the next writes.
  using On = std::integral_constant<bool, true>;
  using Off = std::integral_constant<bool, false>;
  auto run_tiles = [&](bool prologue, auto with_lo) {
    constexpr bool kLo = kSplitP && decltype(with_lo)::value;
    if (prologue) gather_loop_prologue();
    for (int t0 = 0; t0 < n_tiles; t0 += NBUF)
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        const int t = t0 + b;
        if (t >= n_tiles) break;
        tile_sync(t);
        f32x4 sc[NTT];
        T4 lo[NTT];
        int dph[NDMA];
        dma_plan(t + 2, dph);
        gemm1(b, sc, dph, next_buf(b));
        softmax_p(t, sc, with_lo, lo);
        lds_barrier();
        if constexpr (kLo && NPB == 2) {
          gemm2(b, On{}, On{}, dph, next_buf(b));
        } else {
          gemm2(b, Off{}, On{}, dph, next_buf(b));
          if constexpr (kLo) {
            lds_barrier();
            write_lo(lo);
            lds_barrier();
            gemm2(b, Off{}, Off{}, dph, 0);
          }
        }
      }
    wait_vmcnt<0>();
  };
  using LoOn = On;
  using LoOff = Off;

#pragma unroll
  for (int j = 0; j < NDW; ++j)
#pragma unroll
    for (int ht = 0; ht < HGT; ++ht) acc_o[j][ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < (CH && n_chunks > 0 ? n_chunks : 1); ++c) {
    if (CH && c > 0) compact(c);
    if (kSplitP && n_valid >= kLoSplitMinTokens) run_tiles(c > 0, LoOff{});
    else run_tiles(c > 0, LoOn{});
  }
  // exact maxima of the two halves (64 heads); the vote barrier orders them
  if constexpr (TG == 2)
    if (lg == 0) s_mx[th * HG + hq * 16 + li] = m_true;
  if (__syncthreads_or(overflow ? 1 : 0)) {
    if constexpr (TG == 2) m_ref = fmaxf(s_mx[hq * 16 + li], s_mx[HG + hq * 16 + li]);
    else m_ref = m_true;
    l_run = 0.f;
    need_ref = false;
#pragma unroll
    for (int j = 0; j < NDW; ++j)
#pragma unroll
      for (int ht = 0; ht < HGT; ++ht) acc_o[j][ht] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < (CH && n_chunks > 0 ? n_chunks : 1); ++c) {
      if (CH && n_chunks > 1) compact(c);
      run_tiles(true, LoOn{});
    }
  }

  // ---- epilogue ----
  // per head: total sum (token groups), statistics, and for split partials
  // the fp16 scale 2^ex >= max |O / l| over all columns (eight waves).  At
  // 128 heads the statistics overwrite s_p: every wave is past its last
  // GEMM2 (the vote barrier above).
  {
    const float lw = xgroup_sum(l_run);
    if (lg == 0) {
      s_lsum[th * HG + hq * 16 + li] = lw;
      if (th == 0) s_mref[hq * 16 + li] = m_ref;
      if constexpr (TG == 1) s_mx[hq * 16 + li] = m_true;
    }
    if (p.splits > 1) {
#pragma unroll
      for (int ht = 0; ht < HGT; ++ht) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < NDW; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) a = fmaxf(a, fabsf(acc_o[j][ht][r]));
        a = xgroup_max(a);
        if (lg == 0) s_am[wave * HG + ht * 16 + li] = a;
      }
    }
  }
  lds_barrier();
  if (tid < HG) {
    const int h = tid;
    const int head = hg * HG + h;
    const float l_tot = TG == 2 ? s_lsum[h] + s_lsum[HG + h] : s_lsum[h];
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float mt = TG == 2 ? fmaxf(s_mx[h], s_mx[HG + h]) : s_mx[h];
    const float mr = s_mref[h];
    int ex = 0;
    if (p.splits > 1) {
      float a = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) a = fmaxf(a, s_am[w * HG + h]);
      a *= inv;
      if (a > 0.f) (void)frexpf(a, &ex);
      ex = ex < kPartMinExp ? kPartMinExp : ex;
    }
    s_mul[h] = ldexpf(inv, -ex);
    if (head < p.n1) {
      const int64_t orow = row * p.n1 + head;
      if (p.splits == 1) {
        if (p.return_lse) {
          const bool any = p.return_lse == 1 && l_tot > 0.f;
          p.smax[orow] = any ? mt * kLn2 : 0.f;
          p.ssum[orow] = any ? l_tot * fast_exp2(mr - mt) : 0.f;
        }
      } else {
        const int64_t prow = (int64_t)split * p.rows * p.n1 + orow;
        const f32x4 ml = {mr, l_tot, mt, ldexpf(1.f, ex)};
        *(f32x4*)(p.part_ml + prow * 4) = ml;
      }
    }
  }
  lds_barrier();
  // O rows staged in the (idle) tile ring as [head][D] in the output type
  // (or fp16 partials), 64 heads at a time, then stored as whole rows, 16
  // bytes per lane
  constexpr int SROW = D * 2 + 16;
  constexpr int SH = 64;  // heads per staging round
  static_assert(SH * SROW <= NBUF * BUF_BYTES, "epilogue staging");
  typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
  const bool to_out = p.splits == 1;
  float mulv[HGT];
#pragma unroll
  for (int ht = 0; ht < HGT; ++ht) mulv[ht] = s_mul[ht * 16 + li];
#pragma unroll
  for (int hh = 0; hh < HG / SH; ++hh) {
    if (hh > 0) lds_barrier();  // the previous round's rows are stored
#pragma unroll
    for (int hl = 0; hl < SH / 16; ++hl) {
      const int ht = hh * (SH / 16) + hl;
#pragma unroll
      for (int j = 0; j < NDW; ++j) {
        const f32x4 v = acc_o[j][ht] * mulv[ht];
        u16x4 w;
        if (to_out) {
          const T4 o = {E::from_f32(v[0]), E::from_f32(v[1]), E::from_f32(v[2]), E::from_f32(v[3])};
          w = __builtin_bit_cast(u16x4, o);
        } else {
          const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
          w = __builtin_bit_cast(u16x4, o);
        }
        *(u16x4*)(smem + (hl * 16 + li) * SROW + (wave * (NDW * 16) + j * 16 + lg * 4) * 2) = w;
      }
    }
    lds_barrier();
    constexpr int CPR = D * 2 / 16;
    static_assert(SH * CPR % NTHR == 0, "store loop");
#pragma unroll
    for (int i = 0; i < SH * CPR / NTHR; ++i) {
      const int c = i * NTHR + tid;
      const int r = c / CPR, col = c % CPR;
      const u32x4 val = *(const u32x4*)(smem + r * SROW + col * 16);
      const int head = hg * HG + hh * SH + r;
      if (head < p.n1) {
        const int64_t orow = row * p.n1 + head;
        unsigned char* dst = to_out ? (unsigned char*)p.out + orow * (D * 2)
                                    : (unsigned char*)(p.part_o + ((int64_t)split * p.rows * p.n1 + orow) * D);
        *(u32x4*)(dst + col * 16) = val;
      }
    }
  }
}

// Merge per-split partials: one wave per (row, head).  Partial i holds
// O_i / l_i (as scale_i * stored value), l_i relative to its reference max
// r_i, and its exact max t_i (log2 units); the merged output is
// sum_i w_i O_i / l_i / sum_i w_i with w_i = 2^(r_i - M) l_i.
// Lane s reads the record of split s, the weights are formed on the lanes
// and broadcast with readlane, and each lane reads its D/64 columns of the
// splits.  With at most eight splits (every decode launch) all loads go out
// together; above that, the columns of eight splits at a time.
template <int D, typename T>
__global__ __launch_bounds__(256) void sfa_combine_kernel(SfaFwdParams p) {
  using E = Elem<T>;
  constexpr int PER = D / 64;
  typedef _Float16 hvec __attribute__((ext_vector_type(PER)));
  const int lane = threadIdx.x & 63;
  // (row, head) of this wave, with the forward launch's XCD mapping (rows
  // rows_per_xcd * x .. of XCD x = blockIdx & 7), so the partials a wave
  // reads were written through the same XCD's L2
  const int bpr = (p.n1 + 3) / 4;  // blocks per row
  const int jb = (int)(blockIdx.x >> 3);
  const int64_t crow = (int64_t)(blockIdx.x & 7) * p.rows_per_xcd + jb / bpr;
  const int chead = (jb % bpr) * 4 + (int)(threadIdx.x >> 6);
  if (crow >= p.rows || chead >= p.n1) return;
  const int64_t rh = crow * p.n1 + chead;
  const int64_t sstride = p.rows * p.n1;  // (row, head) records per split
  if (p.splits <= 8) {
    // every load up front (lane s < splits: the record of split s; all
    // lanes: their columns of every split), so the wave waits for one
    // memory round trip; the partials are read once (non-temporal)
    f32x4 ml = {-INFINITY, 0.f, -INFINITY, 0.f};
    if (lane < p.splits) ml = *(const f32x4*)(p.part_ml + ((int64_t)lane * sstride + rh) * 4);
    hvec v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < p.splits) v[u] = __builtin_nontemporal_load((const hvec*)(p.part_o + ((int64_t)u * sstride + rh) * D + lane * PER));
    const bool has = ml[1] > 0.f;
    const float mref8 = wave_max(has ? ml[0] : -INFINITY);
    const float mtrue8 = wave_max(has ? ml[2] : -INFINITY);
    float acc8[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) acc8[e] = 0.f;
    float L8 = 0.f;
    if (mref8 != -INFINITY) {
      const float w = has ? fast_exp2(ml[0] - mref8) * ml[1] : 0.f;
      const float wsc = w * ml[3];
      L8 = wave_sum(w);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (u >= p.splits) break;
        const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wsc), u));
        if (wu == 0.f) continue;  // split without attended tokens
#pragma unroll
        for (int e = 0; e < PER; ++e) acc8[e] += wu * (float)v[u][e];
      }
    }
    const float inv8 = L8 > 0.f ? 1.f / L8 : 0.f;
    T* op8 = (T*)p.out + rh * D + lane * PER;
#pragma unroll
    for (int j = 0; j < PER; ++j) op8[j] = E::from_f32(acc8[j] * inv8);
    if (p.return_lse && lane == 0) {
      const bool any = p.return_lse == 1 && L8 > 0.f;
      p.smax[rh] = any ? mtrue8 * kLn2 : 0.f;
      p.ssum[rh] = any ? L8 * fast_exp2(mref8 - mtrue8) : 0.f;
    }
    return;
  }
  float mref = -INFINITY, mtrue = -INFINITY;
  for (int s = lane; s < p.splits; s += 64) {
    const f32x4 ml = *(const f32x4*)(p.part_ml + ((int64_t)s * sstride + rh) * 4);
    if (ml[1] > 0.f) {
      mref = fmaxf(mref, ml[0]);
      mtrue = fmaxf(mtrue, ml[2]);
    }
  }
  mref = wave_max(mref);
  mtrue = wave_max(mtrue);
  float acc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) acc[j] = 0.f;
  float L = 0.f;
  if (mref != -INFINITY) {
    for (int s0 = 0; s0 < p.splits; s0 += 64) {
      const int s = s0 + lane;
      float w = 0.f, wsc = 0.f;
      if (s < p.splits) {
        const f32x4 ml = *(const f32x4*)(p.part_ml + ((int64_t)s * sstride + rh) * 4);
        if (ml[1] > 0.f) {
          w = fast_exp2(ml[0] - mref) * ml[1];
          wsc = w * ml[3];
        }
      }
      L += wave_sum(w);
      const int n = min(64, p.splits - s0);
      for (int j = 0; j < n; j += 8) {
        hvec v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (j + u < n)
            v[u] = *(const hvec*)(p.part_o + ((int64_t)(s0 + j + u) * sstride + rh) * D + lane * PER);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (j + u >= n) break;
          const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wsc), j + u));
          if (wu == 0.f) continue;  // split without attended tokens
#pragma unroll
          for (int e = 0; e < PER; ++e) acc[e] += wu * (float)v[u][e];
        }
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  T* op = (T*)p.out + rh * D + lane * PER;
#pragma unroll
  for (int j = 0; j < PER; ++j) op[j] = E::from_f32(acc[j] * inv);
  if (p.return_lse && lane == 0) {
    const bool any = p.return_lse == 1 && L > 0.f;
    p.smax[rh] = any ? mtrue * kLn2 : 0.f;
    p.ssum[rh] = any ? L * fast_exp2(mref - mtrue) : 0.f;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Waves and head tiles (of 16 heads) per wave of the 128-head kernel; every
// configuration covers 128 heads per workgroup, so one gathered KV row
// serves all heads of a row.  D=512 runs two waves per SIMD (8 x 16 heads):
// LDS reads from a single wave per SIMD are latency-bound, and 16 heads keep
// the O accumulator (128 registers) plus Q fragments within the 256
// registers of a half SIMD.
template <int D> struct SfaCfg {
  static constexpr int NW = D >= 512 ? 8 : 4;
  static constexpr int HT = D >= 512 ? 1 : 2;
};
constexpr int kSfaHeadsPerWg = 128;

// Token splits: when the (row, head group) units fill fewer than half the
// CUs, enough splits to fill them, with at least 256 positions per split.
// From half the CUs up one split per unit: two splits of half the work
// would take the same two rounds on the CUs, plus the merge.  A split's
// range has no length limit (it is compacted in chunks), so the split
// workspace is below (cus + units) <= 1.5 * cus partial rows of N1 heads
// (about 51 MB at 256 CUs, N1 = 128, D = 512).  The workspace query and the
// launch use the same count.
//
// Kernel choice: D = 512 launches that split tokens with 64-head workgroups
// run sfa_fwd_ds_kernel with 64 heads (decode: 44.8 us against 46.6 with
// 128 heads and twice the splits); other D = 512 launches run it with 128
// heads (each KV row gathered once per row; prefill 4.64 ms against 4.77
// for sfa_fwd_kernel); D < 512 runs sfa_fwd_kernel (128 heads).
static int sfa_fwd_plan_splits(int64_t rows, int64_t n1, int64_t total_pos, int heads_per_wg) {
  const int cus = device_cu_count();
  const int64_t units = rows * ((n1 + heads_per_wg - 1) / heads_per_wg);
  if (2 * units > cus) return 1;
  const int64_t want = (cus + units - 1) / units;
  const int64_t by_len = (total_pos + 255) / 256;
  const int64_t splits = want < by_len ? want : by_len;
  return splits < 1 ? 1 : (int)splits;
}

// ---------------------------------------------------------------------------
// Scratch of dsa_sfa_fwd_noalloc: the split partials live in this
// fixed-size device array instead of a caller's workspace, for callers that
// cannot allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc).  Every GPU the library runs on holds its own copy until the
// process ends.  64 MiB covers the split workspace of every shape on a
// 256-CU device (at most 1.5 * CUs partial rows of N1 <= 128 heads: about
// 51 MB at D = 512); larger needs are rejected.  Calls on one GPU share the
// array: concurrent calls on one device race.  Every partial a launch reads
// is written by the same launch, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
constexpr size_t kSfaScratchBytes = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[kSfaScratchBytes];

// Device address of `scratch` per device, looked up once per device with
// that device current.  The host-side name `scratch` is only a handle for
// the lookup; kernels get the looked-up address.
static std::atomic<void*> g_scratch_ptr[64];
static std::mutex g_scratch_mu;

size_t sfa_fwd_scratch_bytes() { return kSfaScratchBytes; }

int sfa_fwd_scratch(void** ptr) {
  int dev = -1;
  DSA_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("device ordinal %d out of range for the scratch table", dev);
    return DSA_ERR_UNSUPPORTED;
  }
  void* a = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!a) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    a = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!a) {
      DSA_HIP(hipGetSymbolAddress(&a, HIP_SYMBOL(scratch)));
      if (!a) {
        set_error("hipGetSymbolAddress returned a null address for the scratch array");
        return DSA_ERR_HIP;
      }
      g_scratch_ptr[dev].store(a, std::memory_order_release);
    }
  }
  *ptr = a;
  return DSA_OK;
}

enum SfaFwdKind { kFwdWide, kFwdDs64, kFwdDs128 };
static SfaFwdKind sfa_fwd_kind(int64_t rows, int64_t n1, int64_t d, int64_t total_pos) {
  if (d != 512 || (test_flags() & kTestFwdWide)) return kFwdWide;
  if (sfa_fwd_plan_splits(rows, n1, total_pos, kSfaDsHeads) > 1) return kFwdDs64;
  return kFwdDs128;
}
static int sfa_fwd_heads_per_wg(int64_t rows, int64_t n1, int64_t d, int64_t total_pos) {
  return sfa_fwd_kind(rows, n1, d, total_pos) == kFwdDs64 ? kSfaDsHeads : kSfaHeadsPerWg;
}

static size_t sfa_fwd_ws_for(int64_t splits, int64_t rows, int64_t n1, int64_t d) {
  if (splits <= 1) return 0;
  return (size_t)splits * rows * n1 * (d * sizeof(_Float16) + 4 * sizeof(float));
}

// At D = 512 the kernels that compact and run a split's positions in
// several pieces (a range above kSfaMaxList) run out of registers and spill
// (56 - 628 bytes per lane), so a D = 512 launch takes at least
// ceil(total_pos / kSfaMaxList) token splits and every workgroup's range
// fits the list in one piece (the combine kernel merges the splits).
// one_list = false keeps the splits that fill the CUs and lets the chunked
// kernel take long ranges: the no-alloc entry point falls back to it when
// the extra splits' partials would not fit its scratch, and so does any
// launch whose extra partials would pass kSfaOneListMaxWs.
constexpr size_t kSfaOneListMaxWs = 4ull << 30;
static int sfa_fwd_splits_for(int64_t rows, int64_t n1, int64_t d, int64_t total_pos, bool one_list) {
  const int fill = sfa_fwd_plan_splits(rows, n1, total_pos, sfa_fwd_heads_per_wg(rows, n1, d, total_pos));
  if (!one_list || d != 512 || (test_flags() & kTestFwdWide)) return fill;
  const int64_t need = (total_pos + kSfaMaxList - 1) / kSfaMaxList;
  if (need <= fill) return fill;
  if (sfa_fwd_ws_for(need, rows, n1, d) > kSfaOneListMaxWs) return fill;
  return (int)need;
}

int sfa_fwd_splits(int64_t rows, int64_t n1, int64_t d, int64_t total_pos, bool one_list) {
  return sfa_fwd_splits_for(rows, n1, d, total_pos, one_list);
}

size_t sfa_fwd_workspace_bytes(int64_t rows, int64_t n1, int64_t d, int64_t total_pos, bool one_list) {
  return sfa_fwd_ws_for(sfa_fwd_splits_for(rows, n1, d, total_pos, one_list), rows, n1, d);
}

template <int D, typename T>
static hipError_t launch_sfa_fwd(SfaFwdParams& p, SfaFwdKind kind, hipStream_t stream) {
  const int heads_per_wg = kind == kFwdDs64 ? kSfaDsHeads : kSfaHeadsPerWg;
  const int64_t rows_per_xcd = (p.rows + 7) / 8;
  p.rows_per_xcd = (int)rows_per_xcd;
  const int64_t blocks = 8 * rows_per_xcd * p.splits * ((p.n1 + heads_per_wg - 1) / heads_per_wg);
  const bool buf = p.kv_rows * (int64_t)D * 2 < (1ll << 31) && !(test_flags() & kTestForceGlobalGather);
  using C = SfaCfg<D>;
  static_assert(C::NW * C::HT * 16 == kSfaHeadsPerWg, "heads per workgroup");
  const bool chunked = p.pos_per_split > kSfaMaxList;
  const dim3 grid((unsigned)blocks), block(C::NW * 64);
  auto launch_ds = [&](auto hg) {
    constexpr int HG = decltype(hg)::value;
    if constexpr (D == 512) {
      if (buf && !chunked)
        hipLaunchKernelGGL((sfa_fwd_ds_kernel<D, T, HG, true, false>), grid, dim3(512), 0, stream, p);
      else if (buf)
        hipLaunchKernelGGL((sfa_fwd_ds_kernel<D, T, HG, true, true>), grid, dim3(512), 0, stream, p);
      else if (!chunked)
        hipLaunchKernelGGL((sfa_fwd_ds_kernel<D, T, HG, false, false>), grid, dim3(512), 0, stream, p);
      else
        hipLaunchKernelGGL((sfa_fwd_ds_kernel<D, T, HG, false, true>), grid, dim3(512), 0, stream, p);
    }
  };
  if (kind == kFwdDs64) {
    launch_ds(std::integral_constant<int, 64>{});
  } else if (kind == kFwdDs128) {
    launch_ds(std::integral_constant<int, 128>{});
  } else if (buf && !chunked)
    hipLaunchKernelGGL((sfa_fwd_kernel<D, T, C::HT, C::NW, true, false>), grid, block, 0, stream, p);
  else if (buf)
    hipLaunchKernelGGL((sfa_fwd_kernel<D, T, C::HT, C::NW, true, true>), grid, block, 0, stream, p);
  else if (!chunked)
    hipLaunchKernelGGL((sfa_fwd_kernel<D, T, C::HT, C::NW, false, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((sfa_fwd_kernel<D, T, C::HT, C::NW, false, true>), grid, block, 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  const int64_t cblocks = 8 * rows_per_xcd * ((p.n1 + 3) / 4);
  hipLaunchKernelGGL((sfa_combine_kernel<D, T>), dim3((unsigned)cblocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

int sfa_fwd_run(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, void* attention_out, float* softmax_max,
                float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                int64_t d, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                int64_t max_blocks, int64_t page_size, int32_t sparse_block_size,
                int32_t sparse_mode, int64_t pre_tokens, int64_t next_tokens, int32_t layout_query,
                int32_t layout_kv, int32_t dtype, float scale_value, int32_t return_lse, void* workspace,
                hipStream_t stream, bool one_list) {
  SfaFwdParams p;
  p.q = query;
  p.qr = query_rope;
  p.k = key;
  p.kr = key_rope;
  p.idx = sparse_indices;
  p.act_q = actual_seq_q;
  p.act_k = actual_seq_kv;
  p.block_table = block_table;
  p.out = attention_out;
  p.smax = softmax_max;
  p.ssum = softmax_sum;
  p.rows = q_rows;
  p.kv_rows = kv_rows;
  p.batch = (int32_t)batch;
  p.s1 = (int32_t)s1;
  p.s2 = layout_kv == DSA_LAYOUT_PA_BSND ? (int32_t)(max_blocks * page_size) : (int32_t)s2;
  p.n1 = (int32_t)n1;
  p.K = (int32_t)sparse_count;
  p.bs = sparse_block_size;
  p.mode = sparse_mode;
  p.band_pre = band_clamp(pre_tokens);
  p.band_next = band_clamp(next_tokens);
  p.layout_q = layout_query;
  p.layout_kv = layout_kv;
  p.max_blocks = (int32_t)max_blocks;
  p.page_size = (int32_t)page_size;
  const int64_t total_pos = sparse_count * (int64_t)sparse_block_size;
  const SfaFwdKind kind = sfa_fwd_kind(q_rows, n1, d, total_pos);
  p.splits = sfa_fwd_splits_for(q_rows, n1, d, total_pos, one_list);
  p.pos_per_split = (int32_t)((total_pos + p.splits - 1) / p.splits);
  p.part_o = nullptr;
  p.part_ml = nullptr;
  if (p.splits > 1) {
    p.part_o = (_Float16*)workspace;
    p.part_ml = (float*)(p.part_o + (size_t)p.splits * q_rows * n1 * d);
  }
  p.scale_log2 = scale_value * kLog2e;
  // 1: write the statistics; 2: write zeros to the caller's buffers (given
  // without return_lse), so that the caller needs no fill of its own
  p.return_lse = return_lse ? 1 : (softmax_max && softmax_sum ? 2 : 0);
  p.rows_per_xcd = 0;
  hipError_t e;
  if (dtype == DSA_DTYPE_BF16) {
    e = d == 512 ? launch_sfa_fwd<512, bf16>(p, kind, stream)
      : d == 256 ? launch_sfa_fwd<256, bf16>(p, kind, stream)
                 : launch_sfa_fwd<128, bf16>(p, kind, stream);
  } else {
    e = d == 512 ? launch_sfa_fwd<512, f16>(p, kind, stream)
      : d == 256 ? launch_sfa_fwd<256, f16>(p, kind, stream)
                 : launch_sfa_fwd<128, f16>(p, kind, stream);
  }
  if (e != hipSuccess) return hip_fail(e, "sfa_fwd launch");
  return DSA_OK;
}

}  // namespace dsa
