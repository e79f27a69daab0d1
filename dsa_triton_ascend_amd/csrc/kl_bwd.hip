// Sparse lightning-indexer KL-loss backward for gfx950.
//
// Semantics follow the reference kernels `_indexer_grad_kl_loss_kernel` and
// `_scatter_dkey_index_kernel` (sparse_lightning_indexer_grad_kl_loss_triton.py:
// 74-263, 266-317) and the golden `numpy_reference` (sli_grad_kl_loss_numpy.py:
// 16-152).  For every query row (b, s1) with s1 < act_q, over the first
// n = min(topK, max(act_k - act_q + s1 + 1, 0)) slots (kernel line 107), each
// slot's token clamped to [0, S2) with no -1 test (lines 58, 63, 300):
//   relu[g,k] = max(qi_g . ki_k, 0),  I[k] = sum_g w_g relu[g,k]     (119-136)
//   p[k] = (1/N1) sum_h exp(s[h,k] - max_h) / (sum_h + 1e-8),
//          s[h,k] = (q_h . k_k + qr_h . kr_k) * scale                 (145-177)
//   sI = exp(I - max I) / (sum exp + 1e-8), dI = sI - p               (180-207)
//   loss += sum_k P (log P - log Q), P = max(p, 1e-8), Q = max(sI, 1e-8) (208-216)
//   dW_g = sum_k dI relu[g,k]; dQi_g = sum_k dI w_g 1[relu>0] ki_k  (224-260)
//   dKi[token_k] += sum_g dI w_g 1[relu>0] qi_g                       (307-317)
//
// Design:
//  * kl_bwd_row_kernel: one workgroup of 8 waves per query row.  Pass A
//    streams tiles of 32 slots (K, K_rope, K_index rows gathered straight
//    into an LDS ring by LDS-DMA, the next tile's gather in flight during
//    the current tile's MFMAs).  Waves 0-3 compute: each scores 32 heads of
//    the teacher on the 32x32x16 MFMA (Q fragments resident in registers,
//    log2 of each head's softmax denominator in LDS) and sums their
//    probabilities per slot, then scores index heads 16*w .. +15 over the
//    tile.  Waves 4-7 issue the next tile's gather and reduce the previous
//    tile's partial sums into p and I.  I and p of the row stay in LDS.
//    Pass B is the softmax/KL over the row.  Pass C re-streams
//    K_index by LDS-DMA, pipelined over the tiles: waves 0-3 recompute a
//    tile's index scores (cheaper than storing Nidx1 x topK ReLUs), form
//    dS and accumulate dW, while waves 4-7 take the previous tile: dQi
//    (dQi^T = Ki^T . dS^T through the transposing LDS read) in registers,
//    and the per-slot dKi contributions c[k] = dS[:,k]^T . Qi, written to
//    their token's bucket as fp16 scaled by a per-row power of two.
//  * dKi without floating-point atomics: before the row kernel the slots are
//    bucketed by target token (an integer count that records each slot's
//    place, and a scan), the row kernel stores each contribution at its
//    place, so a token's contributions are consecutive, and a token's
//    contributions are summed in fixed point (each rounded to a grid 2^-e
//    and added as integer-valued doubles below 2^52), with the exponent
//    fixed by the largest row maximum among the token's slots (raised by
//    the row kernel with integer atomics on the float bits) and their count
//    (long tokens split over up to 16 waves whose partial sums meet in
//    int64 atomics): these additions are exact and associative, so the
//    result does not depend on the bucket order or the split and the output
//    is deterministic.
//  * The loss is written per row and summed by one workgroup in a fixed
//    order (the reference adds rows with an atomic).
#include "kl_generic.h"

namespace dsa {

struct KlParams {
  KlMap m;
  int32_t ring;   // pass A tile buffers in LDS (1 or 2)
  int32_t ringb;  // bytes of the LDS ring region: max(ring tile buffers, pass C's)
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
  // dKi contribution c of each slot (128 values), stored as fp16 c * 2^e_row
  // (e_row set from an a-priori bound of |c| over the row) at the slot's
  // place in its token's bucket: row offs[token] + rank[slot]
  _Float16* cbuf;
  float* rowmax;     // [rows] max |c| over the row's slots
  int32_t* rowexp;   // [rows] e_row
  const int32_t* offs;  // [tokens + 1] bucket starts
  const int32_t* rank;  // [rows * topK] the slot's place in its token's bucket (within its row chunk)
  const int32_t* cbase; // [chunks][tokens] the row chunk's start within each bucket, or null
  int32_t chunk_rows, tokens;
  int32_t* posrow;      // [rows * topK] row of the contribution at each bucket position
  uint32_t* tokmax;     // [tokens] largest row maximum among the token's slots (float bits)
  float* loss_part;  // [rows]
  int32_t n1, nidx, topk, w_dtype;
  float scale_log2;  // scale * log2(e)
};

constexpr int kKlTile = 32;
constexpr int kKlDi = 128;
constexpr int kKlWaves = 8;
constexpr int kKlMaxNidx = 64;
// the row's I, p and token arrays (12 bytes per slot) share the LDS with
// the static arrays (about 21 KB) and the ring region (at most 50 KB)
constexpr int kKlMaxTopk = 7168;
constexpr int kKlDsRow = kKlMaxNidx + 8;  // padded LDS row of dS^T (elements)
// Pass C's use of the ring region: four K_index tile buffers (32 rows of
// 128 bf16/fp16) and the dS^T hi / lo tiles of two consecutive tiles.
constexpr int kKlPcKiBytes = kKlTile * kKlDi * 2;
constexpr int kKlPcDsBytes = 2 * kKlTile * kKlDsRow * 2;
constexpr int kKlPcBufs = 4;
constexpr int kKlPcBytes = kKlPcBufs * kKlPcKiBytes + 2 * kKlPcDsBytes;

// Zero source row of the pass-A gather (slots past the row's end and
// tokens of -1 pages).
__device__ __attribute__((aligned(16))) unsigned char g_kl_zero_row[1024];

// One 16-byte-per-lane DMA from global memory straight into LDS: lane L's
// 16 bytes land at lds_base + 16*L (LDS address taken from M0).  Inline
// asm, so that the compiler does not drain the DMAs before every LDS read;
// the loop waits for them with an explicit vmcnt.
__device__ __forceinline__ void kl_dma16(unsigned lds_base, const void* gaddr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(gaddr) : "memory");
}

// Bytes of one pass-A tile buffer: K, K_rope and K_index rows of 32 slots.
template <int D, int DR>
constexpr int kl_tile_bytes() { return kKlTile * (D * 2 + DR * 2 + kKlDi * 2); }

template <int D, int DR, typename T>
__global__ __launch_bounds__(kKlWaves * 64, 1) void kl_bwd_row_kernel(KlParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int DI = kKlDi;
  constexpr int TILE = kKlTile;
  constexpr int NT = kKlWaves * 64;
  constexpr int KSN = D / 32, KSR = DR / 32, KS = KSN + KSR;
  constexpr int ROW = D * 2;            // K row bytes in LDS
  constexpr int IROW = DI * 2;          // K_index row bytes
  constexpr int CN = D / 8, CR = DR / 8, CI = DI / 8;  // 16-byte chunks per row
  // pass-A gather: every DMA moves 1 KB (64 lanes x 16 bytes) = TPK K rows,
  // 8 rope rows or TPI K_index rows
  constexpr int TPK = 64 / CN, TPI = 64 / CI;
  constexpr int KD = TILE / TPK, RD = DR > 0 ? TILE / 8 : 0, ID = TILE / TPI;
  static_assert(TPK * CN == 64 && TPI * CI == 64 && (DR == 0 || CR == 8), "gather assignment");
  // pass-C gather: one K_index chunk per thread
  static_assert(TILE * CI == NT, "pass C gather");
  constexpr int BUF_K = TILE * ROW, BUF_R = TILE * DR * 2;
  constexpr int BUF = kl_tile_bytes<D, DR>();
  constexpr bool kF16 = __is_same(T, f16);

  // per-wave partial sums of a pass-A tile, double-buffered by tile parity
  __shared__ __attribute__((aligned(16))) float s_red[2][kKlWaves][TILE];
  __shared__ __attribute__((aligned(16))) float s_redi[2][4][TILE];
  // [0, 8) and [8, 16): per-wave pass-B sums / maxima; [16]: fp16 weight
  // max; [17, 25): per-wave max |Qi|
  __shared__ float s_misc[3 * kKlWaves + 4];
  __shared__ __attribute__((aligned(16))) float s_m2p[128];  // pass A: per-head offset of the teacher exponent
  // the row's index queries (kKlMaxNidx heads, rows padded by 16 bytes so
  // that 16 heads' 16-byte reads hit distinct banks; heads >= Nidx1 zero)
  constexpr int QIR = DI + 8;
  __shared__ __attribute__((aligned(16))) T s_qi[kKlMaxNidx * QIR];
  // dynamic: the ring region (pass A's p.ring tile buffers of BUF bytes;
  // pass C's K_index tiles and dS^T tiles), then I (then dI) and p of the
  // row, and its clamped token rows
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dynb[];
  unsigned char* const ring = s_dynb;
  float* s_I = (float*)(s_dynb + p.ringb);
  float* s_p = s_I + p.topk;
  int* s_tok = (int*)(s_p + p.topk);

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int row = p.m.rows - 1 - (int)blockIdx.x;  // long causal rows first
  const KlRow ri = kl_row_info(p.m, row);
  const int n = ri.n;

  if (n <= 0) {
    // inactive or empty row: zero gradients, no loss (kernel lines 103-105)
    for (int e = tid; e < p.nidx * DI; e += NT) ((T*)p.dqi)[(int64_t)row * p.nidx * DI + e] = E::from_f32(0.f);
    for (int g = tid; g < p.nidx; g += NT) store_w(p.dw, (int64_t)row * p.nidx + g, p.w_dtype, 0.f);
    if (tid == 0) {
      p.loss_part[row] = 0.f;
      p.rowmax[row] = 0.f;
      p.rowexp[row] = 0;
    }
    return;
  }
  const int nt = (n + TILE - 1) / TILE;
  const u32x4 z4 = {0u, 0u, 0u, 0u};

  // ---- resident fragments ----
  // pass A teacher: waves 0-3 take heads 32*wave .. +31 on
  // v_mfma_f32_32x32x16 (A operand: head 32*wave + lane%32, k-step ks = d
  // 16*ks + 8*(lane/32) .. +7, nope k-steps then rope)
  constexpr int KS16 = (D + DR) / 16, KSN16 = D / 16;
  const bool twave = wave < 4;
  const bool wave_heads = twave && wave * 32 < p.n1;
  const int thead = wave * 32 + (lane & 31);
  const bool thv = twave && thead < p.n1;
  const int64_t throw_ = (int64_t)row * p.n1 + (thv ? thead : 0);
  V8 qf[KS16];
#pragma unroll
  for (int ks = 0; ks < KS16; ++ks) {
    const int d8 = (lane >> 5) * 8;
    u32x4 v = z4;
    if (thv) {
      if (ks < KSN16) v = *(const u32x4*)((const T*)p.q + throw_ * D + ks * 16 + d8);
      else v = *(const u32x4*)((const T*)p.qr + throw_ * DR + (ks - KSN16) * 16 + d8);
    }
    qf[ks] = as_v8<V8>(v);
  }
  // C register r of the 32x32 product is head 32*wave + 8*(r/4) + 4*(lane/32)
  // + r%4 (column: slot lane%32).  p = exp2(s*scale*log2e - m2 - log2(l +
  // 1e-8)): the max and the normalisation fold into one offset; +inf masks
  // heads >= N1
  // (kept in LDS, s_m2p[head], and read per tile)
  for (int h = tid; h < 128; h += NT) {
    const bool v = h < p.n1;
    const int64_t hr = (int64_t)row * p.n1 + (v ? h : 0);
    s_m2p[h] = v ? p.smax[hr] * kLog2e + __log2f(p.ssum[hr] + 1e-8f) : INFINITY;
  }
  // index heads 16*hg4 .. +15 (hg4 = wave mod 4), g = 16*hg4 + li.  Pass A
  // scores them on wave hg4 (both halves of the tile); pass C on waves hg4
  // (scores, dS, dW) and 4 + hg4 (dQi, contributions).
  const int hg4 = wave & 3;
  const bool ihg = hg4 * 16 < p.nidx;
  const bool iwave = wave < 4 && ihg;
  const int g = hg4 * 16 + li;
  const bool gva = ihg && g < p.nidx;
  const bool gv = iwave && gva;
  const int64_t grow = (int64_t)row * p.nidx + (gva ? g : 0);
  // index Q fragments (A operand of the index scores: head g, d 32*ks +
  // 8*lg ..) from the row's index queries staged in LDS
  for (int e = tid; e < kKlMaxNidx * (DI / 8); e += NT) {
    const int gg = e / (DI / 8), c = e - gg * (DI / 8);
    const u32x4 v = gg < p.nidx ? *(const u32x4*)((const T*)p.qi + ((int64_t)row * p.nidx + gg) * DI + c * 8) : z4;
    *(u32x4*)&s_qi[gg * QIR + c * 8] = v;
  }
  auto qif_load = [&](int ks) -> V8 { return as_v8<V8>(*(const u32x4*)&s_qi[g * QIR + ks * 32 + lg * 8]); };
  const float wg = gv ? load_w(p.w, grow, p.w_dtype) : 0.f;
  float wr[4];  // weights of index heads 16*hg4 + 4*lg + r (pass A layout)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int gg = hg4 * 16 + lg * 4 + r;
    wr[r] = (ihg && gg < p.nidx) ? load_w(p.w, (int64_t)row * p.nidx + gg, p.w_dtype) : 0.f;
  }
  // per-wave partial sums of a tile; waves without heads keep zeros
  for (int e = tid; e < 2 * kKlWaves * TILE; e += NT) (&s_red[0][0][0])[e] = 0.f;
  for (int e = tid; e < 2 * 4 * TILE; e += NT) (&s_redi[0][0][0])[e] = 0.f;

  const unsigned char* kb = (const unsigned char*)p.k;
  const unsigned char* krb = (const unsigned char*)p.kr;
  const unsigned char* kib = (const unsigned char*)p.ki;

  // ================= pass A: teacher p and index scores I =================
  for (int k = tid; k < n; k += NT) s_tok[k] = kl_token(p.m, ri, p.idx, row, k);
  __syncthreads();

  // unconditional LDS reads (index clamped into the row) and a select: a
  // read under a lane condition is masked on its own and waited for alone
  auto slot_tok = [&](int k) {
    const int v = s_tok[k < n ? k : n - 1];
    return k < n ? v : -1;
  };
  // Tile t into ring buffer b, gathered by waves 4-7 (iw = wave - 4): K
  // DMAs iw, iw+4, ..., rope DMA iw (iw < RD) and K_index DMAs iw, iw+4.  A
  // lane's 16 bytes land at its fixed slot of the buffer; it loads the
  // source chunk that the XOR swizzle puts there (LDS chunk c of a row holds
  // source chunk c ^ swz), so reads use the same addressing as a swizzled
  // store would.  A wave stalls at each DMA it issues while the CU's load
  // path is busy; on waves 4-7 those stalls leave the teacher waves 0-3 of
  // the same SIMDs running their MFMAs.  The token ids of a tile are read
  // from LDS first: the DMA asm is a compiler memory barrier, so a read
  // placed between two DMAs would wait for its own LDS round trip.
  constexpr int NIS = 4;
  static_assert(RD <= NIS, "one rope DMA per issuing wave");
  const int iw = wave - NIS;
  const bool a_issuer = iw >= 0;
  constexpr int NKW = (KD + NIS - 1) / NIS, NIW = (ID + NIS - 1) / NIS;
  auto issue_a = [&](int t, int b) {
    const unsigned base = (unsigned)(uintptr_t)(ring + b * BUF);
    int tk_k[NKW], tok_k[NKW], tk_i[NIW], tok_i[NIW], tk_r = 0, tok_r = -1;
#pragma unroll
    for (int u = 0; u < NKW; ++u) {
      const int j = u * NIS + iw;
      tk_k[u] = j * TPK + lane / CN;
      tok_k[u] = (KD % NIS == 0 || j < KD) ? slot_tok(t * TILE + tk_k[u]) : -1;
    }
    if (DR > 0 && iw < RD) {
      tk_r = iw * 8 + (lane >> 3);
      tok_r = slot_tok(t * TILE + tk_r);
    }
#pragma unroll
    for (int u = 0; u < NIW; ++u) {
      const int j = u * NIS + iw;
      tk_i[u] = j * TPI + lane / CI;
      tok_i[u] = (ID % NIS == 0 || j < ID) ? slot_tok(t * TILE + tk_i[u]) : -1;
    }
#pragma unroll
    for (int u = 0; u < NKW; ++u) {
      const int j = u * NIS + iw;
      if (KD % NIS == 0 || j < KD) {
        const int ch = (lane % CN) ^ nope_swz(tk_k[u]);
        kl_dma16(base + j * 1024, tok_k[u] >= 0 ? (const void*)(kb + (int64_t)tok_k[u] * ROW + ch * 16)
                                                : (const void*)(g_kl_zero_row + ch * 16));
      }
    }
    if (DR > 0 && iw < RD) {
      const int ch = (lane & 7) ^ rope_swz(tk_r);
      kl_dma16(base + BUF_K + iw * 1024, tok_r >= 0 ? (const void*)(krb + (int64_t)tok_r * (DR * 2) + ch * 16)
                                                    : (const void*)(g_kl_zero_row + ch * 16));
    }
#pragma unroll
    for (int u = 0; u < NIW; ++u) {
      const int j = u * NIS + iw;
      if (ID % NIS == 0 || j < ID) {
        const int ch = (lane % CI) ^ nope_swz(tk_i[u]);
        kl_dma16(base + BUF_K + BUF_R + j * 1024,
                 tok_i[u] >= 0 ? (const void*)(kib + (int64_t)tok_i[u] * IROW + ch * 16)
                               : (const void*)(g_kl_zero_row + ch * 16));
      }
    }
  };

  // One barrier per tile.  With two buffers, tile t+1 is issued right
  // after tile t's barrier into the buffer tile t-1 used (every wave is past
  // it); with one, after a second barrier behind the tile's MFMAs.  The loop
  // has no other global memory traffic, so vmcnt(0) waits for exactly the
  // issuing wave's share of the tile.  The per-slot sums of tile t-1
  // (complete at tile t's barrier) are reduced by wave 4 while the others
  // start tile t; the partial-sum buffers alternate, and wave 4 has reduced
  // tile t-2 from a buffer before any wave passes tile t's barrier to
  // overwrite it.
  auto reduce_a = [&](int t) {
    const int q = tid - NIS * 64;
    if (q >= 0 && q < TILE) {
      const int k = t * TILE + q;
      if (k < n) {
        float ps = 0.f, is = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) ps += s_red[t & 1][w2][q];
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) is += s_redi[t & 1][w2][q];
        s_p[k] = ps * (1.f / (float)p.n1);
        s_I[k] = is;
      }
    }
  };
  if (a_issuer) issue_a(0, 0);
  for (int t = 0; t < nt; ++t) {
    const int b = p.ring == 2 ? (t & 1) : 0;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    if (a_issuer && p.ring == 2 && t + 1 < nt) issue_a(t + 1, b ^ 1);
    if (t > 0) reduce_a(t - 1);
    const unsigned char* s_k = ring + b * BUF;
    const unsigned char* s_kr = s_k + BUF_K;
    const unsigned char* s_kia = s_k + BUF_K + BUF_R;

    // Teacher scores S[head][slot] = Q . K^T for the wave's 32 heads on
    // v_mfma_f32_32x32x16: B operand K[slot lane%32][d 16*ks + 8*(lane/32)
    // .. +7], one 16-byte LDS read per lane and k-step.  A lane's 16 results
    // are 16 heads of slot lane%32; their probabilities sum in the lane and
    // then with lane lane^32 (the other 16 heads).
    if (wave_heads) {
      f32x16 acc = {};
      // K fragments read PF k-steps ahead of their MFMA; the scheduling
      // barrier after each MFMA keeps the reads there (one wave per SIMD
      // runs these MFMAs: nothing else hides an LDS round trip)
      constexpr int PF = 4;
      // chunk 2*ks + hf of slot sl sits at (2*ks + hf) ^ swz(sl); with the
      // swizzle below 16 that is 16*(ks/8) + ((2*(ks%8)) ^ (hf ^ swz)): eight
      // lane offsets plus an immediate (nope), four for the rope rows
      const int sl = lane & 31, hf = lane >> 5;
      const int xn = hf ^ nope_swz(sl), xr = hf ^ rope_swz(sl);
      auto a_read = [&](int ks) -> u32x4 {
        const unsigned char* a =
            ks < KSN16 ? s_k + sl * ROW + (ks >> 3) * 256 + (((2 * (ks & 7)) ^ xn) * 16)
                       : s_kr + sl * (DR * 2) + (((2 * (ks - KSN16)) ^ xr) * 16);
        return *(const u32x4*)a;
      };
      u32x4 fa[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) fa[i] = a_read(i);
#pragma unroll
      for (int ks = 0; ks < KS16; ++ks) {
        const V8 bv = as_v8<V8>(fa[ks % PF]);
        if (ks + PF < KS16) fa[ks % PF] = a_read(ks + PF);
        acc = E::mfma32(qf[ks], bv, acc);
        __builtin_amdgcn_sched_barrier(0);
      }
      float ps = 0.f;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x4 mo = *(const f32x4*)&s_m2p[wave * 32 + 8 * r4 + 4 * hf];
#pragma unroll
        for (int r = 0; r < 4; ++r) ps += fast_exp2(acc[4 * r4 + r] * p.scale_log2 - mo[r]);
      }
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
      ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      if (lane < 32) s_red[t & 1][wave][lane] = ps;
    }
    // index scores I[slot] = sum_g w_g ReLU(qi_g . ki) on wave hg4 (after
    // its teacher scores; waves 4-7 are busy with the gather): index heads
    // 16*hg4 .. +15 for both halves of the tile
    if (twave && ihg) {
      // all twelve LDS reads first (query fragments, both halves' key
      // fragments), so their round trips overlap
      V8 qf_i[DI / 32];
      u32x4 kfi[2][DI / 32];
#pragma unroll
      for (int ks = 0; ks < DI / 32; ++ks) qf_i[ks] = qif_load(ks);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int ks = 0; ks < DI / 32; ++ks) {
          const int tk = tt * 16 + li;
          kfi[tt][ks] = *(const u32x4*)(s_kia + tk * IROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16));
        }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < DI / 32; ++ks) acc = E::mfma(qf_i[ks], as_v8<V8>(kfi[tt][ks]), acc);
        Split3 sp;
#pragma unroll
        for (int r = 0; r < 4; ++r) split3_set(sp, r, wr[r] * relu_bits(acc[r]));
        const f32x4 sum = split3_rowsum(sp);
        if (li == 0) *(f32x4*)&s_redi[t & 1][hg4][tt * 16 + lg * 4] = sum;
      }
    }
    if (p.ring == 1 && t + 1 < nt) {
      lds_barrier();
      if (a_issuer) issue_a(t + 1, 0);
    }
  }
  lds_barrier();
  reduce_a(nt - 1);
  lds_barrier();

  // (loaded after pass A, where they would only hold registers)
  V8 qif[DI / 32];
#pragma unroll
  for (int ks = 0; ks < DI / 32; ++ks) qif[ks] = qif_load(ks);
  // A operand of c^T = Qi^T . dS for the 32 columns 32*(wave & 3) + 16*ct
  // + li that pass C gives waves 4-7: Qi[g 32*ks + 8*lg + j][column]
  V8 qib[2][kKlMaxNidx / 32];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int ks = 0; ks < kKlMaxNidx / 32; ++ks) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int gg = ks * 32 + lg * 8 + j;
        T v = E::from_f32(0.f);
        if (gg < p.nidx) v = ((const T*)p.qi)[((int64_t)row * p.nidx + gg) * DI + (wave & 3) * 32 + ct * 16 + li];
        qib[ct][ks][j] = v;
      }
    }
  // ================= pass B: softmax(I), dI, KL =================
  float mx = -INFINITY;
  for (int k = tid; k < n; k += NT) mx = fmaxf(mx, s_I[k]);
  mx = wave_max(mx);
  if (lane == 0) s_misc[wave] = mx;
  lds_barrier();
  mx = s_misc[0];
#pragma unroll
  for (int w2 = 1; w2 < kKlWaves; ++w2) mx = fmaxf(mx, s_misc[w2]);
  float sm = 0.f;
  for (int k = tid; k < n; k += NT) sm += expf(s_I[k] - mx);
  sm = wave_sum(sm);
  lds_barrier();
  if (lane == 0) s_misc[wave] = sm;
  lds_barrier();
  sm = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < kKlWaves; ++w2) sm += s_misc[w2];
  const float inv_sm = 1.f / (sm + 1e-8f);
  float kl = 0.f, dmax = 0.f;
  for (int k = tid; k < n; k += NT) {
    const float si = expf(s_I[k] - mx) * inv_sm;
    const float pk = s_p[k];
    const float di = si - pk;
    const float pc = fmaxf(pk, 1e-8f), sc = fmaxf(si, 1e-8f);
    kl += pc * (logf(pc) - logf(sc));
    s_I[k] = di;
    dmax = fmaxf(dmax, fabsf(di));
  }
  kl = wave_sum(kl);
  dmax = wave_max(dmax);
  lds_barrier();
  if (lane == 0) {
    s_misc[wave] = kl;
    s_misc[kKlWaves + wave] = dmax;
  }
  lds_barrier();
  if (tid == 0) {
    float s = 0.f;
    for (int w2 = 0; w2 < kKlWaves; ++w2) s += s_misc[w2];
    p.loss_part[row] = s;
  }
  // Each slot's place in its token's bucket (the buckets were counted and
  // scanned before this kernel), into p's array, dead after the loop above:
  // the contributions go straight to their token's range, which the
  // reduction then reads contiguously.  A slot of a -1 page has none.
  int* const s_pos = (int*)s_p;
  for (int k = tid; k < n; k += NT) {
    const int t = s_tok[k];
    const int pos = t < 0 ? -1
                    : p.offs[t] + p.rank[(int64_t)row * p.topk + k] +
                          (p.cbase ? p.cbase[(int64_t)(row / p.chunk_rows) * p.tokens + t] : 0);
    s_pos[k] = pos;
    if (pos >= 0) p.posrow[pos] = row;
  }
  // fp16 operands: dS is carried as 2^es * dS so that hi/lo parts stay in
  // the fp16 normal range; the products are scaled back by 2^-es.
  float ds_scale = 1.f, ds_unscale = 1.f;
  if (kF16) {
    float dm = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kKlWaves; ++w2) dm = fmaxf(dm, s_misc[kKlWaves + w2]);
    float wm = fabsf(wg);
    wm = wave_max(wm);
    if (lane == 0) s_misc[2 * kKlWaves] = 0.f;
    lds_barrier();
    if (lane == 0 && wave < 4) atomicMax((int*)&s_misc[2 * kKlWaves], __float_as_int(wm));
    lds_barrier();
    wm = s_misc[2 * kKlWaves];
    const float bound = dm * wm;
    int e = 0;
    if (bound > 0.f) {
      frexpf(bound, &e);  // bound < 2^e
      e = 14 - e;         // scaled bound < 2^14
      e = max(-60, min(60, e));
    }
    ds_scale = ldexpf(1.f, e);
    ds_unscale = ldexpf(1.f, -e);
  }

  // Scale of the row's fp16 contributions: |c[slot][j]| = |sum_g dS[g][slot]
  // Qi[g][j]| <= max|dI| * sum_g |w_g| * max|Qi|; with that bound below
  // 2^(14 - e) the stored c * 2^e stays in fp16's normal range.
  float c_scale = 1.f;
  int c_exp = 0;
  {
    float dm = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kKlWaves; ++w2) dm = fmaxf(dm, s_misc[kKlWaves + w2]);
    float ws = lane < p.nidx ? fabsf(load_w(p.w, (int64_t)row * p.nidx + lane, p.w_dtype)) : 0.f;
    ws = wave_sum(ws);
    float qm = 0.f;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int ks = 0; ks < kKlMaxNidx / 32; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) qm = fmaxf(qm, fabsf(E::to_f32(qib[ct][ks][j])));
    qm = wave_max(qm);
    lds_barrier();
    if (lane == 0) s_misc[2 * kKlWaves + 1 + wave] = qm;
    lds_barrier();
#pragma unroll
    for (int w2 = 0; w2 < kKlWaves; ++w2) qm = fmaxf(qm, s_misc[2 * kKlWaves + 1 + w2]);
    const float bound = dm * ws * qm;
    if (bound > 0.f && bound < INFINITY) {
      int e;
      frexpf(bound, &e);  // bound < 2^e
      c_exp = max(-100, min(100, 14 - e));
      c_scale = ldexpf(1.f, c_exp);
    }
  }

  // ================= pass C: dW, dQi, dKi contributions =================
  // Software-pipelined over the tiles with one barrier per tile.  In step t,
  // waves 0-3 recompute tile t's index scores from its K_index tile, form
  // dS (hi / lo) into the dS^T tile of parity t & 1, and accumulate dW;
  // waves 4-7 take tile t-1: its dQi product (K_index and dS^T tiles through
  // the transposing read) and the slots' dKi contributions, which they
  // store.  Waves w and w + 4 own the same 16 index heads.  Waves 0-3
  // gather the K_index tiles by LDS-DMA into four buffers, two tiles ahead;
  // they issue no other global memory operation in the loop, so their vmcnt
  // counts exactly these DMAs (two per wave and tile).  The buffer that tile
  // t+2 is issued into held tile t-2, which waves 0-3 read in step t-2 and
  // waves 4-7 in step t-1, both before step t's barrier; the dS^T tile of
  // parity t & 1 held tile t-2, likewise finished before that barrier.
  static_assert(ID == 8 && kKlTile * DI * 2 == 8 * 1024, "two K_index DMAs per wave of waves 0-3");
  unsigned char* const pc_ki = ring;
  T* const pc_ds = (T*)(ring + kKlPcBufs * kKlPcKiBytes);  // [parity][hi / lo][slot][kKlDsRow]
  // columns g >= Nidx1 of the dS^T tiles stay zero (waves without index
  // heads never write theirs); the K rows of pass A no longer need the space
  for (int e = tid; e < 2 * kKlPcDsBytes / 8; e += NT) ((uint2*)pc_ds)[e] = make_uint2(0u, 0u);
  f32x4 acc_dqi[DI / 16];
#pragma unroll
  for (int dt = 0; dt < DI / 16; ++dt) acc_dqi[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float dw_acc = 0.f, cmax = 0.f;
  const bool dma_wave = wave < 4;
  auto issue_c = [&](int t) {
    const unsigned base = (unsigned)(uintptr_t)(pc_ki + (t % kKlPcBufs) * kKlPcKiBytes);
    int tk[2], tok[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      tk[u] = (u * 4 + wave) * TPI + lane / CI;
      tok[u] = slot_tok(t * TILE + tk[u]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ch = (lane % CI) ^ nope_swz(tk[u]);
      kl_dma16(base + (u * 4 + wave) * 1024, tok[u] >= 0 ? (const void*)(kib + (int64_t)tok[u] * IROW + ch * 16)
                                                         : (const void*)(g_kl_zero_row + ch * 16));
    }
  };
  if (dma_wave) {
    issue_c(0);
    if (nt > 1) issue_c(1);
  }
  for (int t = 0; t <= nt; ++t) {
    if (dma_wave && t < nt) {
      if (t + 1 < nt) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    lds_barrier();
    if (dma_wave && t + 2 < nt) issue_c(t + 2);
    if (iwave && t < nt) {
      const unsigned char* s_ki = pc_ki + (t % kKlPcBufs) * kKlPcKiBytes;
      T* const dsh = pc_ds + (t & 1) * 2 * TILE * kKlDsRow;
      T* const dsl_ = dsh + TILE * kKlDsRow;
      f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < DI / 32; ++ks)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int tk = tt * 16 + li;
          const unsigned char* a = s_ki + tk * IROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16);
          acc[tt] = E::mfma(as_v8<V8>(*(const u32x4*)a), qif[ks], acc[tt]);
        }
      // dS^T of slots 16*tt + 4*lg + r, head g; the slots' dI read together
      // (unconditional, clamped)
      float dis[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = t * TILE + (j >> 2) * 16 + lg * 4 + (j & 3);
        dis[j] = s_I[k < n ? k : n - 1];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tt = j >> 2, r = j & 3;
        const int tk = tt * 16 + lg * 4 + r;
        const int k = t * TILE + tk;
        const float relu = relu_bits(acc[tt][r]);
        const float di = (k < n && gv) ? dis[j] : 0.f;
        dw_acc += di * relu;
        const float ds = relu > 0.f ? di * wg * ds_scale : 0.f;
        const T hi = E::from_f32(ds);
        const T lo = E::from_f32(ds - E::to_f32(hi));
        dsh[tk * kKlDsRow + g] = hi;
        dsl_[tk * kKlDsRow + g] = lo;
      }
    }
    if (!dma_wave && t > 0) {
      // c^T[d][slot] = sum_g Qi^T[d][g] dS^T[slot][g] for tile t-1: C
      // register r of a lane is column d = 32*(wave & 3) + 16*ct + 4*lg + r
      // of slot 16*tt + li, so a lane stores 4 consecutive fp16 values
      const int tp = t - 1;
      const T* const dsh = pc_ds + (tp & 1) * 2 * TILE * kKlDsRow;
      const T* const dsl_ = dsh + TILE * kKlDsRow;
      if (ihg) {
        // dQi^T[d][g] += Ki^T[d][slot] . dS^T[slot][g] for this wave's 16
        // heads.  Both operands come through the transposing read: rows
        // 4*lg + li/4 (+16), 16-byte chunk 2*dt + (li&3)/2 (+8 bytes for odd
        // li) of a [slot][column] tile gives k-slot 8*lg + j as slot
        // (j>>2)*16 + 4*lg + (j&3) in either operand.
        const unsigned char* s_ki = pc_ki + (tp % kKlPcBufs) * kKlPcKiBytes;
        const int r1 = lg * 4 + (li >> 2);
        const int hb = (li & 3) >> 1;
        auto tr8 = [&](const unsigned char* q1, const unsigned char* q2) -> V8 {
          const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)q1));
          const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)q2));
          const i16x8 wv = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
          return __builtin_bit_cast(V8, wv);
        };
        constexpr int DSR = kKlDsRow * 2;  // bytes of a dS^T row
        const int dso = (2 * hg4 + hb) * 16 + (li & 1) * 8;
        const V8 dsf = tr8((const unsigned char*)dsh + r1 * DSR + dso, (const unsigned char*)dsh + (r1 + 16) * DSR + dso);
        const V8 dsl = tr8((const unsigned char*)dsl_ + r1 * DSR + dso, (const unsigned char*)dsl_ + (r1 + 16) * DSR + dso);
#pragma unroll
        for (int dt = 0; dt < DI / 16; ++dt) {
          const int ch = 2 * dt + hb;
          const V8 kt = tr8(s_ki + r1 * IROW + ((ch ^ nope_swz(r1)) * 16) + (li & 1) * 8,
                            s_ki + (r1 + 16) * IROW + ((ch ^ nope_swz(r1 + 16)) * 16) + (li & 1) * 8);
          acc_dqi[dt] = E::mfma(kt, dsf, acc_dqi[dt]);
          acc_dqi[dt] = E::mfma(kt, dsl, acc_dqi[dt]);
        }
      }
      f32x4 acc[2][2] = {{{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int ks = 0; ks < kKlMaxNidx / 32; ++ks) {
          const V8 bh = as_v8<V8>(*(const u32x4*)&dsh[(tt * 16 + li) * kKlDsRow + ks * 32 + lg * 8]);
          const V8 bl = as_v8<V8>(*(const u32x4*)&dsl_[(tt * 16 + li) * kKlDsRow + ks * 32 + lg * 8]);
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            acc[tt][ct] = E::mfma(qib[ct][ks], bh, acc[tt][ct]);
            acc[tt][ct] = E::mfma(qib[ct][ks], bl, acc[tt][ct]);
          }
        }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int k = tp * TILE + tt * 16 + li;
        if (k < n) {
          const int pos = s_pos[k];
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            _Float16 h[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float c = acc[tt][ct][r] * ds_unscale;
              cmax = __builtin_elementwise_maximum(cmax, fabsf(c));  // NaN-propagating
              h[r] = (_Float16)(c * c_scale);
            }
            if (pos >= 0)
              *(uint2*)(p.cbuf + (int64_t)pos * DI + (wave & 3) * 32 + ct * 16 + lg * 4) = __builtin_bit_cast(uint2, h);
          }
        }
      }
    }
  }

  // ---- epilogue: dW (waves 0-3), dQi (waves 4-7), row maximum of |c| ----
  if (iwave) {
    const float dwv = xgroup_sum(dw_acc);
    if (lg == 0 && gv) store_w(p.dw, grow, p.w_dtype, dwv);
  }
  if (!dma_wave && gva) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T* dst = (T*)p.dqi + grow * DI;
#pragma unroll
    for (int dt = 0; dt < DI / 16; ++dt) {
      const T4 o = {E::from_f32(acc_dqi[dt][0] * ds_unscale), E::from_f32(acc_dqi[dt][1] * ds_unscale),
                    E::from_f32(acc_dqi[dt][2] * ds_unscale), E::from_f32(acc_dqi[dt][3] * ds_unscale)};
      *(T4*)(dst + dt * 16 + lg * 4) = o;
    }
  }
  // a non-finite contribution (NaN kept by the maximum above) makes the row
  // maximum infinite, which turns its tokens' dKi into NaN in the reduction
  cmax = cmax < INFINITY ? cmax : INFINITY;
  cmax = wave_max(cmax);
  lds_barrier();
  if (lane == 0) s_misc[wave] = cmax;
  lds_barrier();
  if (tid == 0) {
    float m = 0.f;
    for (int w2 = 0; w2 < kKlWaves; ++w2) m = fmaxf(m, s_misc[w2]);
    p.rowmax[row] = m;
    p.rowexp[row] = c_exp;
    s_misc[3 * kKlWaves] = m;
  }
  // the row maximum raises its tokens' maxima (non-negative floats order as
  // their bit patterns), which fix the reduction's fixed-point exponents
  lds_barrier();
  const unsigned mbits = __float_as_uint(s_misc[3 * kKlWaves]);
  for (int k = tid; k < n; k += NT) {
    const int t = s_tok[k];
    if (t >= 0) atomicMax(&p.tokmax[t], mbits);
  }
}

// ---------------------------------------------------------------------------
// dKi: bucket slots by target token, then a fixed-point sum per token
// ---------------------------------------------------------------------------
struct KlScatter {
  KlMap m;
  const int32_t* idx;
  int32_t* cnt;         // [tokens]
  int32_t* rank;        // [rows * topK] the slot's place among its token's slots
};

__global__ __launch_bounds__(256) void kl_zero_kernel(int32_t* a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] = 0;
}

// the count's old value is the slot's place in the token's bucket (run
// before the row kernel, which stores each contribution at that place)
__global__ __launch_bounds__(256) void kl_bucket_kernel(KlScatter s) {
  const int row = blockIdx.x;
  const int k = blockIdx.y * 256 + threadIdx.x;
  const KlRow r = kl_row_info(s.m, row);
  if (k >= r.n) return;
  const int t = kl_token(s.m, r, s.idx, row, k);
  if (t < 0) return;  // a -1 page: no gradient target
  s.rank[(int64_t)row * s.m.topk + k] = atomicAdd(&s.cnt[t], 1);
}

// Ranks without global atomics on hot counters (a causal row set sends
// thousands of rows' slots to each early token, and the returning global
// atomics of kl_bucket_kernel serialise on those counters): a workgroup
// owns a chunk of consecutive rows, counts their slots per token in LDS
// (the slot's rank within the chunk is the LDS counter's old value) and
// writes the chunk's counts; kl_rank_scan_kernel turns them into each
// chunk's start within each bucket and the buckets' totals.  For key sets
// up to kKlRankMaxTok tokens (the LDS counters).
constexpr int kKlRankMaxTok = 16384;
constexpr int kKlRankMaxChunks = 512;
constexpr int kKlRankThreads = 512;

__global__ __launch_bounds__(kKlRankThreads) void kl_rank_local_kernel(KlScatter s, int32_t* ccnt, int chunk_rows,
                                                                       int tokens) {
  extern __shared__ int s_cnt[];  // [tokens]
  constexpr int U = 8;            // slots per thread in flight
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * chunk_rows, r1 = min(s.m.rows, r0 + chunk_rows);
  for (int i = tid; i < tokens; i += kKlRankThreads) s_cnt[i] = 0;
  __syncthreads();
  const int64_t total = (int64_t)(r1 - r0) * s.m.topk;
  for (int64_t e0 = 0; e0 < total; e0 += (int64_t)kKlRankThreads * U) {
    int tk[U];
    int64_t slot[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = e0 + (int64_t)u * kKlRankThreads + tid;
      const int rr = (int)(e / s.m.topk), k = (int)(e - (int64_t)rr * s.m.topk);
      const int row = r0 + rr;
      tk[u] = -1;
      slot[u] = (int64_t)row * s.m.topk + k;
      if (e < total) {
        const KlRow r = kl_row_info(s.m, row);
        if (k < r.n) tk[u] = kl_token(s.m, r, s.idx, row, k);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (tk[u] >= 0) s.rank[slot[u]] = atomicAdd(&s_cnt[tk[u]], 1);
  }
  __syncthreads();
  for (int i = tid; i < tokens; i += kKlRankThreads) ccnt[(int64_t)blockIdx.x * tokens + i] = s_cnt[i];
}

// ccnt[c][t] -> the start of chunk c within token t's bucket (exclusive
// prefix over the chunks), cnt[t] = the bucket's size.  A workgroup takes 64
// tokens; each of its 16 waves a contiguous run of chunks.
__global__ __launch_bounds__(1024) void kl_rank_scan_kernel(int32_t* ccnt, int32_t* cnt, int nchunks, int tokens) {
  __shared__ int32_t s_part[16][64];
  const int lane = threadIdx.x & 63, part = threadIdx.x >> 6;
  const int t = blockIdx.x * 64 + lane;
  const int per = (nchunks + 15) / 16;
  const int c0 = min(nchunks, part * per), c1 = min(nchunks, c0 + per);
  int32_t sum = 0;
  if (t < tokens)
    for (int c = c0; c < c1; ++c) sum += ccnt[(int64_t)c * tokens + t];
  s_part[part][lane] = sum;
  __syncthreads();
  int32_t run = 0, tot = 0;
  for (int q = 0; q < 16; ++q) {
    run += q < part ? s_part[q][lane] : 0;
    tot += s_part[q][lane];
  }
  if (t < tokens) {
    for (int c = c0; c < c1; ++c) {
      int32_t* a = ccnt + (int64_t)c * tokens + t;
      const int32_t v = *a;
      *a = run;
      run += v;
    }
    if (part == 0) cnt[t] = tot;
  }
}

// exclusive scan of cnt[0..n) into offs[0..n] (one workgroup)
__global__ __launch_bounds__(1024) void kl_scan_kernel(const int32_t* cnt, int32_t* offs, int n) {
  __shared__ int32_t s_sum[1024];
  const int tid = threadIdx.x;
  const int per = (n + 1023) / 1024;
  const int lo = min(n, tid * per), hi = min(n, lo + per);
  int32_t s = 0;
  for (int i = lo; i < hi; ++i) s += cnt[i];
  s_sum[tid] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int32_t v = tid >= o ? s_sum[tid - o] : 0;
    __syncthreads();
    s_sum[tid] += v;
    __syncthreads();
  }
  int32_t run = tid > 0 ? s_sum[tid - 1] : 0;
  for (int i = lo; i < hi; ++i) {
    offs[i] = run;
    run += cnt[i];
  }
  if (tid == 1023) offs[n] = s_sum[1023];
}

// dKi[t] = sum of the token's slot contributions, in fixed point with the
// exponent fixed by the token's largest row maximum and slot count (every
// partial sum is an integer below 2^52, exact as a double and as an int64).  A token's slots are split into up to
// `parts` (at most kKlReduceParts) parts of at least kKlReduceChunk slots,
// one wave each; the host sets `parts` from the average slots per token, so
// that sparsely hit tokens keep a grid of one wave per token: a
// token with one part writes dKi directly; the parts of a longer token add
// their partial sums into an int64 accumulator with integer atomics, which
// kl_reduce_finish_kernel converts.  Integer addition is exact and
// associative, so the result does not depend on the split or on the order.
constexpr int kKlReduceParts = 16;
constexpr int kKlReduceChunk = 256;

__device__ __forceinline__ int kl_reduce_parts(int len, int parts) {
  return max(1, min(parts, (len + kKlReduceChunk - 1) / kKlReduceChunk));
}
// fixed-point exponent: len * bm < 2^(52 - e), so every partial sum of
// terms rounded to the grid 2^-e is an integer below 2^52, exact in a double
__device__ __forceinline__ int kl_fixed_exp(float bm, int len) {
  int ex;
  frexp((double)bm * (double)len, &ex);
  return 52 - ex;
}

// di: contribution columns (the index head dim), a multiple of 8; a wave
// covers 128 columns per sweep (two per lane).
template <typename T>
__global__ __launch_bounds__(256) void kl_reduce_kernel(const _Float16* cbuf, const int32_t* rowexp,
                                                        const uint32_t* tokmax, const int32_t* offs,
                                                        const int32_t* posrow, long long* acc, T* dki, int ntok,
                                                        int parts, int di) {
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int t = w / parts, part = w - t * parts;
  const int lane = threadIdx.x & 63;
  if (t >= ntok) return;
  const int o0 = __builtin_amdgcn_readfirstlane(offs[t]);
  const int len = __builtin_amdgcn_readfirstlane(offs[t + 1]) - o0;
  const int np = kl_reduce_parts(len, parts);
  if (part >= np) return;
  const float bm = __uint_as_float(tokmax[t]);
  for (int col = 2 * lane; col < ((di + 127) & ~127); col += 128) {
    const bool cv = col < di;
    T* dst = dki + (int64_t)t * di + col;
    if (!(bm < INFINITY)) {  // non-finite contributions: no fixed-point scale exists
      if (part == 0 && cv) {
        dst[0] = Elem<T>::from_f32(NAN);
        dst[1] = Elem<T>::from_f32(NAN);
      }
      continue;
    }
    double a0 = 0.0, a1 = 0.0;
    int e = 0;
    if (bm > 0.f) {
      e = kl_fixed_exp(bm, len);
      const int L = (len + np - 1) / np;
      const int i1 = min(len, (part + 1) * L);
      // A contribution is c16 * 2^-e_row; its fixed-point value is
      // rint(c16 * 2^(e - e_row)) (scaled and rounded in fp32, where it is
      // exact, then widened to a double; an integer below 2^52 either way),
      // and the sums of such values stay below 2^52 (the exponent's bound), so the
      // double additions are exact and their order does not matter (an
      // integer shift-and-round per element, with branches or branch-free,
      // and a conversion to int64 per element measured slower).  The
      // token's contributions are consecutive rows; the rows' exponents of
      // 64 positions come in with one load per lane and are broadcast with
      // readlane; 16 contribution rows are in flight at a time.
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      constexpr int U = 16;
      for (int base = part * L; base < i1; base += 64) {
        const int cnt = min(64, i1 - base);
        const int kv = lane < cnt ? e - rowexp[posrow[o0 + base + lane]] : 0;
        for (int u0 = 0; u0 < cnt; u0 += U) {
          h2 v[U];
  #pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t pos = (int64_t)o0 + base + u0 + u;
            v[u] = (u0 + u < cnt && cv) ? *(const h2*)(cbuf + pos * di + col) : (h2){0, 0};
          }
  #pragma unroll
          for (int u = 0; u < U; ++u) {
            // a nonzero c16 (>= 2^-24) has c16 * 2^kv < 2^52, so kv < 76;
            // a zero one may come with a larger kv, which must not reach
            // fp32's infinity (0 * inf is NaN)
            const float sc = ldexpf(1.f, min(__builtin_amdgcn_readlane(kv, u0 + u), 80));
            a0 += (double)__builtin_rintf((float)v[u].x * sc);
            a1 += (double)__builtin_rintf((float)v[u].y * sc);
          }
        }
      }
    }
    if (!cv) continue;
    if (np == 1) {
      const double us = ldexp(1.0, -e);
      dst[0] = Elem<T>::from_f32((float)(a0 * us));
      dst[1] = Elem<T>::from_f32((float)(a1 * us));
    } else {
      // the parts' exact integer sums meet in int64 atomics
      unsigned long long* ap = (unsigned long long*)acc + (int64_t)t * di + col;
      atomicAdd(ap, (unsigned long long)(long long)a0);
      atomicAdd(ap + 1, (unsigned long long)(long long)a1);
    }
  }
}

// dKi of the tokens with more than one part, from their accumulators
template <typename T>
__global__ __launch_bounds__(256) void kl_reduce_finish_kernel(const uint32_t* tokmax, const int32_t* offs,
                                                               const long long* acc, T* dki, int ntok, int parts,
                                                               int di) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= ntok) return;
  const int len = offs[t + 1] - offs[t];
  if (kl_reduce_parts(len, parts) == 1) return;
  const float bm = __uint_as_float(tokmax[t]);
  if (!(bm < INFINITY)) return;
  const int e = bm > 0.f ? kl_fixed_exp(bm, len) : 0;
  const double us = ldexp(1.0, -e);
  for (int col = 2 * lane; col < di; col += 128) {
    const long long* ap = acc + (int64_t)t * di + col;
    T* dst = dki + (int64_t)t * di + col;
    dst[0] = Elem<T>::from_f32((float)((double)ap[0] * us));
    dst[1] = Elem<T>::from_f32((float)((double)ap[1] * us));
  }
}

// loss = sum of the per-row terms, in a fixed order (one workgroup)
__global__ __launch_bounds__(256) void kl_loss_kernel(const float* part, int rows, float* loss) {
  __shared__ double s[256];
  double a = 0.0;
  for (int i = threadIdx.x; i < rows; i += 256) a += (double)part[i];
  s[threadIdx.x] = a;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) s[threadIdx.x] += s[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = (float)s[0];
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct KlWs {
  size_t cbuf, rowmax, rowexp, loss, cnt, tokmax, acc, offs, rank, posrow, pi, ccnt, total;
  int32_t chunk_rows, nchunks;  // row chunks of the LDS ranking (0: global atomics)
};

// pi (the generic path's per-slot p / I) is laid out for every call: the
// workspace query does not know Nidx1, which also selects the generic path
static KlWs kl_ws_layout(int64_t rows, int64_t tokens, int64_t topk, int64_t di) {
  KlWs w;
  size_t o = 0;
  w.cbuf = o;
  o += align256((size_t)rows * topk * di * sizeof(_Float16));
  w.rowmax = o;
  o += align256((size_t)rows * sizeof(float));
  w.rowexp = o;
  o += align256((size_t)rows * sizeof(int32_t));
  w.loss = o;
  o += align256((size_t)rows * sizeof(float));
  w.cnt = o;
  o += align256((size_t)tokens * sizeof(int32_t));
  w.tokmax = o;
  o += align256((size_t)tokens * sizeof(uint32_t));
  w.acc = o;
  o += align256((size_t)tokens * di * sizeof(long long));
  w.offs = o;
  o += align256((size_t)(tokens + 1) * sizeof(int32_t));
  w.rank = o;
  o += align256((size_t)rows * topk * sizeof(int32_t));
  w.posrow = o;
  o += align256((size_t)rows * topk * sizeof(int32_t));
  w.pi = o;
  o += align256((size_t)rows * topk * 2 * sizeof(float));
  // the LDS ranking's per-chunk counts: at most kKlRankMaxChunks chunks of
  // at least 16 rows
  w.chunk_rows = 0;
  w.nchunks = 0;
  if (tokens <= kKlRankMaxTok && rows > 0) {
    w.chunk_rows = (int32_t)std::max<int64_t>(16, (rows + kKlRankMaxChunks - 1) / kKlRankMaxChunks);
    w.nchunks = (int32_t)((rows + w.chunk_rows - 1) / w.chunk_rows);
  }
  w.ccnt = o;
  o += align256((size_t)w.nchunks * tokens * sizeof(int32_t));
  w.total = o;
  return w;
}

size_t kl_bwd_workspace_bytes(int64_t q_rows, int64_t kv_rows, int64_t topk, int64_t d_idx) {
  return kl_ws_layout(q_rows, kv_rows, topk, d_idx).total;
}

// limits of the whole operator (the generic path's); the fused row kernel
// takes d_idx = 128, Nidx1 <= kKlMaxNidx and topK <= kKlMaxTopk
int kl_bwd_max_topk() { return 1 << 20; }
int kl_bwd_max_nidx() { return kGenMaxNidx; }
int kl_bwd_max_didx() { return kGenMaxDi; }

// The row kernel's dynamic LDS: the pass-A tile ring, then I, p and the
// token rows of a row (3 x topK x 4 bytes).  Two tile buffers when they fit
// beside the row's arrays and the static LDS, else one (top-k over about
// 5000 at D = 512).
constexpr int kKlLdsBytes = 160 * 1024;

template <int D, int DR, typename T>
static hipError_t run_kl_row(KlParams p, int rows, int64_t topk, hipStream_t stream) {
  const void* fn = (const void*)kl_bwd_row_kernel<D, DR, T>;
  // the kernel's static LDS (a property of the code object; the local
  // static's initialisation is thread-safe)
  static const int static_lds = [] {
    hipFuncAttributes fa;
    return hipFuncGetAttributes(&fa, (const void*)kl_bwd_row_kernel<D, DR, T>) == hipSuccess
               ? (int)fa.sharedSizeBytes : -1;
  }();
  if (static_lds < 0) return hipErrorInvalidDeviceFunction;
  const int buf = kl_tile_bytes<D, DR>();
  const int rowb = (int)(3 * topk * sizeof(float));
  p.ring = static_lds + std::max(2 * buf, kKlPcBytes) + rowb <= kKlLdsBytes ? 2 : 1;
  p.ringb = std::max(p.ring * buf, kKlPcBytes);
  const int dyn = p.ringb + rowb;
  if (static_lds + dyn > kKlLdsBytes) return hipErrorInvalidConfiguration;
  // raised on every call: a host-side setting, cheap next to the kernel, and
  // right for whichever device is current and for concurrent callers
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, dyn);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((kl_bwd_row_kernel<D, DR, T>), dim3(rows), dim3(kKlWaves * 64), (size_t)dyn, stream, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t dispatch_kl_row(const KlParams& p, int rows, int d, int dr, int64_t topk, hipStream_t stream) {
  if (dr == 64) {
    if (d == 128) return run_kl_row<128, 64, T>(p, rows, topk, stream);
    if (d == 256) return run_kl_row<256, 64, T>(p, rows, topk, stream);
    return run_kl_row<512, 64, T>(p, rows, topk, stream);
  }
  if (d == 128) return run_kl_row<128, 0, T>(p, rows, topk, stream);
  if (d == 256) return run_kl_row<256, 0, T>(p, rows, topk, stream);
  return run_kl_row<512, 0, T>(p, rows, topk, stream);
}

int kl_bwd_run(const void* query, const void* key, const void* query_rope, const void* key_rope,
               const void* query_index, const void* key_index, const void* weights, const int32_t* sparse_indices,
               const float* softmax_max, const float* softmax_sum, const int32_t* act_q, const int32_t* act_k,
               const int32_t* block_table, void* d_query_index, void* d_key_index, void* d_weights, float* loss,
               int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t d_rope, int64_t nidx,
               int64_t d_idx, int64_t topk, int64_t q_rows, int64_t kv_rows, int64_t max_blocks,
               int64_t page_size, int32_t layout_q, int32_t layout_k, int32_t dtype, int32_t w_dtype,
               float scale_value, void* workspace, hipStream_t stream) {
  const int64_t rows = q_rows, tokens = kv_rows;
  const KlWs L = kl_ws_layout(rows, tokens, topk, d_idx);
  unsigned char* ws = (unsigned char*)workspace;
  KlMap m;
  m.act_q = act_q;
  m.act_k = act_k;
  m.block_table = block_table;
  m.kv_rows = kv_rows;
  m.batch = (int32_t)batch;
  m.s1 = (int32_t)s1;
  m.s2 = (int32_t)s2;
  m.rows = (int32_t)rows;
  m.topk = (int32_t)topk;
  m.max_blocks = (int32_t)max_blocks;
  m.page_size = (int32_t)page_size;
  m.layout_q = layout_q;
  m.layout_k = layout_k;

  KlParams p;
  p.m = m;
  p.q = query;
  p.qr = query_rope;
  p.k = key;
  p.kr = key_rope;
  p.qi = query_index;
  p.ki = key_index;
  p.w = weights;
  p.idx = sparse_indices;
  p.smax = softmax_max;
  p.ssum = softmax_sum;
  p.dqi = d_query_index;
  p.dw = d_weights;
  p.cbuf = (_Float16*)(ws + L.cbuf);
  p.rowmax = (float*)(ws + L.rowmax);
  p.rowexp = (int32_t*)(ws + L.rowexp);
  p.loss_part = (float*)(ws + L.loss);
  p.n1 = (int32_t)n1;
  p.nidx = (int32_t)nidx;
  p.topk = (int32_t)topk;
  p.w_dtype = w_dtype;
  p.scale_log2 = scale_value * kLog2e;

  KlScatter s;
  s.m = m;
  s.idx = sparse_indices;
  s.cnt = (int32_t*)(ws + L.cnt);
  s.rank = (int32_t*)(ws + L.rank);
  int32_t* const offs = (int32_t*)(ws + L.offs);
  uint32_t* const tokmax = (uint32_t*)(ws + L.tokmax);
  int32_t* const posrow = (int32_t*)(ws + L.posrow);
  long long* acc = (long long*)(ws + L.acc);
  int32_t* const ccnt = L.nchunks > 0 ? (int32_t*)(ws + L.ccnt) : nullptr;
  p.offs = offs;
  p.rank = s.rank;
  p.cbase = ccnt;
  p.chunk_rows = L.chunk_rows > 0 ? L.chunk_rows : 1;
  p.tokens = (int32_t)tokens;
  p.posrow = posrow;
  p.tokmax = tokmax;

  // parts per token of the dKi reduction: about avg_slots / 64,
  // 1..kKlReduceParts (long causal rows give every early token thousands of
  // slots; a long context with few slots per token keeps one wave per token)
  const int64_t avg = tokens > 0 ? rows * topk / tokens : 0;
  const int parts = (int)std::max<int64_t>(1, std::min<int64_t>(kKlReduceParts, (avg + 63) / 64));
  // counters, token maxima and (when tokens are split) the accumulators,
  // cnt .. acc or cnt .. offs, cleared by a kernel (no memset nodes when the
  // caller captures).  The count pass records each slot's place in its
  // token's bucket and the scan the buckets' starts, before the row kernel:
  // it stores each contribution at its place and raises its tokens' maxima.
  const int64_t zn = (int64_t)(((parts > 1 ? L.offs : L.acc) - L.cnt) / sizeof(int32_t));
  hipLaunchKernelGGL(kl_zero_kernel, dim3((unsigned)((zn + 255) / 256)), dim3(256), 0, stream, s.cnt, zn);
  DSA_HIP(hipGetLastError());
  if (ccnt) {
    const size_t lds = (size_t)tokens * sizeof(int32_t);
    if (lds > 64 * 1024)
      DSA_HIP(hipFuncSetAttribute((const void*)kl_rank_local_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds));
    hipLaunchKernelGGL(kl_rank_local_kernel, dim3((unsigned)L.nchunks), dim3(kKlRankThreads), lds, stream, s, ccnt,
                       (int)L.chunk_rows, (int)tokens);
    DSA_HIP(hipGetLastError());
    hipLaunchKernelGGL(kl_rank_scan_kernel, dim3((unsigned)((tokens + 63) / 64)), dim3(1024), 0, stream, ccnt, s.cnt,
                       (int)L.nchunks, (int)tokens);
    DSA_HIP(hipGetLastError());
  } else {
    const dim3 bgrid((unsigned)rows, (unsigned)((topk + 255) / 256));
    hipLaunchKernelGGL(kl_bucket_kernel, bgrid, dim3(256), 0, stream, s);
    DSA_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(kl_scan_kernel, dim3(1), dim3(1024), 0, stream, s.cnt, offs, (int)tokens);
  DSA_HIP(hipGetLastError());
  const bool bf = dtype == DSA_DTYPE_BF16;
  // the fused row kernel where it applies (d_idx = 128, Nidx1 <= 64, topK
  // <= 8192, and its LDS fits: it returns hipErrorInvalidConfiguration
  // before launching otherwise), else the generic path
  hipError_t e = hipErrorInvalidConfiguration;
  if (d_idx == kKlDi && nidx <= kKlMaxNidx && topk <= kKlMaxTopk && !(test_flags() & kTestKlGeneric))
    e = bf ? dispatch_kl_row<bf16>(p, (int)rows, (int)d, (int)d_rope, topk, stream)
           : dispatch_kl_row<f16>(p, (int)rows, (int)d, (int)d_rope, topk, stream);
  if (e == hipErrorInvalidConfiguration) {
    KlGenParams g;
    g.m = m;
    g.q = query;
    g.qr = query_rope;
    g.k = key;
    g.kr = key_rope;
    g.qi = query_index;
    g.ki = key_index;
    g.w = weights;
    g.idx = sparse_indices;
    g.smax = softmax_max;
    g.ssum = softmax_sum;
    g.dqi = d_query_index;
    g.dw = d_weights;
    g.cbuf = p.cbuf;
    g.rowmax = p.rowmax;
    g.rowexp = p.rowexp;
    g.offs = offs;
    g.rank = s.rank;
    g.cbase = ccnt;
    g.chunk_rows = p.chunk_rows;
    g.tokens = (int32_t)tokens;
    g.posrow = posrow;
    g.tokmax = tokmax;
    g.loss_part = p.loss_part;
    g.pi = (float*)(ws + L.pi);
    g.n1 = (int32_t)n1;
    g.nidx = (int32_t)nidx;
    g.di = (int32_t)d_idx;
    g.dip = (int32_t)((d_idx + 31) / 32 * 32);
    g.topk = (int32_t)topk;
    g.w_dtype = w_dtype;
    g.scale_log2 = scale_value * kLog2e;
    e = kl_gen_run(g, (int)rows, (int)d, (int)d_rope, bf, stream);
  }
  DSA_HIP(e);
  const dim3 rgrid((unsigned)((tokens * parts + 3) / 4));
  const dim3 fgrid((unsigned)((tokens + 3) / 4));
  if (bf) {
    hipLaunchKernelGGL(kl_reduce_kernel<bf16>, rgrid, dim3(256), 0, stream, p.cbuf, p.rowexp, tokmax, offs,
                       posrow, acc, (bf16*)d_key_index, (int)tokens, parts, (int)d_idx);
    DSA_HIP(hipGetLastError());
    hipLaunchKernelGGL(kl_reduce_finish_kernel<bf16>, fgrid, dim3(256), 0, stream, tokmax, offs, acc,
                       (bf16*)d_key_index, (int)tokens, parts, (int)d_idx);
  } else {
    hipLaunchKernelGGL(kl_reduce_kernel<f16>, rgrid, dim3(256), 0, stream, p.cbuf, p.rowexp, tokmax, offs,
                       posrow, acc, (f16*)d_key_index, (int)tokens, parts, (int)d_idx);
    DSA_HIP(hipGetLastError());
    hipLaunchKernelGGL(kl_reduce_finish_kernel<f16>, fgrid, dim3(256), 0, stream, tokmax, offs, acc,
                       (f16*)d_key_index, (int)tokens, parts, (int)d_idx);
  }
  DSA_HIP(hipGetLastError());
  hipLaunchKernelGGL(kl_loss_kernel, dim3(1), dim3(256), 0, stream, p.loss_part, (int)rows, loss);
  DSA_HIP(hipGetLastError());
  return DSA_OK;
}

}  // namespace dsa
