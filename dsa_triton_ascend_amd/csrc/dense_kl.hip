// Dense lightning-indexer softmax LSE and dense KL-loss backward for gfx950
// (the dense warm-up stage of DSA indexer training).
//
// Semantics follow the reference kernels `_dense_indexer_stats_kernel`,
// `_dense_loss_kernel`, `_dense_main_grad_kernel` and
// `_dense_dkey_index_kernel` (dense_loss_backward_triton.py:129-397).  For a
// query row (b, s1) with s1 < act_q, over the visible keys t < L,
// L = min(max(act_k - act_q + s1 + 1, 0), S2) (lines 139-141):
//   I[t]  = sum_g w_g ReLU(qi_g . ki_t)                                 (56-72)
//   imax  = max_t I, isum = sum_t exp(I - imax)                         (146-177)
//   p[t]  = (1/N1) sum_h exp(s_h[t] - max_h) / (sum_h + 1e-8),
//           s_h[t] = (q_h . k[t, h/G] + qr_h . kr[t, h/G]) * scale      (75-126)
//   student = exp(I - imax) / max(isum, 1e-8), zero unless isum > 0     (204-228)
//   dI = student - p; loss += sum_t P (log P - log Q) with P, Q clamped
//   to 1e-8 (300-318); dW_g = sum_t dI ReLU_g;
//   dQi_g = sum_t dI w_g 1[dot > 0] ki_t (230-249);
//   dKi[t] = sum over rows and g of dI w_g 1[dot > 0] qi_g (384-397).
//
// Design (the reference recomputes the index scores in all four kernels and
// scatters dKi with fp32 atomics):
//  * dense_index_kernel: one workgroup per query row streams the visible key
//    index rows through LDS; 16 index heads per wave on MFMA, the weighted
//    ReLU head-sum as an exact three-part bf16 product with a ones matrix.
//    Writes I to a row-major fp32 buffer [rows, S2] and the row's LSE
//    (online per thread, merged at the end).
//  * dense_teacher_kernel: one workgroup per query row streams K / K_rope
//    through a two-buffer LDS ring.  Waves 0-3 score 32 heads each on the
//    32x32x16 MFMA (Q resident, one key row serves every head); waves 4-7
//    stage the next tile and reduce the previous one: p, then dI = student
//    - p against the index LSE, overwriting I in place; per-row loss.  For
//    GQA the key heads are visited in turn and heads of other key heads
//    are masked.
//  * dense_index_grad_kernel: one workgroup per row: index scores again,
//    dW in registers, dQi^T = Ki^T . dS^T through the transposing LDS read.
//  * dense_dki_kernel: key-major.  A workgroup owns 128 keys (16 per wave,
//    their index rows resident in registers as MFMA B operands) and a slice
//    of the query rows that see them; per row it stages the row's index
//    query in LDS 32 heads at a time, recomputes the ReLU mask, and
//    accumulates dKi^T = Qi^T . C^T with C = dI w 1[dot > 0].  Slices write
//    fp32 partials that dense_dki_reduce_kernel sums in a fixed order, so
//    dKi is deterministic and no atomics are used.
// fp16 operands carry dS scaled by a per-row power of two (from the row's
// max |dI| and max |w|) so that its hi / lo parts stay in the fp16 normal
// range; products are scaled back in fp32.
#include "kl_common.h"

namespace dsa {

struct DkParams {
  const void* q;
  const void* qr;
  const void* k;
  const void* kr;
  const void* qi;
  const void* ki;
  const void* w;
  const float* smax;   // [B, N2, S1, G]
  const float* ssum;
  const float* imax;   // [rows] index LSE used by the backward kernels
  const float* isum;
  float* imax_out;     // [rows] written by dense_index_kernel (may be null)
  float* isum_out;
  const int32_t* act_q;
  const int32_t* act_k;
  float* ibuf;         // [rows, S2]: I, then dI (null: the LSE alone)
  float* loss_part;    // [rows]
  int32_t* dexp;       // [rows] fp16 dS scale exponent
  float* part;         // [splits, B*S2, DI] dKi partials
  void* dqi;
  void* dw;
  int32_t batch, s1, s2, n1, n2, g, nidx, w_dtype, splits;
  float scale_log2;    // scale * log2(e)
};

constexpr int kDkTile = 32;         // keys per tile (row kernels)
constexpr int kDkThreads = 512;     // 8 waves
constexpr int kDkKeys = 128;        // keys per workgroup (dKi kernel)
constexpr int kDkMaxHeads = 128;    // N1 and Nidx1 bound (8 waves x 16)

struct DkRow {
  int b, s1, vis;
  bool valid;
};

__device__ __forceinline__ DkRow dk_row(const DkParams& p, int row) {
  DkRow r;
  r.b = row / p.s1;
  r.s1 = row - r.b * p.s1;
  const int aq = p.act_q ? p.act_q[r.b] : p.s1;
  const int ak = p.act_k ? p.act_k[r.b] : p.s2;
  r.valid = r.s1 < aq;
  r.vis = r.valid ? min(max(ak - aq + r.s1 + 1, 0), p.s2) : 0;
  return r;
}

// fp16 dS scale 2^e with max|dS| * 2^e < 2^14 (bound = max|dI| * max|w|)
__device__ __forceinline__ int dk_scale_exp(float bound) {
  int e = 0;
  if (bound > 0.f) {
    frexpf(bound, &e);
    e = max(-60, min(60, 14 - e));
  }
  return e;
}

// Index-key tile [kDkTile][DI] staged through registers: NJ 16-byte chunks
// per thread, rows past `lim` read as zeros.
template <int DI>
struct KiTile {
  static constexpr int CI = DI / 8;
  static constexpr int NJ = kDkTile * CI / kDkThreads;
  static_assert(kDkTile * CI == NJ * kDkThreads, "index tile assignment");
  u32x4 r[NJ];
  __device__ __forceinline__ void load(const unsigned char* kib, int64_t row0, int t0, int lim, int tid) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = tid + j * kDkThreads;
      const int tk = e / CI, ch = e - tk * CI;
      const u32x4 z = {0u, 0u, 0u, 0u};
      r[j] = t0 + tk < lim ? *(const u32x4*)(kib + (row0 + t0 + tk) * (DI * 2) + ch * 16) : z;
    }
  }
  __device__ __forceinline__ void store(unsigned char* s, int tid) const {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = tid + j * kDkThreads;
      const int tk = e / CI, ch = e - tk * CI;
      *(u32x4*)(s + tk * (DI * 2) + ((ch ^ nope_swz(tk)) * 16)) = r[j];
    }
  }
};

// ---------------------------------------------------------------------------
// index scores I and their LSE
// ---------------------------------------------------------------------------
template <int DI, typename T>
__global__ __launch_bounds__(kDkThreads, 1) void dense_index_kernel(DkParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int TILE = kDkTile;
  constexpr int KSI = DI / 32;
  constexpr int IROW = DI * 2;
  __shared__ __attribute__((aligned(16))) unsigned char s_ki[TILE * IROW];
  __shared__ __attribute__((aligned(16))) float s_redi[8][TILE];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int row = blockIdx.x;
  const DkRow ri = dk_row(p, row);
  if (ri.vis <= 0) {
    if (tid == 0 && p.imax_out) {
      p.imax_out[row] = -INFINITY;
      p.isum_out[row] = 0.f;
    }
    return;
  }
  const int nwi = (p.nidx + 15) >> 4;  // waves with index heads
  const bool iwave = wave < nwi;
  const int g = wave * 16 + li;
  const bool gv = g < p.nidx;
  const int64_t grow = (int64_t)row * p.nidx + (gv ? g : 0);
  const u32x4 z4 = {0u, 0u, 0u, 0u};
  V8 qif[KSI];
#pragma unroll
  for (int ks = 0; ks < KSI; ++ks) {
    const u32x4 v = *(const u32x4*)((const T*)p.qi + grow * DI + ks * 32 + lg * 8);
    qif[ks] = as_v8<V8>(gv ? v : z4);
  }
  float wr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int gg = wave * 16 + lg * 4 + r;
    wr[r] = (iwave && gg < p.nidx) ? load_w(p.w, (int64_t)row * p.nidx + gg, p.w_dtype) : 0.f;
  }
  const unsigned char* kib = (const unsigned char*)p.ki;
  const int64_t krow0 = (int64_t)ri.b * p.s2;
  float m = -INFINITY, s = 0.f;  // online LSE of this thread's keys (threads < TILE)
  KiTile<DI> kt;
  kt.load(kib, krow0, 0, ri.vis, tid);
  for (int t0 = 0; t0 < ri.vis; t0 += TILE) {
    lds_barrier();
    kt.store(s_ki, tid);
    lds_barrier();
    if (t0 + TILE < ri.vis) kt.load(kib, krow0, t0 + TILE, ri.vis, tid);
    if (iwave) {
      f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < KSI; ++ks)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int tk = tt * 16 + li;
          const unsigned char* a = s_ki + tk * IROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16);
          acc[tt] = E::mfma(qif[ks], as_v8<V8>(*(const u32x4*)a), acc[tt]);
        }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        Split3 sp;
#pragma unroll
        for (int r = 0; r < 4; ++r) split3_set(sp, r, wr[r] * relu_bits(acc[tt][r]));
        const f32x4 sum = split3_rowsum(sp);
        if (li == 0) *(f32x4*)&s_redi[wave][tt * 16 + lg * 4] = sum;
      }
    }
    lds_barrier();
    if (tid < TILE) {
      const int t = t0 + tid;
      if (t < ri.vis) {
        float I = 0.f;
        for (int w2 = 0; w2 < nwi; ++w2) I += s_redi[w2][tid];
        if (p.ibuf) p.ibuf[(int64_t)row * p.s2 + t] = I;
        if (I > m) {
          s = s * expf(m - I) + 1.f;
          m = I;
        } else {
          s += expf(I - m);
        }
      }
    }
  }
  if (wave == 0) {
    const float mm = wave_max(m);  // finite: the row has a visible key
    const float ss = wave_sum(m == -INFINITY ? 0.f : s * expf(m - mm));
    if (lane == 0 && p.imax_out) {
      p.imax_out[row] = mm;
      p.isum_out[row] = ss;
    }
  }
}

// ---------------------------------------------------------------------------
// teacher p, dI = student - p (in place over I), per-row loss
// ---------------------------------------------------------------------------
template <int D, int DR, typename T>
__global__ __launch_bounds__(kDkThreads, 1) void dense_teacher_kernel(DkParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int TILE = kDkTile;
  constexpr int NT = kDkThreads;
  constexpr int KS16 = (D + DR) / 16, KSN16 = D / 16;
  constexpr int ROW = D * 2;
  constexpr int CN = D / 8, CR = DR / 8;
  constexpr int NF = NT / 2;  // feed threads (waves 4-7)
  constexpr int NJ_N = TILE * CN / NF;
  static_assert(TILE * CN == NJ_N * NF && TILE * CR <= NF, "tile assignment");
  __shared__ __attribute__((aligned(16))) unsigned char s_k[2][TILE * ROW];
  __shared__ __attribute__((aligned(16))) unsigned char s_kr[2][DR > 0 ? TILE * DR * 2 : 16];
  __shared__ __attribute__((aligned(16))) float s_red[2][4][TILE];
  __shared__ __attribute__((aligned(16))) float s_m2p[128];
  __shared__ __attribute__((aligned(16))) int s_kvh[128];
  // Q rope rows of the 128 heads (A operands of the last k-steps, read
  // just before use: resident they would not fit beside the nope part);
  // 144-byte rows keep a wave's 16-byte reads bank-conflict free
  constexpr int QRR = DR + 8;
  __shared__ __attribute__((aligned(16))) T s_qr[DR > 0 ? 128 * QRR : 8];
  __shared__ float s_wm[8];
  __shared__ float s_kl, s_dmax;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rows = p.batch * p.s1;
  const int row = rows - 1 - (int)blockIdx.x;  // long causal rows first
  const DkRow ri = dk_row(p, row);
  const float isum = p.isum[row];
  const bool has_valid = ri.valid && isum > 0.f;  // reference line 205
  float* irow = p.ibuf + (int64_t)row * p.s2;
  if (!has_valid || ri.vis <= 0) {
    for (int t = tid; t < ri.vis; t += NT) irow[t] = 0.f;
    if (tid == 0) {
      p.loss_part[row] = 0.f;
      p.dexp[row] = 0;
    }
    return;
  }
  const float imax = p.imax[row];
  const float inv_isum = 1.f / fmaxf(isum, 1e-8f);
  const u32x4 z4 = {0u, 0u, 0u, 0u};

  // Waves 0-3 compute: wave w scores heads 32*w .. +31 on
  // v_mfma_f32_32x32x16 (A operand: head 32*w + lane%32, k-step ks = d
  // 16*ks + 8*(lane/32) .. +7, nope k-steps then rope; Q resident).  Waves
  // 4-7 feed: they load the next tile into registers and write it into the
  // two-buffer LDS ring, and wave 4 reduces the previous tile's partial sums
  // into dI.  One barrier per item.
  const bool cwave = wave < 4;
  const bool wave_heads = cwave && wave * 32 < p.n1;
  const int thead = wave * 32 + (lane & 31);
  const bool thv = cwave && thead < p.n1;
  const int64_t hrow = (int64_t)row * p.n1 + (thv ? thead : 0);
  V8 qf[KSN16];
#pragma unroll
  for (int ks = 0; ks < KSN16; ++ks)
    qf[ks] = as_v8<V8>(thv ? *(const u32x4*)((const T*)p.q + hrow * D + ks * 16 + (lane >> 5) * 8) : z4);
  for (int e = tid; e < (DR > 0 ? 128 * (DR / 8) : 0); e += NT) {
    const int h = e / (DR / 8), c = e - h * (DR / 8);
    const int64_t hr = (int64_t)row * p.n1 + (h < p.n1 ? h : 0);
    *(u32x4*)&s_qr[h * QRR + c * 8] = h < p.n1 ? *(const u32x4*)((const T*)p.qr + hr * DR + c * 8) : z4;
  }
  // per head: p = exp2(s*scale*log2e - m2 - log2(l + 1e-8)) (the max and the
  // normalisation folded into one offset; +inf masks heads >= N1) and the
  // key head, -1 past N1.  C register r of the 32x32 product is head 32*w +
  // 8*(r/4) + 4*(lane/32) + r%4, column (key) lane%32.
  for (int h = tid; h < 128; h += NT) {
    const bool v = h < p.n1;
    const int n2 = v ? h / p.g : 0, gg = v ? h - n2 * p.g : 0;
    const int64_t si = (((int64_t)ri.b * p.n2 + n2) * p.s1 + ri.s1) * p.g + gg;
    s_m2p[h] = v ? p.smax[si] * kLog2e + __log2f(p.ssum[si] + 1e-8f) : INFINITY;
    s_kvh[h] = v ? n2 : -1;
  }
  for (int e = tid; e < 2 * 4 * TILE; e += NT) (&s_red[0][0][0])[e] = 0.f;
  const int n2_lo = wave_heads ? (wave * 32) / p.g : 0;
  const int n2_hi = wave_heads ? (min(wave * 32 + 31, p.n1 - 1)) / p.g : -1;
  // row maximum of |w| (fp16 dS scale)
  float wm = 0.f;
  for (int gg = tid; gg < p.nidx; gg += NT) wm = fmaxf(wm, fabsf(load_w(p.w, (int64_t)row * p.nidx + gg, p.w_dtype)));

  const unsigned char* kb = (const unsigned char*)p.k;
  const unsigned char* krb = (const unsigned char*)p.kr;
  const int nt = (ri.vis + TILE - 1) / TILE;
  const int items = nt * p.n2;
  // item i: tile i / N2, key head i % N2; key row (b*S2 + t)*N2 + n2
  const int f = tid - NF;  // feed thread index (>= 0 on waves 4-7)
  // feed thread f loads 16-byte chunk ch0 of keys tk0 + TKS*j (nope) and
  // chunk chr of key tkr (rope)
  constexpr int TKS = NF / CN;
  static_assert(NF % CN == 0 && (DR == 0 || NF == TILE * CR), "feed assignment");
  const int fs = f >= 0 ? f : 0;
  const int tk0 = fs / CN, ch0 = fs - tk0 * CN;
  const int tkr = fs / (CR > 0 ? CR : 1), chr = fs - tkr * CR;
  u32x4 pre_n[NJ_N], pre_r = z4;
  // keys past the row's end load its last visible key instead: their
  // scores are never reduced, and every load stays unconditional (a load
  // under a lane branch makes the compiler wait for all earlier loads)
  const int64_t rb = (int64_t)ri.b * p.s2;
  auto load_item = [&](int i) {
    const int t0 = (i / p.n2) * TILE, n2 = i - (i / p.n2) * p.n2;
#pragma unroll
    for (int j = 0; j < NJ_N; ++j) {
      const int t = min(t0 + tk0 + j * TKS, ri.vis - 1);
      pre_n[j] = *(const u32x4*)(kb + ((rb + t) * p.n2 + n2) * ROW + ch0 * 16);
    }
    if (DR > 0) {
      const int t = min(t0 + tkr, ri.vis - 1);
      pre_r = *(const u32x4*)(krb + ((rb + t) * p.n2 + n2) * (DR * 2) + chr * 16);
    }
  };
  auto store_item = [&](int b) {
#pragma unroll
    for (int j = 0; j < NJ_N; ++j) {
      const int tk = tk0 + j * TKS;
      *(u32x4*)(s_k[b] + tk * ROW + ((ch0 ^ nope_swz(tk)) * 16)) = pre_n[j];
    }
    if (DR > 0) *(u32x4*)(s_kr[b] + tkr * (DR * 2) + ((chr ^ rope_swz(tkr)) * 16)) = pre_r;
  };
  // wave 4, lanes < TILE: the student of a tile (its index scores), loaded
  // one item ahead of the reduction, which turns them into dI in place
  const int q = tid - NF;
  const bool red_lane = q >= 0 && q < TILE;
  float kl = 0.f, dmax = 0.f, pre_i = 0.f, cur_i = 0.f;
  auto reduce_item = [&](int i) {
    const int t = (i / p.n2) * TILE + q;
    if (red_lane && t < ri.vis) {
      float ps = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) ps += s_red[i & 1][w2][q];
      const float pk = ps * (1.f / (float)p.n1);
      const float st = expf(cur_i - imax) * inv_isum;
      const float di = st - pk;
      const float pc = fmaxf(pk, 1e-8f), qc = fmaxf(st, 1e-8f);
      kl += pc * (logf(pc) - logf(qc));
      dmax = fmaxf(dmax, fabsf(di));
      irow[t] = di;
    }
  };

  if (!cwave) {
    load_item(0);
    store_item(0);
    pre_i = irow[min(q & (TILE - 1), ri.vis - 1)];
    if (items > 1) load_item(1);
  }
  float ps_acc = 0.f;
  for (int i = 0; i < items; ++i) {
    const int n2 = i - (i / p.n2) * p.n2;
    const int b = i & 1;
    lds_barrier();
    if (!cwave) {
      // item i+1 into the buffer item i-1 used (every wave is past it)
      if (i + 1 < items) store_item(b ^ 1);
      // the previous item's tile, when that was its last key head
      if (i > 0 && n2 == 0) {
        cur_i = pre_i;
        reduce_item(i - 1);
      }
      // (every feed lane loads, clamped, so that the load is unconditional)
      if (n2 == 0) pre_i = irow[min((i / p.n2) * TILE + (q & (TILE - 1)), ri.vis - 1)];
      if (i + 2 < items) load_item(i + 2);
    } else {
      if (n2 >= n2_lo && n2 <= n2_hi) {
        // S[head][key] on the 32x32x16 MFMA: B operand K[key lane%32][d
        // 16*ks + 8*(lane/32) .. +7].  K fragments read PF k-steps ahead
        // of their MFMA; the scheduling barrier after each MFMA keeps the
        // reads there (one wave per SIMD runs these MFMAs: nothing else
        // hides an LDS round trip).  Chunk 2*ks + hf of key sl sits at
        // (2*ks + hf) ^ swz(sl) = 16*(ks/8) + ((2*(ks%8)) ^ (hf ^ swz)).
        const unsigned char* sk = s_k[b];
        const unsigned char* skr = s_kr[b];
        const int sl = lane & 31, hf = lane >> 5;
        const int xn = hf ^ nope_swz(sl), xr = hf ^ rope_swz(sl);
        auto a_read = [&](int ks) -> u32x4 {
          const unsigned char* a = ks < KSN16 ? sk + sl * ROW + (ks >> 3) * 256 + (((2 * (ks & 7)) ^ xn) * 16)
                                              : skr + sl * (DR * 2) + (((2 * (ks - KSN16)) ^ xr) * 16);
          return *(const u32x4*)a;
        };
        constexpr int PF = 4, KSR16 = KS16 - KSN16;
        f32x16 acc = {};
        u32x4 fa[PF];
        V8 qrf[KSR16 > 0 ? KSR16 : 1];
#pragma unroll
        for (int j = 0; j < PF; ++j) fa[j] = a_read(j);
#pragma unroll
        for (int ks = 0; ks < KS16; ++ks) {
          if (KSR16 > 0 && ks + 2 >= KSN16 && ks + 2 < KS16) {
            const int u = ks + 2 - KSN16;
            qrf[u] = *(const V8*)&s_qr[thead * QRR + u * 16 + hf * 8];
          }
          const V8 bv = as_v8<V8>(fa[ks % PF]);
          if (ks + PF < KS16) fa[ks % PF] = a_read(ks + PF);
          acc = E::mfma32(ks < KSN16 ? qf[ks < KSN16 ? ks : 0] : qrf[ks < KSN16 ? 0 : ks - KSN16], bv, acc);
          __builtin_amdgcn_sched_barrier(0);
        }
        // the lane's 16 heads of key lane%32 (heads of other key heads
        // masked), then the other 16 from lane lane^32
        float ps = 0.f;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int h0 = wave * 32 + 8 * r4 + 4 * hf;
          const f32x4 mo = *(const f32x4*)&s_m2p[h0];
          const i32x4 kv = *(const i32x4*)&s_kvh[h0];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            ps += kv[r] == n2 ? fast_exp2(acc[4 * r4 + r] * p.scale_log2 - mo[r]) : 0.f;
        }
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
        ps_acc += __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      }
      if (n2 == p.n2 - 1) {
        // both halves of the wave hold the sums: no lane branch
        s_red[b][wave][lane & 31] = ps_acc;
        ps_acc = 0.f;
      }
    }
  }
  lds_barrier();
  if (!cwave) {
    cur_i = pre_i;
    reduce_item(items - 1);
  }
  // loss and max |dI| live in wave 4 (lanes < TILE); max |w| in waves 0-1
  kl = wave_sum(kl);
  dmax = wave_max(dmax);
  wm = wave_max(wm);
  if (lane == 0) s_wm[wave] = wm;
  if (tid == NF) {
    s_kl = kl;
    s_dmax = dmax;
  }
  lds_barrier();
  if (tid == 0) {
    float w_all = 0.f;
    for (int w2 = 0; w2 < 8; ++w2) w_all = fmaxf(w_all, s_wm[w2]);
    p.loss_part[row] = s_kl;
    p.dexp[row] = dk_scale_exp(s_dmax * w_all);
  }
}

// ---------------------------------------------------------------------------
// dW and dQi (row-major)
// ---------------------------------------------------------------------------
template <int DI, typename T>
__global__ __launch_bounds__(kDkThreads, 1) void dense_index_grad_kernel(DkParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int TILE = kDkTile;
  constexpr int KSI = DI / 32;
  constexpr int IROW = DI * 2;
  constexpr bool kF16 = __is_same(T, f16);
  __shared__ __attribute__((aligned(16))) unsigned char s_ki[TILE * IROW];
  __shared__ float s_di[TILE];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int rows = p.batch * p.s1;
  const int row = rows - 1 - (int)blockIdx.x;
  const DkRow ri = dk_row(p, row);
  const bool has_valid = ri.valid && p.isum[row] > 0.f;
  if (!has_valid || ri.vis <= 0) {
    for (int e = tid; e < p.nidx * DI; e += kDkThreads)
      ((T*)p.dqi)[(int64_t)row * p.nidx * DI + e] = E::from_f32(0.f);
    for (int gg = tid; gg < p.nidx; gg += kDkThreads) store_w(p.dw, (int64_t)row * p.nidx + gg, p.w_dtype, 0.f);
    return;
  }
  const int nwi = (p.nidx + 15) >> 4;
  const bool iwave = wave < nwi;
  const int g = wave * 16 + li;
  const bool gv = g < p.nidx;
  const int64_t grow = (int64_t)row * p.nidx + (gv ? g : 0);
  const u32x4 z4 = {0u, 0u, 0u, 0u};
  V8 qif[KSI];
#pragma unroll
  for (int ks = 0; ks < KSI; ++ks) {
    const u32x4 v = *(const u32x4*)((const T*)p.qi + grow * DI + ks * 32 + lg * 8);
    qif[ks] = as_v8<V8>(gv ? v : z4);
  }
  const float wg = gv ? load_w(p.w, grow, p.w_dtype) : 0.f;
  float ds_scale = 1.f, ds_unscale = 1.f;
  if (kF16) {
    const int e = p.dexp[row];
    ds_scale = ldexpf(1.f, e);
    ds_unscale = ldexpf(1.f, -e);
  }
  const float* irow = p.ibuf + (int64_t)row * p.s2;
  const unsigned char* kib = (const unsigned char*)p.ki;
  const int64_t krow0 = (int64_t)ri.b * p.s2;

  f32x4 acc_dqi[DI / 16];
#pragma unroll
  for (int dt = 0; dt < DI / 16; ++dt) acc_dqi[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float dw_acc = 0.f;
  KiTile<DI> kt;
  kt.load(kib, krow0, 0, ri.vis, tid);
  float dpre = tid < TILE && tid < ri.vis ? irow[tid] : 0.f;
  for (int t0 = 0; t0 < ri.vis; t0 += TILE) {
    lds_barrier();
    kt.store(s_ki, tid);
    if (tid < TILE) s_di[tid] = dpre;
    lds_barrier();
    if (t0 + TILE < ri.vis) {
      kt.load(kib, krow0, t0 + TILE, ri.vis, tid);
      dpre = tid < TILE && t0 + TILE + tid < ri.vis ? irow[t0 + TILE + tid] : 0.f;
    }
    if (iwave) {
      // C[key 4*lg + r][head li] (keys tt*16 + ..)
      f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < KSI; ++ks)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int tk = tt * 16 + li;
          const unsigned char* a = s_ki + tk * IROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16);
          acc[tt] = E::mfma(as_v8<V8>(*(const u32x4*)a), qif[ks], acc[tt]);
        }
      // dS^T as B operand: k = 8*lg + j is key (j>>2)*16 + 4*lg + (j&3)
      V8 dsf, dsl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tt = j >> 2, r = j & 3;
        const int tk = tt * 16 + lg * 4 + r;
        const float relu = relu_bits(acc[tt][r]);
        const float di = gv ? s_di[tk] : 0.f;  // zero past the visible range
        dw_acc += di * relu;
        const float ds = relu > 0.f ? di * wg * ds_scale : 0.f;
        const T hi = E::from_f32(ds);
        dsf[j] = hi;
        dsl[j] = E::from_f32(ds - E::to_f32(hi));
      }
      // dQi^T[d][g] += Ki^T[d][key] . dS^T[key][g] (Ki^T via the transposing read)
      const int r1 = lg * 4 + (li >> 2);
      const int hb = (li & 3) >> 1;
#pragma unroll
      for (int dt = 0; dt < DI / 16; ++dt) {
        const int ch = 2 * dt + hb;
        const unsigned char* p1 = s_ki + r1 * IROW + ((ch ^ nope_swz(r1)) * 16) + (li & 1) * 8;
        const unsigned char* p2 = s_ki + (r1 + 16) * IROW + ((ch ^ nope_swz(r1 + 16)) * 16) + (li & 1) * 8;
        const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
        const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
        const i16x8 wv = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
        acc_dqi[dt] = E::mfma(__builtin_bit_cast(V8, wv), dsf, acc_dqi[dt]);
        acc_dqi[dt] = E::mfma(__builtin_bit_cast(V8, wv), dsl, acc_dqi[dt]);
      }
    }
  }
  if (iwave) {
    const float dwv = xgroup_sum(dw_acc);
    if (lg == 0 && gv) store_w(p.dw, grow, p.w_dtype, dwv);
    if (gv) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T* dst = (T*)p.dqi + grow * DI;
#pragma unroll
      for (int dt = 0; dt < DI / 16; ++dt) {
        const T4 o = {E::from_f32(acc_dqi[dt][0] * ds_unscale), E::from_f32(acc_dqi[dt][1] * ds_unscale),
                      E::from_f32(acc_dqi[dt][2] * ds_unscale), E::from_f32(acc_dqi[dt][3] * ds_unscale)};
        *(T4*)(dst + dt * 16 + lg * 4) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dKi (key-major partials + fixed-order reduction)
// ---------------------------------------------------------------------------
template <int DI, typename T>
__global__ __launch_bounds__(kDkThreads, 1) void dense_dki_kernel(DkParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KSI = DI / 32;
  constexpr int IROW = DI * 2;
  constexpr int CI = DI / 8;
  constexpr int GC = 32;                       // index heads per staged chunk
  constexpr int NJ = GC * CI / kDkThreads;     // 16-byte chunks per thread
  static_assert(GC * CI == NJ * kDkThreads, "chunk assignment");
  constexpr bool kF16 = __is_same(T, f16);
  __shared__ __attribute__((aligned(16))) unsigned char s_qi[GC * IROW];
  __shared__ float s_w[GC];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int ntiles = (p.s2 + kDkKeys - 1) / kDkKeys;
  const int split = blockIdx.x % p.splits;
  const int bt = blockIdx.x / p.splits;
  const int b = bt / ntiles;
  const int t0 = (bt - b * ntiles) * kDkKeys;
  const int key = t0 + wave * 16 + li;  // this lane's key (MFMA column)
  const bool kv = key < p.s2;
  const u32x4 z4 = {0u, 0u, 0u, 0u};

  // resident index-key fragments (B operand): key li, d = ks*32 + 8*lg ..
  V8 kif[KSI];
  {
    const int64_t kr = (int64_t)b * p.s2 + (kv ? key : 0);
#pragma unroll
    for (int ks = 0; ks < KSI; ++ks) {
      const u32x4 v = *(const u32x4*)((const T*)p.ki + kr * DI + ks * 32 + lg * 8);
      kif[ks] = as_v8<V8>(kv ? v : z4);
    }
  }
  // the query rows of batch b that see any key of the tile, sliced by split
  const int aq = p.act_q ? p.act_q[b] : p.s1;
  const int ak = p.act_k ? p.act_k[b] : p.s2;
  const int lo_all = max(0, t0 - ak + aq);
  const int hi_all = min(aq, p.s1);
  const int cnt = max(hi_all - lo_all, 0);
  const int per = (cnt + p.splits - 1) / p.splits;
  const int r_lo = lo_all + split * per;
  const int r_hi = min(hi_all, r_lo + per);
  const int nchunk = (p.nidx + GC - 1) / GC;

  f32x4 acc[DI / 16];
#pragma unroll
  for (int dt = 0; dt < DI / 16; ++dt) acc[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // items: (row, chunk of 32 index heads), rows with isum <= 0 included
  // (their dI is zero); staged through registers one item ahead
  const int items = max(r_hi - r_lo, 0) * nchunk;
  u32x4 pre[NJ];
  float pre_w = 0.f;
  auto load_item = [&](int i) {
    const int s1 = r_lo + i / nchunk, c = i - (i / nchunk) * nchunk;
    const int64_t row = (int64_t)b * p.s1 + s1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = tid + j * kDkThreads;
      const int gr = e / CI, ch = e - gr * CI;
      const int gg = c * GC + gr;
      pre[j] = gg < p.nidx ? *(const u32x4*)((const unsigned char*)p.qi + (row * p.nidx + gg) * IROW + ch * 16) : z4;
    }
    if (tid < GC) {
      const int gg = c * GC + tid;
      pre_w = gg < p.nidx ? load_w(p.w, row * p.nidx + gg, p.w_dtype) : 0.f;
    }
  };
  if (items > 0) load_item(0);
  float di = 0.f, ds_scale = 1.f, ds_unscale = 1.f;
  for (int i = 0; i < items; ++i) {
    const int s1 = r_lo + i / nchunk, c = i - (i / nchunk) * nchunk;
    const int64_t row = (int64_t)b * p.s1 + s1;
    if (c == 0) {
      // this row's dI at the lane's key (zero past the row's visible range)
      const int vis = min(max(ak - aq + s1 + 1, 0), p.s2);
      di = (kv && key < vis && p.isum[row] > 0.f) ? p.ibuf[row * p.s2 + key] : 0.f;
      if (kF16) {
        const int e = p.dexp[row];
        ds_scale = ldexpf(1.f, e);
        ds_unscale = ldexpf(1.f, -e);
      }
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = tid + j * kDkThreads;
      const int gr = e / CI, ch = e - gr * CI;
      *(u32x4*)(s_qi + gr * IROW + ((ch ^ nope_swz(gr)) * 16)) = pre[j];
    }
    if (tid < GC) s_w[tid] = pre_w;
    lds_barrier();
    if (i + 1 < items) load_item(i + 1);
    // dots C[g = gt*16 + 4*lg + r][key li] over the chunk's 32 heads
    f32x4 dot[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < KSI; ++ks)
#pragma unroll
      for (int gt = 0; gt < 2; ++gt) {
        const int gr = gt * 16 + li;
        const unsigned char* a = s_qi + gr * IROW + (((ks * 4 + lg) ^ nope_swz(gr)) * 16);
        dot[gt] = E::mfma(as_v8<V8>(*(const u32x4*)a), kif[ks], dot[gt]);
      }
    // C^T as B operand: k = 8*lg + j is head (j>>2)*16 + 4*lg + (j&3)
    V8 cf, cl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int gt = j >> 2, r = j & 3;
      const int gr = gt * 16 + lg * 4 + r;
      const float cv = dot[gt][r] > 0.f ? di * s_w[gr] * ds_scale : 0.f;
      const T hi = E::from_f32(cv);
      cf[j] = hi;
      cl[j] = E::from_f32(cv - E::to_f32(hi));
    }
    // dKi^T[d][key] += Qi^T[d][g] . C^T[g][key] (Qi^T via the transposing read)
    const int r1 = lg * 4 + (li >> 2);
    const int hb = (li & 3) >> 1;
#pragma unroll
    for (int dt = 0; dt < DI / 16; ++dt) {
      const int ch = 2 * dt + hb;
      const unsigned char* p1 = s_qi + r1 * IROW + ((ch ^ nope_swz(r1)) * 16) + (li & 1) * 8;
      const unsigned char* p2 = s_qi + (r1 + 16) * IROW + ((ch ^ nope_swz(r1 + 16)) * 16) + (li & 1) * 8;
      const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
      const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
      const i16x8 wv = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
      if (kF16) {
        f32x4 t = E::mfma(__builtin_bit_cast(V8, wv), cf, (f32x4){0.f, 0.f, 0.f, 0.f});
        t = E::mfma(__builtin_bit_cast(V8, wv), cl, t);
        acc[dt] += t * ds_unscale;
      } else {
        acc[dt] = E::mfma(__builtin_bit_cast(V8, wv), cf, acc[dt]);
        acc[dt] = E::mfma(__builtin_bit_cast(V8, wv), cl, acc[dt]);
      }
    }
  }
  // partial [split][b*S2 + key][d]: rows d = dt*16 + 4*lg + r of column key
  if (kv) {
    float* dst = p.part + ((int64_t)split * p.batch * p.s2 + (int64_t)b * p.s2 + key) * DI;
#pragma unroll
    for (int dt = 0; dt < DI / 16; ++dt) *(f32x4*)(dst + dt * 16 + lg * 4) = acc[dt];
  }
}

template <typename T>
__global__ __launch_bounds__(256) void dense_dki_reduce_kernel(const float* part, T* dki, int64_t n4, int splits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  f32x4 s = *(const f32x4*)(part + 4 * i);
  for (int j = 1; j < splits; ++j) s += *(const f32x4*)(part + (int64_t)j * n4 * 4 + 4 * i);
  typedef T T4 __attribute__((ext_vector_type(4)));
  const T4 o = {Elem<T>::from_f32(s[0]), Elem<T>::from_f32(s[1]), Elem<T>::from_f32(s[2]), Elem<T>::from_f32(s[3])};
  *(T4*)(dki + 4 * i) = o;
}

// loss = sum of the per-row terms in a fixed order (one workgroup)
__global__ __launch_bounds__(256) void dense_loss_kernel(const float* part, int rows, float* loss) {
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
static size_t dk_align(size_t x) { return (x + 255) & ~(size_t)255; }

int dense_kl_splits(int64_t batch, int64_t s1, int64_t s2) {
  const int64_t tiles = batch * ((s2 + kDkKeys - 1) / kDkKeys);
  int64_t sp = (512 + tiles - 1) / tiles;
  const int64_t by_rows = (s1 + 31) / 32;  // at least ~32 rows per slice
  if (sp > by_rows) sp = by_rows;
  if (sp > 16) sp = 16;
  if (sp < 1) sp = 1;
  return (int)sp;
}

struct DkWs {
  size_t ibuf, imax, isum, loss, dexp, part, total;
};

static DkWs dk_ws_layout(int64_t batch, int64_t s1, int64_t s2, int64_t di) {
  const int64_t rows = batch * s1;
  DkWs L;
  size_t o = 0;
  L.ibuf = o;
  o += dk_align((size_t)rows * s2 * sizeof(float));
  L.imax = o;
  o += dk_align((size_t)rows * sizeof(float));
  L.isum = o;
  o += dk_align((size_t)rows * sizeof(float));
  L.loss = o;
  o += dk_align((size_t)rows * sizeof(float));
  L.dexp = o;
  o += dk_align((size_t)rows * sizeof(int32_t));
  L.part = o;
  o += dk_align((size_t)dense_kl_splits(batch, s1, s2) * batch * s2 * di * sizeof(float));
  L.total = o;
  return L;
}

size_t dense_kl_workspace_bytes(int64_t batch, int64_t s1, int64_t s2, int64_t di) {
  return dk_ws_layout(batch, s1, s2, di).total;
}

template <typename T>
static hipError_t dk_index(const DkParams& p, int di, hipStream_t stream) {
  const dim3 grid((unsigned)(p.batch * p.s1));
  if (di == 128) hipLaunchKernelGGL((dense_index_kernel<128, T>), grid, dim3(kDkThreads), 0, stream, p);
  else if (di == 256) hipLaunchKernelGGL((dense_index_kernel<256, T>), grid, dim3(kDkThreads), 0, stream, p);
  else hipLaunchKernelGGL((dense_index_kernel<512, T>), grid, dim3(kDkThreads), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t dk_teacher(const DkParams& p, int d, int dr, hipStream_t stream) {
  const dim3 grid((unsigned)(p.batch * p.s1)), blk(kDkThreads);
  if (dr == 64) {
    if (d == 128) hipLaunchKernelGGL((dense_teacher_kernel<128, 64, T>), grid, blk, 0, stream, p);
    else if (d == 256) hipLaunchKernelGGL((dense_teacher_kernel<256, 64, T>), grid, blk, 0, stream, p);
    else hipLaunchKernelGGL((dense_teacher_kernel<512, 64, T>), grid, blk, 0, stream, p);
  } else {
    if (d == 128) hipLaunchKernelGGL((dense_teacher_kernel<128, 0, T>), grid, blk, 0, stream, p);
    else if (d == 256) hipLaunchKernelGGL((dense_teacher_kernel<256, 0, T>), grid, blk, 0, stream, p);
    else hipLaunchKernelGGL((dense_teacher_kernel<512, 0, T>), grid, blk, 0, stream, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t dk_grads(const DkParams& p, int di, void* d_key_index, hipStream_t stream) {
  const dim3 rgrid((unsigned)(p.batch * p.s1)), blk(kDkThreads);
  const int64_t ntiles = (p.s2 + kDkKeys - 1) / kDkKeys;
  const dim3 kgrid((unsigned)(p.batch * ntiles * p.splits));
  if (di == 128) {
    hipLaunchKernelGGL((dense_index_grad_kernel<128, T>), rgrid, blk, 0, stream, p);
    hipLaunchKernelGGL((dense_dki_kernel<128, T>), kgrid, blk, 0, stream, p);
  } else if (di == 256) {
    hipLaunchKernelGGL((dense_index_grad_kernel<256, T>), rgrid, blk, 0, stream, p);
    hipLaunchKernelGGL((dense_dki_kernel<256, T>), kgrid, blk, 0, stream, p);
  } else {
    hipLaunchKernelGGL((dense_index_grad_kernel<512, T>), rgrid, blk, 0, stream, p);
    hipLaunchKernelGGL((dense_dki_kernel<512, T>), kgrid, blk, 0, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t n4 = (int64_t)p.batch * p.s2 * di / 4;
  hipLaunchKernelGGL((dense_dki_reduce_kernel<T>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream,
                     (const float*)p.part, (T*)d_key_index, n4, p.splits);
  return hipGetLastError();
}

static void dk_common(DkParams& p, const void* query_index, const void* key_index, const void* weights,
                      const int32_t* act_q, const int32_t* act_k, int64_t batch, int64_t s1, int64_t s2,
                      int64_t nidx, int32_t w_dtype) {
  p.qi = query_index;
  p.ki = key_index;
  p.w = weights;
  p.act_q = act_q;
  p.act_k = act_k;
  p.batch = (int32_t)batch;
  p.s1 = (int32_t)s1;
  p.s2 = (int32_t)s2;
  p.nidx = (int32_t)nidx;
  p.w_dtype = w_dtype;
  p.splits = 1;
}

int dense_lse_run(const void* query_index, const void* key_index, const void* weights, const int32_t* act_q,
                  const int32_t* act_k, float* max_index, float* sum_index, int64_t batch, int64_t s1,
                  int64_t s2, int64_t nidx, int64_t di, int32_t dtype, int32_t w_dtype, hipStream_t stream) {
  DkParams p{};
  dk_common(p, query_index, key_index, weights, act_q, act_k, batch, s1, s2, nidx, w_dtype);
  p.imax_out = max_index;
  p.isum_out = sum_index;
  DSA_HIP(dtype == DSA_DTYPE_BF16 ? dk_index<bf16>(p, (int)di, stream) : dk_index<f16>(p, (int)di, stream));
  return DSA_OK;
}

int dense_kl_run(const void* query, const void* key, const void* query_rope, const void* key_rope,
                 const void* query_index, const void* key_index, const void* weights, const float* softmax_max,
                 const float* softmax_sum, const float* max_index, const float* sum_index, const int32_t* act_q,
                 const int32_t* act_k, void* d_query_index, void* d_key_index, void* d_weights, float* loss,
                 int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t n2, int64_t d, int64_t d_rope,
                 int64_t nidx, int64_t di, int32_t dtype, int32_t w_dtype, float scale_value, void* workspace,
                 hipStream_t stream) {
  const DkWs L = dk_ws_layout(batch, s1, s2, di);
  unsigned char* ws = (unsigned char*)workspace;
  DkParams p{};
  dk_common(p, query_index, key_index, weights, act_q, act_k, batch, s1, s2, nidx, w_dtype);
  p.q = query;
  p.k = key;
  p.qr = query_rope;
  p.kr = key_rope;
  p.smax = softmax_max;
  p.ssum = softmax_sum;
  p.n1 = (int32_t)n1;
  p.n2 = (int32_t)n2;
  p.g = (int32_t)(n1 / n2);
  p.scale_log2 = scale_value * kLog2e;
  p.ibuf = (float*)(ws + L.ibuf);
  p.loss_part = (float*)(ws + L.loss);
  p.dexp = (int32_t*)(ws + L.dexp);
  p.part = (float*)(ws + L.part);
  p.splits = dense_kl_splits(batch, s1, s2);
  p.dqi = d_query_index;
  p.dw = d_weights;
  // the index scores always; their LSE unless the caller gives it
  if (max_index && sum_index) {
    p.imax = max_index;
    p.isum = sum_index;
  } else {
    p.imax_out = (float*)(ws + L.imax);
    p.isum_out = (float*)(ws + L.isum);
    p.imax = p.imax_out;
    p.isum = p.isum_out;
  }
  const bool bf = dtype == DSA_DTYPE_BF16;
  DSA_HIP(bf ? dk_index<bf16>(p, (int)di, stream) : dk_index<f16>(p, (int)di, stream));
  DSA_HIP(bf ? dk_teacher<bf16>(p, (int)d, (int)d_rope, stream) : dk_teacher<f16>(p, (int)d, (int)d_rope, stream));
  DSA_HIP(bf ? dk_grads<bf16>(p, (int)di, d_key_index, stream) : dk_grads<f16>(p, (int)di, d_key_index, stream));
  hipLaunchKernelGGL(dense_loss_kernel, dim3(1), dim3(256), 0, stream, p.loss_part, (int)(batch * s1), loss);
  DSA_HIP(hipGetLastError());
  return DSA_OK;
}

}  // namespace dsa
