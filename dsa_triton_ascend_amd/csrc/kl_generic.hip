// Sparse lightning-indexer KL-loss backward for the shapes the fused row
// kernel (kl_bwd.hip) does not take: index heads Nidx1 up to 128, any index
// head dim d_idx up to 256 whose rows are whole 16-byte chunks, and any
// topK.  The reference kernel loops over any Nidx1 and D_idx
// (`_indexer_grad_kl_loss_kernel`, sparse_lightning_indexer_grad_kl_loss_triton.py:
// 119-136, 219-262); the semantics are the fused kernel's (the formulas are
// listed at the top of kl_bwd.hip).  The two kernels here write what the
// fused kernel writes (dQi, dW, the per-row KL term, the per-slot dKi
// contributions c as fp16 scaled by 2^rowexp at the slot's place in its
// token's bucket, the row maxima of |c| and, through them, the token
// maxima), so the fixed-point reduce and loss kernels of kl_bwd.hip finish
// the job unchanged.
//  * kl_gen_score_kernel: one workgroup per (row, 64 slots).  The slots'
//    K, K_rope and K_index rows are gathered into LDS; the teacher score
//    S^T[slot][head] and the index score [slot][index head] run on MFMA
//    (16-head tiles, the query fragments of a tile in registers, waves
//    striding over the tiles).  The teacher probability p and the index
//    score I of every slot go to an fp32 [rows, topK, 2] workspace.
//  * kl_gen_row_kernel: one workgroup per row.  Pass B: softmax of I over
//    the row, dI = softmax(I) - p, the KL term.  Pass C, per 32-slot tile:
//    the index scores again, dS = dI * w * 1[relu > 0], dW += dI * relu,
//    dQi += dS^T . Ki and c = dS . Qi, all in fp32 on the vector ALUs
//    (index heads and dims are small next to the teacher's 128 x 576).
// Every sum runs in a fixed order, so the outputs are deterministic.
#include "kl_generic.h"

namespace dsa {

constexpr int kGenSlots = 64;  // slots per score workgroup
constexpr int kGenTile = 32;   // slots per pass-C tile
constexpr int kGenThreads = 256;

// 16-lane sum (the 16 columns of one MFMA C row group)
__device__ __forceinline__ float row16_sum(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

// LDS row strides: 16 bytes of padding make the 16 rows of an MFMA operand
// read (ds_read_b128, one row per lane) fall in different banks.
__host__ __device__ constexpr int gen_row_bytes(int elems) { return elems * 2 + 16; }

template <int D, int DR>
size_t kl_gen_score_lds(int dip) {
  return (size_t)kGenSlots * (gen_row_bytes(D) + (DR > 0 ? gen_row_bytes(DR) : 0) + gen_row_bytes(dip));
}

template <int D, int DR, typename T>
__global__ __launch_bounds__(kGenThreads) void kl_gen_score_kernel(KlGenParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int S = kGenSlots;
  constexpr int RK = gen_row_bytes(D);
  constexpr int RR = DR > 0 ? gen_row_bytes(DR) : 0;
  constexpr int KSN = D / 32, KS = KSN + DR / 32;
  constexpr int KSI_MAX = kGenMaxDi / 32;
  extern __shared__ __attribute__((aligned(16))) unsigned char g_smem[];
  __shared__ int s_tok[S];
  __shared__ float s_pw[4][S];
  __shared__ float s_iw[4][S];
  unsigned char* const s_k = g_smem;
  unsigned char* const s_kr = s_k + S * RK;
  unsigned char* const s_ki = s_kr + S * RR;
  const int RI = gen_row_bytes(p.dip);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int row = blockIdx.x;
  const KlRow ri = kl_row_info(p.m, row);
  const int k0 = blockIdx.y * S;
  if (k0 >= ri.n) return;
  if (tid < S) s_tok[tid] = k0 + tid < ri.n ? kl_token(p.m, ri, p.idx, row, k0 + tid) : -1;
  __syncthreads();
  // gather: 16-byte chunks of the slots' rows; padding slots, -1 pages and
  // index columns past d_idx are zeros
  {
    const int CK = D / 8, CR = DR / 8, CI = p.dip / 8;
    const int per = CK + CR + CI;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int e = tid; e < S * per; e += kGenThreads) {
      const int s = e / per, c = e - s * per;
      const int tok = s_tok[s];
      u32x4 v = z;
      unsigned char* dst;
      if (c < CK) {
        if (tok >= 0) v = *(const u32x4*)((const T*)p.k + (int64_t)tok * D + c * 8);
        dst = s_k + s * RK + c * 16;
      } else if (c < CK + CR) {
        const int cc = c - CK;
        if (tok >= 0) v = *(const u32x4*)((const T*)p.kr + (int64_t)tok * DR + cc * 8);
        dst = s_kr + s * RR + cc * 16;
      } else {
        const int cc = c - CK - CR;
        if (tok >= 0 && cc * 8 < p.di) v = *(const u32x4*)((const T*)p.ki + (int64_t)tok * p.di + cc * 8);
        dst = s_ki + s * RI + cc * 16;
      }
      *(u32x4*)dst = v;
    }
  }
  __syncthreads();

  // teacher: S^T[slot][head] = K . Q^T (A = K rows from LDS, B = Q rows of
  // the tile's heads), C register r of lane (li, lg) = slot 4*lg + r of the
  // m-tile, head li
  float pacc[S / 16][4];
#pragma unroll
  for (int mt = 0; mt < S / 16; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) pacc[mt][r] = 0.f;
  for (int ht = wave; ht * 16 < p.n1; ht += 4) {
    const int h = ht * 16 + li;
    const bool hv = h < p.n1;
    const int64_t hrow = (int64_t)row * p.n1 + (hv ? h : 0);
    V8 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v;
      if (ks < KSN) v = *(const u32x4*)((const T*)p.q + hrow * D + ks * 32 + lg * 8);
      else v = *(const u32x4*)((const T*)p.qr + hrow * DR + (ks - KSN) * 32 + lg * 8);
      qf[ks] = as_v8<V8>(hv ? v : (u32x4){0u, 0u, 0u, 0u});
    }
    const float m2 = hv ? p.smax[hrow] * kLog2e : 0.f;
    const float inv = hv ? 1.f / (p.ssum[hrow] + 1e-8f) : 0.f;
#pragma unroll
    for (int mt = 0; mt < S / 16; ++mt) {
      const int sl = mt * 16 + li;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const unsigned char* a = ks < KSN ? s_k + sl * RK + (ks * 32 + lg * 8) * 2
                                          : s_kr + sl * RR + ((ks - KSN) * 32 + lg * 8) * 2;
        acc = E::mfma(as_v8<V8>(*(const u32x4*)a), qf[ks], acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = hv ? fast_exp2(acc[r] * p.scale_log2 - m2) * inv : 0.f;
        pacc[mt][r] += row16_sum(e);
      }
    }
  }
  // index scores: [slot][g] = Ki . Qi^T, weighted ReLU summed over g
  float iacc[S / 16][4];
#pragma unroll
  for (int mt = 0; mt < S / 16; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) iacc[mt][r] = 0.f;
  const int ksi = p.dip / 32;
  for (int gt = wave; gt * 16 < p.nidx; gt += 4) {
    const int g = gt * 16 + li;
    const bool gv = g < p.nidx;
    const int64_t grow = (int64_t)row * p.nidx + (gv ? g : 0);
    V8 qif[KSI_MAX];
#pragma unroll
    for (int ks = 0; ks < KSI_MAX; ++ks) {
      const int d0 = ks * 32 + lg * 8;
      const bool dv = gv && ks < ksi && d0 < p.di;
      qif[ks] = as_v8<V8>(dv ? *(const u32x4*)((const T*)p.qi + grow * p.di + d0) : (u32x4){0u, 0u, 0u, 0u});
    }
    const float wg = gv ? load_w(p.w, grow, p.w_dtype) : 0.f;
#pragma unroll
    for (int mt = 0; mt < S / 16; ++mt) {
      const int sl = mt * 16 + li;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSI_MAX; ++ks)
        if (ks < ksi) acc = E::mfma(as_v8<V8>(*(const u32x4*)(s_ki + sl * RI + (ks * 32 + lg * 8) * 2)), qif[ks], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) iacc[mt][r] += row16_sum(wg * relu_bits(acc[r]));
    }
  }
  if (li == 0) {
#pragma unroll
    for (int mt = 0; mt < S / 16; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s_pw[wave][mt * 16 + lg * 4 + r] = pacc[mt][r];
        s_iw[wave][mt * 16 + lg * 4 + r] = iacc[mt][r];
      }
  }
  __syncthreads();
  if (tid < S && k0 + tid < ri.n) {
    const float ps = s_pw[0][tid] + s_pw[1][tid] + s_pw[2][tid] + s_pw[3][tid];
    const float is = s_iw[0][tid] + s_iw[1][tid] + s_iw[2][tid] + s_iw[3][tid];
    float2* o = (float2*)p.pi + (int64_t)row * p.topk + k0 + tid;
    *o = make_float2(ps * (1.f / (float)p.n1), is);
  }
}

// workgroup reductions (fixed order: butterfly in the wave, then the waves
// in order); s_red holds 4 words
__device__ __forceinline__ float block_max4(float v, float* s_red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
}
__device__ __forceinline__ float block_sum4(float v, float* s_red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
}

template <typename T>
__global__ __launch_bounds__(kGenThreads) void kl_gen_row_kernel(KlGenParams p) {
  using E = Elem<T>;
  typedef T T8 __attribute__((ext_vector_type(8)));
  typedef _Float16 H8 __attribute__((ext_vector_type(8)));
  constexpr int TL = kGenTile;
  constexpr int GPT = kGenMaxNidx / 8;     // index heads per thread in the score step (8 head groups)
  constexpr int CPT = kGenMaxDi / 8 / 8;   // 8-column chunks per thread in the c step (8 chunk groups)
  constexpr int QPT = 16;                  // (head, chunk) rows of dQi per thread
  extern __shared__ __attribute__((aligned(16))) unsigned char g_smem[];
  __shared__ float s_red[4];
  __shared__ float s_dI[TL];
  __shared__ int s_tok[TL];
  __shared__ int s_pos[TL];  // the slots' places in their tokens' buckets
  __shared__ float s_w[kGenMaxNidx];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const KlRow ri = kl_row_info(p.m, row);
  const int n = ri.n, ni = p.nidx, di = p.di, nch = di / 8;
  const int RQ = gen_row_bytes(di);  // bytes per Qi / Ki row in LDS
  unsigned char* const s_qi = g_smem;                     // [ni][RQ]
  unsigned char* const s_ki = s_qi + ni * RQ;             // [TL][RQ]
  float* const s_ds = (float*)(s_ki + TL * RQ);           // [TL][ni + 1]
  const int DSR = ni + 1;

  if (n <= 0) {
    // inactive or empty row: zero gradients, no loss
    for (int e = tid; e < ni * di; e += kGenThreads) ((T*)p.dqi)[(int64_t)row * ni * di + e] = E::from_f32(0.f);
    for (int g = tid; g < ni; g += kGenThreads) store_w(p.dw, (int64_t)row * ni + g, p.w_dtype, 0.f);
    if (tid == 0) {
      p.loss_part[row] = 0.f;
      p.rowmax[row] = 0.f;
      p.rowexp[row] = 0;
    }
    return;
  }
  float2* const pi = (float2*)p.pi + (int64_t)row * p.topk;

  // ---- pass B: softmax(I), dI = softmax(I) - p, KL ----
  float mx = -INFINITY;
  for (int k = tid; k < n; k += kGenThreads) mx = fmaxf(mx, pi[k].y);
  mx = block_max4(mx, s_red);
  float sm = 0.f;
  for (int k = tid; k < n; k += kGenThreads) sm += expf(pi[k].y - mx);
  sm = block_sum4(sm, s_red);
  const float inv = 1.f / (sm + 1e-8f);
  float kl = 0.f, dmax = 0.f;
  for (int k = tid; k < n; k += kGenThreads) {
    const float2 v = pi[k];
    const float sI = expf(v.y - mx) * inv;
    const float dI = sI - v.x;
    const float P = fmaxf(v.x, 1e-8f), Q = fmaxf(sI, 1e-8f);
    kl += P * (logf(P) - logf(Q));
    dmax = fmaxf(dmax, fabsf(dI));
    pi[k].x = dI;  // read back by other threads after the barriers below
  }
  kl = block_sum4(kl, s_red);
  dmax = block_max4(dmax, s_red);

  // ---- the row's Qi and weights; the scale of the fp16 contributions ----
  float qm = 0.f;
  for (int e = tid; e < ni * nch; e += kGenThreads) {
    const int g = e / nch, c = e - g * nch;
    const T8 v = *(const T8*)((const T*)p.qi + ((int64_t)row * ni + g) * di + c * 8);
    *(T8*)(s_qi + g * RQ + c * 16) = v;
#pragma unroll
    for (int j = 0; j < 8; ++j) qm = fmaxf(qm, fabsf(E::to_f32(v[j])));
  }
  float wsum = 0.f;
  for (int g = tid; g < ni; g += kGenThreads) {
    const float w = load_w(p.w, (int64_t)row * ni + g, p.w_dtype);
    s_w[g] = w;
    wsum += fabsf(w);
  }
  qm = block_max4(qm, s_red);
  wsum = block_sum4(wsum, s_red);
  // |c[slot][j]| = |sum_g dS[g][slot] Qi[g][j]| <= max|dI| * sum_g |w_g| *
  // max|Qi|; with that bound below 2^(14 - e) the stored c * 2^e stays in
  // fp16's normal range
  int c_exp = 0;
  {
    const float bound = dmax * wsum * qm;
    if (bound > 0.f && bound < INFINITY) {
      int e;
      frexpf(bound, &e);
      c_exp = max(-100, min(100, 14 - e));
    }
  }
  const float c_scale = ldexpf(1.f, c_exp);

  // ---- pass C ----
  // score step: slot ks = tid % 32, index heads g = hg + 8 j (hg = tid / 32)
  const int ks_ = tid & 31, hg = tid >> 5;
  float dw_acc[GPT];
#pragma unroll
  for (int j = 0; j < GPT; ++j) dw_acc[j] = 0.f;
  // dQi step: column chunk qc = tid % nch, heads g = qg + qstep * j
  const int qc = tid % nch, qg = tid / nch, qstep = kGenThreads / nch;
  float dq[QPT][8];
#pragma unroll
  for (int j = 0; j < QPT; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) dq[j][e] = 0.f;
  float cmax = 0.f;
  for (int t0 = 0; t0 < n; t0 += TL) {
    __syncthreads();  // the previous tile's Ki / dS are consumed
    if (tid < TL) {
      const int k = t0 + tid;
      const int tok = k < n ? kl_token(p.m, ri, p.idx, row, k) : -1;
      const int pos = tok < 0 ? -1
                      : p.offs[tok] + p.rank[(int64_t)row * p.topk + k] +
                            (p.cbase ? p.cbase[(int64_t)(row / p.chunk_rows) * p.tokens + tok] : 0);
      s_tok[tid] = tok;
      s_pos[tid] = pos;
      if (pos >= 0) p.posrow[pos] = row;
      s_dI[tid] = k < n ? pi[k].x : 0.f;
    }
    __syncthreads();
    for (int e = tid; e < TL * nch; e += kGenThreads) {
      const int s = e / nch, c = e - s * nch;
      const int tok = s_tok[s];
      T8 v = {};
      if (tok >= 0) v = *(const T8*)((const T*)p.ki + (int64_t)tok * di + c * 8);
      *(T8*)(s_ki + s * RQ + c * 16) = v;
    }
    __syncthreads();
    // index scores of slot ks_ and heads hg + 8 j; dS, dW
    {
      const float dI = s_dI[ks_];
      const unsigned char* kr = s_ki + ks_ * RQ;
#pragma unroll
      for (int j = 0; j < GPT; ++j) {
        const int g = hg + 8 * j;
        if (g < ni) {
          const unsigned char* qr = s_qi + g * RQ;
          float s = 0.f;
          for (int c = 0; c < nch; ++c) {
            const T8 a = *(const T8*)(qr + c * 16), b = *(const T8*)(kr + c * 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf(E::to_f32(a[e]), E::to_f32(b[e]), s);
          }
          const float relu = relu_bits(s);
          dw_acc[j] = fmaf(dI, relu, dw_acc[j]);
          s_ds[ks_ * DSR + g] = s > 0.f ? dI * s_w[g] : 0.f;
        }
      }
    }
    __syncthreads();
    // c[slot][chunk] = sum_g dS[slot][g] Qi[g][chunk]: slot ks_, chunks hg + 8 j
    {
      const int k = t0 + ks_;
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int c = hg + 8 * j;
        if (c < nch) {
          float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          for (int g = 0; g < ni; ++g) {
            const float ds = s_ds[ks_ * DSR + g];
            const T8 q = *(const T8*)(s_qi + g * RQ + c * 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = fmaf(ds, E::to_f32(q[e]), a[e]);
          }
          if (k < n) {
            H8 h;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              cmax = __builtin_elementwise_maximum(cmax, fabsf(a[e]));  // NaN-propagating
              h[e] = (_Float16)(a[e] * c_scale);
            }
            const int pos = s_pos[ks_];
            if (pos >= 0) *(H8*)(p.cbuf + (int64_t)pos * di + c * 8) = h;
          }
        }
      }
    }
    // dQi[g][chunk qc] += sum_slot dS[slot][g] Ki[slot][chunk qc]
    if (qg < qstep) {
#pragma unroll
      for (int j = 0; j < QPT; ++j) {
        const int g = qg + qstep * j;
        if (g < ni) {
          for (int s = 0; s < TL; ++s) {
            const float ds = s_ds[s * DSR + g];
            const T8 kv = *(const T8*)(s_ki + s * RQ + qc * 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) dq[j][e] = fmaf(ds, E::to_f32(kv[e]), dq[j][e]);
          }
        }
      }
    }
  }
  __syncthreads();
  // ---- epilogue ----
  // dQi
#pragma unroll
  for (int j = 0; j < QPT; ++j) {
    const int g = qg + qstep * j;
    if (qg < qstep && g < ni) {
      T8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = E::from_f32(dq[j][e]);
      *(T8*)((T*)p.dqi + ((int64_t)row * ni + g) * di + qc * 8) = o;
    }
  }
  // dW: the 32 slot threads' partial sums of each head, added in slot order
#pragma unroll
  for (int j = 0; j < GPT; ++j) {
    const int g = hg + 8 * j;
    if (g < ni) s_ds[ks_ * DSR + g] = dw_acc[j];
  }
  __syncthreads();
  for (int g = tid; g < ni; g += kGenThreads) {
    float a = 0.f;
    for (int s = 0; s < TL; ++s) a += s_ds[s * DSR + g];
    store_w(p.dw, (int64_t)row * ni + g, p.w_dtype, a);
  }
  // a non-finite contribution (NaN kept above) makes the row maximum
  // infinite: NaN dKi for the row's tokens in the reduction
  cmax = block_max4(cmax < INFINITY ? cmax : INFINITY, s_red);
  if (tid == 0) {
    p.loss_part[row] = kl;
    p.rowmax[row] = cmax;
    p.rowexp[row] = c_exp;
  }
  // the row maximum raises its tokens' maxima (non-negative floats order as
  // their bit patterns)
  for (int k = tid; k < n; k += kGenThreads) {
    const int tok = kl_token(p.m, ri, p.idx, row, k);
    if (tok >= 0) atomicMax(&p.tokmax[tok], __float_as_uint(cmax));
  }
}

size_t kl_gen_row_lds(int nidx, int di) {
  return (size_t)(nidx + kGenTile) * gen_row_bytes(di) + (size_t)kGenTile * (nidx + 1) * sizeof(float);
}

template <int D, int DR, typename T>
static hipError_t launch_gen(const KlGenParams& p, int rows, hipStream_t stream) {
  const size_t lds_s = kl_gen_score_lds<D, DR>(p.dip);
  const void* fs = (const void*)kl_gen_score_kernel<D, DR, T>;
  hipError_t e = hipFuncSetAttribute(fs, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_s);
  if (e != hipSuccess) return e;
  const dim3 sgrid((unsigned)rows, (unsigned)((p.topk + kGenSlots - 1) / kGenSlots));
  hipLaunchKernelGGL((kl_gen_score_kernel<D, DR, T>), sgrid, dim3(kGenThreads), lds_s, stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds_r = kl_gen_row_lds(p.nidx, p.di);
  const void* fr = (const void*)kl_gen_row_kernel<T>;
  e = hipFuncSetAttribute(fr, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_r);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kl_gen_row_kernel<T>, dim3((unsigned)rows), dim3(kGenThreads), lds_r, stream, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t dispatch_gen(const KlGenParams& p, int rows, int d, int dr, hipStream_t stream) {
  if (dr == 64) {
    if (d == 128) return launch_gen<128, 64, T>(p, rows, stream);
    if (d == 256) return launch_gen<256, 64, T>(p, rows, stream);
    return launch_gen<512, 64, T>(p, rows, stream);
  }
  if (d == 128) return launch_gen<128, 0, T>(p, rows, stream);
  if (d == 256) return launch_gen<256, 0, T>(p, rows, stream);
  return launch_gen<512, 0, T>(p, rows, stream);
}

hipError_t kl_gen_run(const KlGenParams& p, int rows, int d, int dr, bool bf16_io, hipStream_t stream) {
  return bf16_io ? dispatch_gen<bf16>(p, rows, d, dr, stream) : dispatch_gen<f16>(p, rows, d, dr, stream);
}

}  // namespace dsa
