// Sparse flash attention backward for gfx950 (MLA-absorb, MQA).
//
// Semantics follow the reference kernel `_sfa_grad_kernel`
// (sparse_flash_attention_grad_triton.py:158-308) and its golden
// (sparse_flash_attention_grad_numpy.py:34-143).  For every active query row
// and every attended token (the forward's masks), with v = key[:, :D]:
//   s     = (q_nope.k_nope + q_rope.k_rope) * scale
//   P     = exp(s - softmax_max) / softmax_sum   (sum <= 0 taken as 1, 233-234)
//   delta = sum_d dO * O                          (237)
//   dS    = P * (dO.v - delta) * scale            (262-267)
//   dq += dS k_nope,  dq_rope += dS k_rope        (271-272)
//   dk += dS^T q_nope, dk_rope += dS^T q_rope, dv += P^T dO   (277-300)
// dq / dq_rope are owned per (row, head) and stored in the query dtype; dk,
// dk_rope and dv are scatter-added in fp32 (many rows select one key row;
// the order of the fp32 additions is not fixed, as in the reference, which
// rejects deterministic=True) and cast to the key dtype afterwards.
//
// Design (one wave = one query row x 16 heads; 1 wave per SIMD, so the wave
// has the whole 512-register file):
//  * Q (nope + rope) and dO fragments of the 16 heads sit in registers as
//    MFMA B operands; so do their transposes Q^T / dO^T (4 heads x 1 column
//    per lane), the B operands of the dK / dV products, built once through
//    LDS.  Per-head statistics (max in log2 units, 1/sum, delta) are
//    lane-local, one head per lane column.
//  * Tiles of 32 attended tokens are gathered into LDS (swizzled 16-byte
//    chunks, the forward's layout).  S^T = K.Q^T and dP^T = K_nope.dO^T share
//    the K fragment reads; P^T and dS^T come out lane-local.
//  * dq^T += K^T.dS^T and dq_rope^T += Kr^T.dS^T read K^T through the
//    transposing LDS load (ds_read_b64_tr_b16), as the forward's P.V.
//  * dS and P go through a 1 KB LDS transpose into the A operand of
//    v_mfma_f32_16x16x16 (tokens x 16 heads); dK/dK_rope = dS^T.Q and
//    dV = P^T.dO come out as 16 tokens x 16 columns tiles whose fp32 values
//    are added to the workspaces with global atomics.
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
  float* dk;
  float* dkr;
  float* dv;
  int64_t rows, kv_rows;
  int32_t batch, s1, s2, n1, K, bs, mode, layout_q, layout_kv, max_blocks, page_size;
  float scale, scale_log2;
};

constexpr int kBwdTile = 32;
constexpr int kBwdList = 2048;  // attended positions resolved per compaction round


template <typename T>
__device__ __forceinline__ short to_bits(float x) {
  return __builtin_bit_cast(short, Elem<T>::from_f32(x));
}

template <int D, typename T>
__global__ __launch_bounds__(64, 1) void sfa_bwd_kernel(SfaBwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int DR = 64;
  constexpr int DC = D + DR;         // columns of dK + dK_rope
  constexpr int KS = DC / 32;        // k-steps of S
  constexpr int KSN = D / 32;        // of which nope
  constexpr int NDT = D / 16;        // d-tiles of dq / dv
  constexpr int NCT = DC / 16;       // column tiles of dk + dk_rope
  constexpr int TILE = kBwdTile;
  constexpr int ROW = D * 2;         // nope row bytes in LDS
  constexpr int QST = DC + 16;       // staging row (elements), padded
  static_assert(D >= 128 && TILE == 32, "layout");

  __shared__ __attribute__((aligned(16))) unsigned char s_k[TILE * ROW];
  __shared__ __attribute__((aligned(16))) unsigned char s_kr[TILE * DR * 2];
  __shared__ int s_list[kBwdList + TILE];
  // dS and P as [token][head], each as a hi and a lo part (bf16 I/O)
  __shared__ __attribute__((aligned(16))) T s_tr[4][TILE][16];

  const int lane = threadIdx.x;
  const int li = lane & 15, lg = lane >> 4;
  const int row = blockIdx.x;
  const int head0 = blockIdx.y * 16;
  const RowInfo ri = sfa_row_info(p, row);
  const int64_t total_pos = (int64_t)p.K * p.bs;
  const int32_t* idx_row = p.idx + (int64_t)row * p.K;

  // ---- per-lane head (head0 + li): fragments and statistics ----
  const int head = head0 + li;
  const bool hv = head < p.n1;
  const int64_t hrow = (int64_t)row * p.n1 + (hv ? head : 0);
  V8 qf[KS], dof[KSN];
  const u32x4 z4 = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    u32x4 v;
    if (ks < KSN) v = *(const u32x4*)((const T*)p.q + hrow * D + ks * 32 + lg * 8);
    else v = *(const u32x4*)((const T*)p.qr + hrow * DR + (ks - KSN) * 32 + lg * 8);
    qf[ks] = as_v8<V8>(hv ? v : z4);
  }
  float delta = 0.f;
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks) {
    const u32x4 v = *(const u32x4*)((const T*)p.dout + hrow * D + ks * 32 + lg * 8);
    const u32x4 o = *(const u32x4*)((const T*)p.out + hrow * D + ks * 32 + lg * 8);
    dof[ks] = as_v8<V8>(hv ? v : z4);
    const V8 dv8 = as_v8<V8>(v), ov8 = as_v8<V8>(o);
#pragma unroll
    for (int j = 0; j < 8; ++j) delta += E::to_f32(dv8[j]) * E::to_f32(ov8[j]);
  }
  delta = xgroup_sum(delta);  // lanes li, li+16, li+32, li+48 cover all D columns
  float m2 = 0.f, inv = 0.f;
  if (hv) {
    const float sm = p.smax[hrow], ss = p.ssum[hrow];
    m2 = sm * kLog2e;
    inv = 1.f / (ss > 0.f ? ss : 1.f);
  } else {
    delta = 0.f;
  }

  // transposed fragments (B operands of the 16x16x16 products):
  // qT[c] = Q[heads 4*lg + j][column c*16 + li], dT[c] = dO[...] likewise,
  // built through LDS (rows of 16 heads, padded to QST elements)
  s16x4 qT[NCT], dT[NDT];
  {
    T* st = (T*)s_k;  // 16 x QST elements fit in the tile buffer
    static_assert(16 * QST * 2 <= TILE * ROW, "staging fits");
    for (int e = lane; e < 16 * DC; e += 64) {
      const int h = e / DC, c = e - h * DC;
      const int hh = head0 + h;
      T v = E::from_f32(0.f);
      if (hh < p.n1) {
        const int64_t r = (int64_t)row * p.n1 + hh;
        v = c < D ? ((const T*)p.q)[r * D + c] : ((const T*)p.qr)[r * DR + (c - D)];
      }
      st[h * QST + c] = v;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      s16x4 f;
#pragma unroll
      for (int j = 0; j < 4; ++j) f[j] = __builtin_bit_cast(short, st[(4 * lg + j) * QST + c * 16 + li]);
      qT[c] = f;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    for (int e = lane; e < 16 * D; e += 64) {
      const int h = e / D, c = e - h * D;
      const int hh = head0 + h;
      T v = E::from_f32(0.f);
      if (hh < p.n1) v = ((const T*)p.dout)[((int64_t)row * p.n1 + hh) * D + c];
      st[h * QST + c] = v;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < NDT; ++c) {
      s16x4 f;
#pragma unroll
      for (int j = 0; j < 4; ++j) f[j] = __builtin_bit_cast(short, st[(4 * lg + j) * QST + c * 16 + li]);
      dT[c] = f;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
  }

  f32x4 acc_dq[NDT], acc_dqr[DR / 16];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_dq[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dt = 0; dt < DR / 16; ++dt) acc_dqr[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // per-lane LDS offsets (tile rows are D*2 / 128 bytes; chunk swizzles as
  // in the forward)
  auto a1_off = [&](int ks, int tt) -> int {
    const int tk = tt * 16 + li;
    if (ks < KSN) return tk * ROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16);
    return tk * (DR * 2) + ((((ks - KSN) * 4 + lg) ^ rope_swz(tk)) * 16);
  };

  for (int64_t c0 = 0; c0 < total_pos; c0 += kBwdList) {
    // ---- compact this range of positions into s_list ----
    const int64_t c1 = min(total_pos, c0 + (int64_t)kBwdList);
    int n_valid = 0;
    for (int64_t b0 = c0; b0 < c1; b0 += 64) {
      const int64_t pos = b0 + lane;
      int phys = 0;
      bool valid = false;
      if (ri.active && pos < c1) valid = sfa_resolve(p, ri, idx_row, (int)pos, &phys);
      const unsigned long long m = __ballot(valid);
      if (valid) s_list[n_valid + __popcll(m & ((1ull << lane) - 1ull))] = phys;
      n_valid += __popcll(m);
    }
    if (lane < TILE) s_list[n_valid + lane] = -1;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const int n_tiles = (n_valid + TILE - 1) / TILE;

    for (int t = 0; t < n_tiles; ++t) {
      // ---- gather the tile (16-byte chunks, swizzled) ----
      constexpr int CPR = D / 8;  // nope chunks per row
#pragma unroll 4
      for (int e = lane; e < TILE * CPR; e += 64) {
        const int tk = e / CPR, ch = e - tk * CPR;
        const int ph = s_list[t * TILE + tk];
        u32x4 v = z4;
        if (ph >= 0) v = *(const u32x4*)((const unsigned char*)p.k + (int64_t)ph * (D * 2) + ch * 16);
        *(u32x4*)(s_k + tk * ROW + ((ch ^ nope_swz(tk)) * 16)) = v;
      }
#pragma unroll
      for (int e = lane; e < TILE * 8; e += 64) {
        const int tk = e >> 3, ch = e & 7;
        const int ph = s_list[t * TILE + tk];
        u32x4 v = z4;
        if (ph >= 0) v = *(const u32x4*)((const unsigned char*)p.kr + (int64_t)ph * (DR * 2) + ch * 16);
        *(u32x4*)(s_kr + tk * (DR * 2) + ((ch ^ rope_swz(tk)) * 16)) = v;
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();

      // ---- S^T = K.Q^T and dP^T = K_nope.dO^T (shared K fragments) ----
      f32x4 acc_s[2], acc_p[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        acc_s[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        acc_p[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const unsigned char* base = ks < KSN ? s_k : s_kr;
          const V8 av = as_v8<V8>(*(const u32x4*)(base + a1_off(ks, tt)));
          acc_s[tt] = E::mfma(av, qf[ks], acc_s[tt]);
          if (ks < KSN) acc_p[tt] = E::mfma(av, dof[ks], acc_p[tt]);
        }

      // ---- P^T, dS^T (token tt*16 + 4*lg + r, head li) ----
      // dS^T as the B operand of K^T.dS^T (token k = 8*lg + j).  For bf16 I/O
      // dS (and P below) are split into bf16 hi + lo parts, so the products
      // carry ~16 bits of them: a single bf16 rounding (2^-9 relative per
      // term) exceeds the fp32-golden tolerance on rows with few tokens.
      constexpr bool kSplit = __is_same(T, bf16);
      V8 dsf, dsf_lo;
      float pv[8], dsv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tt = j >> 2, r = j & 3;
        const int tok = t * TILE + tt * 16 + lg * 4 + r;
        const bool tv = tok < n_valid;
        const float pp = tv ? fast_exp2(acc_s[tt][r] * p.scale_log2 - m2) * inv : 0.f;
        const float ds = pp * (acc_p[tt][r] - delta) * p.scale;
        pv[j] = pp;
        dsv[j] = ds;
        dsf[j] = E::from_f32(ds);
        dsf_lo[j] = E::from_f32(ds - E::to_f32(dsf[j]));
      }

      // ---- dq^T += K^T.dS^T, dq_rope^T += Kr^T.dS^T ----
      // K^T fragment (16 d x 32 tokens) through the transposing read: row
      // r1 = 4*lg + li/4 (and r1 + 16), chunk 2*dt + (li&3)/2, half li&1
      {
        const int r1 = lg * 4 + (li >> 2);
        const int hb = (li & 3) >> 1;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int ch = 2 * dt + hb;
          const unsigned char* p1 = s_k + r1 * ROW + ((ch ^ nope_swz(r1)) * 16) + (li & 1) * 8;
          const unsigned char* p2 = s_k + (r1 + 16) * ROW + ((ch ^ nope_swz(r1 + 16)) * 16) + (li & 1) * 8;
          const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
          const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
          const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
          acc_dq[dt] = E::mfma(__builtin_bit_cast(V8, w), dsf, acc_dq[dt]);
          if (kSplit) acc_dq[dt] = E::mfma(__builtin_bit_cast(V8, w), dsf_lo, acc_dq[dt]);
        }
#pragma unroll
        for (int dt = 0; dt < DR / 16; ++dt) {
          const int ch = 2 * dt + hb;
          const unsigned char* p1 = s_kr + r1 * (DR * 2) + ((ch ^ rope_swz(r1)) * 16) + (li & 1) * 8;
          const unsigned char* p2 = s_kr + (r1 + 16) * (DR * 2) + ((ch ^ rope_swz(r1 + 16)) * 16) + (li & 1) * 8;
          const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
          const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
          const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
          acc_dqr[dt] = E::mfma(__builtin_bit_cast(V8, w), dsf, acc_dqr[dt]);
          if (kSplit) acc_dqr[dt] = E::mfma(__builtin_bit_cast(V8, w), dsf_lo, acc_dqr[dt]);
        }
      }

      // ---- dS, P -> [token][head] in LDS, then 16x16x16 A fragments ----
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tk = (j >> 2) * 16 + lg * 4 + (j & 3);
        const T dh = E::from_f32(dsv[j]), ph = E::from_f32(pv[j]);
        s_tr[0][tk][li] = dh;
        s_tr[1][tk][li] = ph;
        s_tr[2][tk][li] = E::from_f32(dsv[j] - E::to_f32(dh));
        s_tr[3][tk][li] = E::from_f32(pv[j] - E::to_f32(ph));
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        // A[token tt*16 + li][heads 4*lg ..]: 8 bytes
        const s16x4 a_ds = *(const s16x4*)&s_tr[0][tt * 16 + li][4 * lg];
        const s16x4 a_p = *(const s16x4*)&s_tr[1][tt * 16 + li][4 * lg];
        const s16x4 a_ds_lo = *(const s16x4*)&s_tr[2][tt * 16 + li][4 * lg];
        const s16x4 a_p_lo = *(const s16x4*)&s_tr[3][tt * 16 + li][4 * lg];
        // token rows of this lane's C entries: tt*16 + 4*lg + r
        int ph[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ph[r] = s_list[t * TILE + tt * 16 + lg * 4 + r];
#pragma unroll
        for (int c = 0; c < NCT; ++c) {
          f32x4 cd = Mfma16<T>::run(a_ds, qT[c], (f32x4){0.f, 0.f, 0.f, 0.f});
          if (kSplit) cd = Mfma16<T>::run(a_ds_lo, qT[c], cd);
          const int col = c * 16 + li;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (ph[r] < 0) continue;
            if (col < D) atomicAdd(p.dk + (int64_t)ph[r] * D + col, cd[r]);
            else atomicAdd(p.dkr + (int64_t)ph[r] * DR + (col - D), cd[r]);
          }
        }
#pragma unroll
        for (int c = 0; c < NDT; ++c) {
          f32x4 cv = Mfma16<T>::run(a_p, dT[c], (f32x4){0.f, 0.f, 0.f, 0.f});
          if (kSplit) cv = Mfma16<T>::run(a_p_lo, dT[c], cv);
          const int col = c * 16 + li;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (ph[r] >= 0) atomicAdd(p.dv + (int64_t)ph[r] * D + col, cv[r]);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---- dq, dq_rope (head li, columns 16*dt + 4*lg + r) ----
  if (hv) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T* dqp = (T*)p.dq + hrow * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const T4 o = {E::from_f32(acc_dq[dt][0]), E::from_f32(acc_dq[dt][1]), E::from_f32(acc_dq[dt][2]),
                    E::from_f32(acc_dq[dt][3])};
      *(T4*)(dqp + dt * 16 + lg * 4) = o;
    }
    T* dqrp = (T*)p.dqr + hrow * DR;
#pragma unroll
    for (int dt = 0; dt < DR / 16; ++dt) {
      const T4 o = {E::from_f32(acc_dqr[dt][0]), E::from_f32(acc_dqr[dt][1]), E::from_f32(acc_dqr[dt][2]),
                    E::from_f32(acc_dqr[dt][3])};
      *(T4*)(dqrp + dt * 16 + lg * 4) = o;
    }
  }
}

// ---------------------------------------------------------------------------
// Workgroup kernel: 4 waves x 16 heads = 64 heads of one query row.
//
// Per tile of 32 attended tokens (LDS ring of two buffers, filled by LDS DMA
// right after the previous tile's barrier, so a tile's gather overlaps the
// previous tile's products):
//  * each wave: S^T, dP^T, P, dS and dq / dq_rope for its 16 heads, as the
//    one-wave kernel above;
//  * dS and P of the 64 heads go to LDS as [token][head] (bf16 / fp16);
//  * each wave then owns a quarter of the 2D + 64 output columns (dK, dK_rope,
//    dV) and sums them over all 64 heads on MFMA: A = dS^T or P^T [16 tokens
//    x 32 heads] from LDS, B = Q / Q_rope / dO [32 heads x 16 columns]
//    resident in registers for the row; the sums go to the fp32 workspaces.
// The 64-head sum cuts the scatter payload by 4 against one wave per 16
// heads.  One wave per SIMD: each wave has the whole 512-register file.
// ---------------------------------------------------------------------------
constexpr int kBwdWgWaves = 4;
constexpr int kBwdWgHeads = 64;

__device__ __forceinline__ void bwd_dma16(unsigned lds_base, int voff, __amdgpu_buffer_rsrc_t rsrc) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_base), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void bwd_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// MERGE (the shared latent of MLA absorb, value = key[..., :D]): the dV
// contribution of a token is added to its dK nope columns before the
// atomics, so each (row, 64 heads, token) adds D + 64 values instead of
// 2D + 64; dv is not written.
template <int D, typename T, bool MERGE>
__global__ __launch_bounds__(kBwdWgWaves * 64, 1) void sfa_bwd_wg_kernel(SfaBwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int DR = 64;
  constexpr int DC = D + DR;
  constexpr int KS = DC / 32, KSN = D / 32;
  constexpr int NDT = D / 16;
  constexpr int TILE = kBwdTile;
  constexpr int NT = kBwdWgWaves * 64;
  constexpr int ROW = D * 2;
  constexpr int TPI = 1024 / ROW;            // nope rows per DMA (1 KB per DMA)
  constexpr int NDN = TILE / TPI / kBwdWgWaves;  // nope DMAs per wave per tile
  constexpr int NCOL = 2 * D + DR;           // dK | dK_rope | dV columns
  constexpr int NCW = NCOL / 16 / kBwdWgWaves;   // column tiles per wave
  constexpr int NNW = D / 16 / kBwdWgWaves;      // MERGE: nope column tiles per wave
  constexpr int NXB = MERGE ? 2 * NNW + 1 : NCW; // B-operand column tiles per wave
  constexpr int TR = kBwdWgHeads + 8;        // padded [token][head] row
  static_assert(NCOL % (16 * kBwdWgWaves) == 0 && TILE % (TPI * kBwdWgWaves) == 0, "layout");

  __shared__ __attribute__((aligned(1024))) unsigned char s_k[2][TILE * ROW];
  __shared__ __attribute__((aligned(1024))) unsigned char s_kr[2][TILE * DR * 2];
  __shared__ int s_list[kBwdList + TILE];
  __shared__ __attribute__((aligned(16))) T s_t[2][TILE][TR];  // dS, P of the 64 heads
  __shared__ int s_wcnt[kBwdWgWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int row = blockIdx.x;
  const int hbase = blockIdx.y * kBwdWgHeads;
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
  float delta = 0.f;
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks) {
    const u32x4 v = *(const u32x4*)((const T*)p.dout + hrow * D + ks * 32 + lg * 8);
    const u32x4 o = *(const u32x4*)((const T*)p.out + hrow * D + ks * 32 + lg * 8);
    dof[ks] = as_v8<V8>(hv ? v : z4);
    const V8 dv8 = as_v8<V8>(v), ov8 = as_v8<V8>(o);
#pragma unroll
    for (int j = 0; j < 8; ++j) delta += E::to_f32(dv8[j]) * E::to_f32(ov8[j]);
  }
  delta = xgroup_sum(delta);
  float m2 = 0.f, inv = 0.f;
  if (hv) {
    m2 = p.smax[hrow] * kLog2e;
    const float ss = p.ssum[hrow];
    inv = 1.f / (ss > 0.f ? ss : 1.f);
  } else {
    delta = 0.f;
  }
  // B operands of the 64-head sums: column c of [Q nope | Q rope | dO],
  // heads hbase + 32*ks + 8*lg + j.  Tile i is column 16*(wave*NCW + i) + li;
  // with MERGE, tiles i < NNW are Q nope columns 16*(wave*NNW + i) + li,
  // tiles NNW + i the dO columns of the same index, and tile 2*NNW the Q
  // rope columns 16*wave + li.
  V8 xb[NXB][2];
#pragma unroll
  for (int i = 0; i < NXB; ++i) {
    int c = 16 * (wave * NCW + i) + li;
    if (MERGE) {
      if (i < NNW) c = 16 * (wave * NNW + i) + li;
      else if (i < 2 * NNW) c = D + DR + 16 * (wave * NNW + i - NNW) + li;
      else c = D + 16 * wave + li;
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int h = hbase + ks * 32 + lg * 8 + j;
        T v = E::from_f32(0.f);
        if (h < p.n1) {
          const int64_t r = (int64_t)row * p.n1 + h;
          if (c < D) v = ((const T*)p.q)[r * D + c];
          else if (c < D + DR) v = ((const T*)p.qr)[r * DR + (c - D)];
          else v = ((const T*)p.dout)[r * D + (c - D - DR)];
        }
        xb[i][ks][j] = v;
      }
  }
  f32x4 acc_dq[NDT], acc_dqr[DR / 16];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_dq[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dt = 0; dt < DR / 16; ++dt) acc_dqr[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // ---- tile DMA: wave w loads nope rows (j*4 + w)*TPI .. +TPI (lane L ->
  // row + L/CPT, source chunk (L%CPT) ^ nope_swz) and rope rows 8w .. 8w+7 ----
  constexpr int CPT = 64 / TPI;  // chunks per row covered by one DMA
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.k, (short)0, (int)(p.kv_rows * D * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rr =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.kr, (short)0, (int)(p.kv_rows * DR * 2), 0x00020000);
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto issue_tile = [&](int t, int b) {
    int ph[NDN + 1];
#pragma unroll
    for (int j = 0; j < NDN; ++j) ph[j] = s_list[t * TILE + (j * kBwdWgWaves + wave_s) * TPI + lane / CPT];
    ph[NDN] = s_list[t * TILE + wave_s * 8 + (lane >> 3)];
#pragma unroll
    for (int j = 0; j < NDN; ++j) {
      const int tk = (j * kBwdWgWaves + wave_s) * TPI + lane / CPT;
      const int ch = (lane % CPT) ^ nope_swz(tk);
      const unsigned dst = (unsigned)(uintptr_t)&s_k[b][(j * kBwdWgWaves + wave_s) * TPI * ROW];
      bwd_dma16(dst, ph[j] >= 0 ? ph[j] * ROW + ch * 16 : (int)0x80000000, rk);
    }
    {
      const int tk = wave_s * 8 + (lane >> 3);
      const int ch = (lane & 7) ^ rope_swz(tk);
      const unsigned dst = (unsigned)(uintptr_t)&s_kr[b][wave_s * 8 * DR * 2];
      bwd_dma16(dst, ph[NDN] >= 0 ? ph[NDN] * (DR * 2) + ch * 16 : (int)0x80000000, rr);
    }
  };

  for (int64_t c0 = 0; c0 < total_pos; c0 += kBwdList) {
    // ---- compact this range of positions into s_list (stable order) ----
    const int64_t c1 = min(total_pos, c0 + (int64_t)kBwdList);
    int n_valid = 0;
    for (int64_t b0 = c0; b0 < c1; b0 += NT) {
      const int64_t pos = b0 + tid;
      int phys = 0;
      bool valid = false;
      if (ri.active && pos < c1) valid = sfa_resolve(p, ri, idx_row, (int)pos, &phys);
      const unsigned long long m = __ballot(valid);
      if (lane == 0) s_wcnt[wave] = __popcll(m);
      lds_barrier();
      int off = n_valid, tot = 0;
#pragma unroll
      for (int w = 0; w < kBwdWgWaves; ++w) {
        const int c = s_wcnt[w];
        off += w < wave ? c : 0;
        tot += c;
      }
      if (valid) s_list[off + __popcll(m & ((1ull << lane) - 1ull))] = phys;
      n_valid += tot;
      lds_barrier();
    }
    if (tid < TILE) s_list[n_valid + tid] = -1;
    lds_barrier();
    const int n_tiles = (n_valid + TILE - 1) / TILE;
    if (n_tiles > 0) issue_tile(0, 0);

    for (int t = 0; t < n_tiles; ++t) {
      const int b = t & 1;
      bwd_wait_all();  // this tile's DMA (and everything older) has landed
      lds_barrier();
      if (t + 1 < n_tiles) issue_tile(t + 1, b ^ 1);
      const unsigned char* kt = s_k[b];
      const unsigned char* krt = s_kr[b];

      // ---- S^T = K.Q^T and dP^T = K_nope.dO^T (shared K fragments) ----
      f32x4 acc_s[2], acc_p[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        acc_s[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        acc_p[tt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int tk = tt * 16 + li;
          const unsigned char* a = ks < KSN ? kt + tk * ROW + (((ks * 4 + lg) ^ nope_swz(tk)) * 16)
                                            : krt + tk * (DR * 2) + ((((ks - KSN) * 4 + lg) ^ rope_swz(tk)) * 16);
          const V8 av = as_v8<V8>(*(const u32x4*)a);
          acc_s[tt] = E::mfma(av, qf[ks], acc_s[tt]);
          if (ks < KSN) acc_p[tt] = E::mfma(av, dof[ks], acc_p[tt]);
        }

      // ---- P^T, dS^T (token tt*16 + 4*lg + r, head li) ----
      constexpr bool kSplit = __is_same(T, bf16);
      V8 dsf, dsl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tt = j >> 2, r = j & 3;
        const int tk = tt * 16 + lg * 4 + r;
        const bool tv = t * TILE + tk < n_valid;
        const float pp = tv ? fast_exp2(acc_s[tt][r] * p.scale_log2 - m2) * inv : 0.f;
        const float ds = pp * (acc_p[tt][r] - delta) * p.scale;
        const T dh = E::from_f32(ds);
        dsf[j] = dh;
        dsl[j] = E::from_f32(ds - E::to_f32(dh));
        s_t[0][tk][wave * 16 + li] = dh;
        s_t[1][tk][wave * 16 + li] = E::from_f32(pp);
      }

      // ---- dq^T += K^T.dS^T, dq_rope^T += Kr^T.dS^T (transposing reads) ----
      {
        const int r1 = lg * 4 + (li >> 2);
        const int hb = (li & 3) >> 1;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int ch = 2 * dt + hb;
          const unsigned char* p1 = kt + r1 * ROW + ((ch ^ nope_swz(r1)) * 16) + (li & 1) * 8;
          const unsigned char* p2 = kt + (r1 + 16) * ROW + ((ch ^ nope_swz(r1 + 16)) * 16) + (li & 1) * 8;
          const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
          const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
          const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
          acc_dq[dt] = E::mfma(__builtin_bit_cast(V8, w), dsf, acc_dq[dt]);
          if (kSplit) acc_dq[dt] = E::mfma(__builtin_bit_cast(V8, w), dsl, acc_dq[dt]);
        }
#pragma unroll
        for (int dt = 0; dt < DR / 16; ++dt) {
          const int ch = 2 * dt + hb;
          const unsigned char* p1 = krt + r1 * (DR * 2) + ((ch ^ rope_swz(r1)) * 16) + (li & 1) * 8;
          const unsigned char* p2 = krt + (r1 + 16) * (DR * 2) + ((ch ^ rope_swz(r1 + 16)) * 16) + (li & 1) * 8;
          const i16x4 w1 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1));
          const i16x4 w2 = __builtin_bit_cast(i16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p2));
          const i16x8 w = {w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
          acc_dqr[dt] = E::mfma(__builtin_bit_cast(V8, w), dsf, acc_dqr[dt]);
          if (kSplit) acc_dqr[dt] = E::mfma(__builtin_bit_cast(V8, w), dsl, acc_dqr[dt]);
        }
      }
      lds_barrier();  // dS / P of all 64 heads in LDS

      // ---- dK | dK_rope | dV columns of this wave, summed over 64 heads ----
      int ph[2][4];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) ph[tt][r] = s_list[t * TILE + tt * 16 + lg * 4 + r];
      if (MERGE) {
        // nope columns: dS^T.Q + P^T.dO in one accumulator; rope: dS^T.Q_rope
#pragma unroll
        for (int i = 0; i <= NNW; ++i) {
          const bool rope = i == NNW;
          const int c = rope ? 16 * wave + li : 16 * (wave * NNW + i) + li;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              const V8 ads = as_v8<V8>(*(const u32x4*)&s_t[0][tt * 16 + li][ks * 32 + lg * 8]);
              acc = E::mfma(ads, xb[rope ? 2 * NNW : i][ks], acc);
              if (!rope) {
                const V8 ap = as_v8<V8>(*(const u32x4*)&s_t[1][tt * 16 + li][ks * 32 + lg * 8]);
                acc = E::mfma(ap, xb[NNW + (rope ? 0 : i)][ks], acc);
              }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int pr = ph[tt][r];
              if (pr < 0) continue;
              if (rope) atomicAdd(p.dkr + (int64_t)pr * DR + c, acc[r]);
              else atomicAdd(p.dk + (int64_t)pr * D + c, acc[r]);
            }
          }
        }
        continue;
      }
#pragma unroll
      for (int i = 0; i < NCW; ++i) {
        const int ct = wave * NCW + i;
        const int sel = ct < (D + DR) / 16 ? 0 : 1;  // dS for dK / dK_rope, P for dV
        const int c = 16 * ct + li;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const V8 a = as_v8<V8>(*(const u32x4*)&s_t[sel][tt * 16 + li][ks * 32 + lg * 8]);
            acc = E::mfma(a, xb[i][ks], acc);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int pr = ph[tt][r];
            if (pr < 0) continue;
            if (c < D) atomicAdd(p.dk + (int64_t)pr * D + c, acc[r]);
            else if (c < D + DR) atomicAdd(p.dkr + (int64_t)pr * DR + (c - D), acc[r]);
            else atomicAdd(p.dv + (int64_t)pr * D + (c - D - DR), acc[r]);
          }
        }
      }
    }
    bwd_wait_all();
    lds_barrier();  // s_list is rebuilt for the next range
  }

  // ---- dq, dq_rope (head li, columns 16*dt + 4*lg + r) ----
  if (hv) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T* dqp = (T*)p.dq + hrow * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const T4 o = {E::from_f32(acc_dq[dt][0]), E::from_f32(acc_dq[dt][1]), E::from_f32(acc_dq[dt][2]),
                    E::from_f32(acc_dq[dt][3])};
      *(T4*)(dqp + dt * 16 + lg * 4) = o;
    }
    T* dqrp = (T*)p.dqr + hrow * DR;
#pragma unroll
    for (int dt = 0; dt < DR / 16; ++dt) {
      const T4 o = {E::from_f32(acc_dqr[dt][0]), E::from_f32(acc_dqr[dt][1]), E::from_f32(acc_dqr[dt][2]),
                    E::from_f32(acc_dqr[dt][3])};
      *(T4*)(dqrp + dt * 16 + lg * 4) = o;
    }
  }
}

__global__ __launch_bounds__(256) void bwd_fill_kernel(uint32_t* a, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] = v;
}

// fp32 workspace -> output dtype
template <typename T>
__global__ __launch_bounds__(256) void cast_f32_kernel(const float* src, T* dst, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 3 < n) {
    const float4 v = *(const float4*)(src + i);
    typedef T T4 __attribute__((ext_vector_type(4)));
    const T4 o = {Elem<T>::from_f32(v.x), Elem<T>::from_f32(v.y), Elem<T>::from_f32(v.z), Elem<T>::from_f32(v.w)};
    *(T4*)(dst + i) = o;
  } else {
    for (int64_t j = i; j < n; ++j) dst[j] = Elem<T>::from_f32(src[j]);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
size_t sfa_bwd_workspace_bytes(int64_t kv_rows, int64_t d) {
  return (size_t)kv_rows * (size_t)(d + 64 + d) * sizeof(float);
}

// The workgroup kernel gathers with buffer loads (32-bit offsets): key
// tensors of 2 GiB and more take the one-wave kernel.
// The workgroup kernel (merged when `merge`) or, for key tensors of 2 GiB
// and more, the one-wave kernel (never merged).  Returns whether the dK
// workspace already holds dk + dv.
template <int D, typename T>
static hipError_t launch_sfa_bwd(const SfaBwdParams& p, bool merge, bool* merged, hipStream_t stream) {
  *merged = false;
  if ((int64_t)p.kv_rows * D * 2 < (1ll << 31)) {
    const dim3 grid((unsigned)p.rows, (unsigned)((p.n1 + kBwdWgHeads - 1) / kBwdWgHeads));
    if (merge) {
      hipLaunchKernelGGL((sfa_bwd_wg_kernel<D, T, true>), grid, dim3(kBwdWgWaves * 64), 0, stream, p);
      *merged = true;
    } else {
      hipLaunchKernelGGL((sfa_bwd_wg_kernel<D, T, false>), grid, dim3(kBwdWgWaves * 64), 0, stream, p);
    }
  } else {
    hipLaunchKernelGGL((sfa_bwd_kernel<D, T>), dim3((unsigned)p.rows, (unsigned)((p.n1 + 15) / 16)), dim3(64), 0,
                       stream, p);
  }
  return hipGetLastError();
}

// d_key = dk + dv (fp32 workspaces summed before the cast)
template <typename T>
__global__ __launch_bounds__(256) void cast_sum_f32_kernel(const float* a, const float* b, T* dst, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 3 < n) {
    const float4 x = *(const float4*)(a + i), y = *(const float4*)(b + i);
    typedef T T4 __attribute__((ext_vector_type(4)));
    const T4 o = {Elem<T>::from_f32(x.x + y.x), Elem<T>::from_f32(x.y + y.y), Elem<T>::from_f32(x.z + y.z),
                  Elem<T>::from_f32(x.w + y.w)};
    *(T4*)(dst + i) = o;
  } else {
    for (int64_t j = i; j < n; ++j) dst[j] = Elem<T>::from_f32(a[j] + b[j]);
  }
}

template <typename T>
static hipError_t launch_cast_sum(const float* a, const float* b, void* dst, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 1023) / 1024;
  hipLaunchKernelGGL((cast_sum_f32_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, stream, a, b, (T*)dst, n);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_cast(const float* src, void* dst, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 1023) / 1024;
  hipLaunchKernelGGL((cast_f32_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, stream, src, (T*)dst, n);
  return hipGetLastError();
}

int sfa_bwd_run(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, const void* d_out, const void* out, const float* softmax_max,
                const float* softmax_sum, const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                void* d_query, void* d_query_rope, void* d_key, void* d_key_rope, void* d_value,
                int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t sparse_count,
                int64_t q_rows, int64_t kv_rows, int32_t sparse_block_size, int32_t sparse_mode,
                int32_t layout, int32_t dtype, float scale_value, void* workspace, hipStream_t stream) {
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
  float* ws = (float*)workspace;
  p.dk = ws;
  p.dkr = ws + kv_rows * d;
  p.dv = ws + kv_rows * (d + 64);
  p.rows = q_rows;
  p.kv_rows = kv_rows;
  p.batch = (int32_t)batch;
  p.s1 = (int32_t)s1;
  p.s2 = (int32_t)s2;
  p.n1 = (int32_t)n1;
  p.K = (int32_t)sparse_count;
  p.bs = sparse_block_size;
  p.mode = sparse_mode;
  p.layout_q = layout;
  p.layout_kv = layout;
  p.max_blocks = 0;
  p.page_size = 1;
  p.scale = scale_value;
  p.scale_log2 = scale_value * kLog2e;
  // the fp32 accumulators start at zero (a fill kernel: no memset node when
  // the caller captures the call in a graph)
  const int64_t nacc = (int64_t)(sfa_bwd_workspace_bytes(kv_rows, d) / 4);
  hipLaunchKernelGGL(bwd_fill_kernel, dim3((unsigned)((nacc + 255) / 256)), dim3(256), 0, stream, (uint32_t*)workspace,
                     nacc, 0u);
  DSA_HIP(hipGetLastError());
  bool merged = false;
  if (q_rows > 0) {
    hipError_t e;
    const bool bf = dtype == DSA_DTYPE_BF16;
    const bool merge = d_value == nullptr;
    if (d == 128) e = bf ? launch_sfa_bwd<128, bf16>(p, merge, &merged, stream)
                         : launch_sfa_bwd<128, f16>(p, merge, &merged, stream);
    else if (d == 256) e = bf ? launch_sfa_bwd<256, bf16>(p, merge, &merged, stream)
                              : launch_sfa_bwd<256, f16>(p, merge, &merged, stream);
    else e = bf ? launch_sfa_bwd<512, bf16>(p, merge, &merged, stream)
                : launch_sfa_bwd<512, f16>(p, merge, &merged, stream);
    DSA_HIP(e);
  }
  const bool bf = dtype == DSA_DTYPE_BF16;
  auto cast = [&](const float* src, void* dst, int64_t n) {
    return bf ? launch_cast<bf16>(src, dst, n, stream) : launch_cast<f16>(src, dst, n, stream);
  };
  if (d_value) {
    DSA_HIP(cast(p.dk, d_key, kv_rows * d));
    DSA_HIP(cast(p.dv, d_value, kv_rows * d));
  } else if (merged) {
    DSA_HIP(cast(p.dk, d_key, kv_rows * d));  // dk already holds dk + dv
  } else {
    // shared latent: d_key = dk + dv
    DSA_HIP(bf ? launch_cast_sum<bf16>(p.dk, p.dv, d_key, kv_rows * d, stream)
               : launch_cast_sum<f16>(p.dk, p.dv, d_key, kv_rows * d, stream));
  }
  DSA_HIP(cast(p.dkr, d_key_rope, kv_rows * 64));
  return DSA_OK;
}

}  // namespace dsa
