// Backward of the small-head attention (8 heads x 16 dims, merged width E = 128) for gfx950.
//
// Gradients of O = softmax(q' k'^T + bias) V per head, q' = cast(rope(q) scale), k' = cast(rope(k)),
// as the reference's training kernels compute them (scripts/tabicl_tpu_pallas_attn.py:87-122 for
// hx, :512-560 for the packed kernels):
//   P  = softmax, recomputed in fp32           dP = dO V^T (fp32)
//   D  = sum over the head's 16 dims of dO * O (the stored forward output)
//   dS = P * (dP - D), cast to the input dtype
//   dq' = dS k',  dk' = dS^T q',  dv = cast(P)^T dO   (fp32 accumulation)
//   dq = rope_bwd(dq' scale), dk = rope_bwd(dk'),  rope_bwd(y) = y cos - R(y sin)
// The reference keeps all keys of a batch element on chip (at most 1024). Here:
//   ss_bwd_kernel  bf16 with both lengths <= 128 (row, CLS): one fused kernel per (batch element,
//                  4 heads) with every row resident in LDS (described above its definition).
// Otherwise keys and queries are tiled, so any length works:
//   sb_dq_kernel   workgroup = (batch element, run of 128-query blocks, head); wave = 16 queries.
//                  Per block: per-query softmax statistics (row maximum and log2 of the sum, in log2
//                  units) and D, written to the workspace, then P, dP, dS and dq'. Keys in one tile
//                  (<= 128): one fill per run and one pass per block with the scores in registers;
//                  longer: two sweeps over the key tiles.
//   sb_dkdv_kernel workgroup = (batch element, 128 keys, head); wave = 16 keys. Walks the query
//                  tiles with the workspace's statistics and D: P, dP, dS, dk' and dv.
// No atomics, no cross-workgroup reduction: each gradient element is written once.
// MFMA 16x16x16 (bf16) or 4 x 16x16x4 (fp32), lane layout of mfma16x16x16 in common.h.
#include "common.h"
#include "launch.h"

namespace {

constexpr int SB_E = 128;
constexpr int SB_H = 8;
constexpr int SB_D = 16;
constexpr int SB_NW = 8;             // waves per workgroup
constexpr int SB_QB = 16 * SB_NW;    // queries per dq workgroup
constexpr int SB_KB = 16 * SB_NW;    // keys per dk/dv workgroup
constexpr int SB_KT = 128;           // key tile of the dq kernel
constexpr int SB_QT = 128;           // query tile of the dk/dv kernel
constexpr float SB_BIAS_FLOOR = -1e37f;

struct SbParams {
  const void* q;
  int64_t q_sb, q_sr;
  const void* k;
  int64_t k_sb, k_sr;
  const void* v;
  int64_t v_sb, v_sr;
  const void* o;     // [B, Lq, E]
  const void* dout;  // [B, Lq, E]
  void* dq;
  int64_t dq_sb, dq_sr;
  void* dk;
  int64_t dk_sb, dk_sr;
  void* dv;
  int64_t dv_sb, dv_sr;
  const float* bias;
  int64_t bias_sb;
  const float* cq;
  const float* sq;
  const float* ck;
  const float* sk;
  int rope, half, rot;
  // RoPE tables: log2 of the row stride (elements) and the column mask; [L, E] tables: 7 (E = 128) and
  // E - 1; one head's [L, 16] columns shared by every head (TABICL_ROPE_SHARED_TABLES): 4 and 15
  int tab_ss, tab_cm;
  float scale;
  int B, Lq, Lk;
  int qbpw;  // query blocks per dq workgroup
  // per (batch, head, query), [B][H][Lq] each: the row maximum m of the log2-domain scores and
  // log2 of the sum of exp2(x - m) (kept apart: with every key at the bias floor, m + log2(l)
  // would round back to m), and D
  float* mx;
  float* ll;
  float* dd;
};

// 16x16 tile with a 32-deep contraction over two 16-deep halves: A = [a0 | a1], B = [b0 | b1], i.e. the
// sum of the two 16x16x16 products a0 b0 + a1 b1 in one v_mfma_f32_16x16x32_bf16 (k-slot 8 kap + j of
// lane (l16, kap) holds slot 4 kap + j of the first half for j < 4 and of the second half for j >= 4,
// in A and B alike). On gfx950 it issues in the cycles of one 16x16x16 product.
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x4 a0, bf16x4 a1, bf16x4 b0, bf16x4 b1, f32x4 c) {
  const bf16x8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
  const bf16x8 b = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <typename T> struct SbTile {
  static constexpr int PAD = 16 / sizeof(T);
  static constexpr int RSTR = SB_D + PAD;   // row-major tile: 16 dims per row
  static constexpr int TSTR = 128 + PAD;    // transposed copy (fp32 only): 128 rows per dim
  static constexpr int T_ELEMS = sizeof(T) == 2 ? 4 : SB_D * TSTR;
};

// Per-key additive term in log2 units (reference: bias added to the fp32 scores; -1e30 stays
// finite, so a row with every key masked is uniform).
__device__ __forceinline__ float sb_b2(const SbParams& p, int b, int key) {
  if (key >= p.Lk) return TA_NEG_INF;
  return p.bias ? fmaxf(p.bias[b * p.bias_sb + key] * TA_LOG2E, SB_BIAS_FLOOR) : 0.f;
}

// Head g's first column in row `row` of a RoPE table (either table form).
__device__ __forceinline__ const float* sb_tab_row(const float* t, int64_t row, int g, const SbParams& p) {
  return t + (row << p.tab_ss) + ((g * SB_D) & p.tab_cm);
}

// Dims d0..d0+3 of q' (rope, scale, cast) or of k' (rope, cast; scale = 1) of one row; cs / sn: the
// row's table row at the first column of d0's head (sb_tab_row). RP: the call has a RoPE form
// (p.rope != 0); the sb kernels are compiled with and without it.
template <typename T, bool RP>
__device__ __forceinline__ typename OpVec<T, 4>::type sb_prep4(const T* row, const float* cs, const float* sn,
                                                              int d0, const SbParams& p, float scale) {
  typedef typename OpVec<T, 4>::type Op4;
  Op4 r;
  if constexpr (RP) {
    const f32x4 y = rope4<T>(row, cs, sn, d0, p.rope, p.half, p.rot, d0 & (SB_D - 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = from_f32<T>(y[j] * scale);
  } else {
    const Op4 raw = *(const Op4*)(row + d0);
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = scale == 1.f ? raw[j] : from_f32<T>(to_f32<T>(raw[j]) * scale);
  }
  return r;
}

// rope_bwd of one 16-dim head row held as 4 dims per lane (lane (l16, kap): dims 4 kap .. 4 kap + 3
// of row l16), exchanged through this wave's LDS scratch [16][17]; cs / sn at the row's position,
// head g's first column of the table row (sb_tab_row), or null rows for no RoPE.
template <bool RP>
__device__ __forceinline__ f32x4 sb_rope_bwd(f32x4 y, float* scr, int l16, int kap, const float* cs,
                                            const float* sn, const SbParams& p) {
  if constexpr (!RP) return y;
#pragma unroll
  for (int r = 0; r < 4; ++r) scr[l16 * 17 + 4 * kap + r] = y[r];
  __builtin_amdgcn_wave_barrier();
  f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int jd = 4 * kap + r;
    int pt;
    float sg;
    rope_partner(jd, p.rope, p.half, p.rot, &pt, &sg);
    const float yp = scr[l16 * 17 + pt];
    out[r] = y[r] * cs[jd] - sg * yp * sn[pt];
  }
  __builtin_amdgcn_wave_barrier();
  return out;
}

// Transposed operand of a 16x16x16 product, A[i][4 kap + j] = tile[row0 + 4 kap + j][i] for lane
// (i = l16, kap). bf16: straight from the row-major tile with ds_read_b64_tr_b16 (lane 4j + c of a
// 16-lane group points at row 4 kap + j, columns 4c..4c+3, and receives column l16 of those four
// rows); fp32: from the transposed copy the fill wrote.
template <typename T>
__device__ __forceinline__ typename OpVec<T, 4>::type sb_opT(const T* rows, const T* tcopy, int row0, int l16,
                                                            int kap) {
  typedef SbTile<T> L;
  if constexpr (sizeof(T) == 2) {
    const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(rows + (row0 + 4 * kap + (l16 >> 2)) * L::RSTR + 4 * (l16 & 3)));
    return __builtin_bit_cast(bf16x4, t);
  } else {
    return *(const f32x4*)(tcopy + l16 * L::TSTR + row0 + 4 * kap);
  }
}

// ---------------------------------------------------------------------------------------------
// dq (and the per-query softmax statistics and D)
// ---------------------------------------------------------------------------------------------
template <typename T, bool RP>
__device__ __forceinline__ void sb_fill_keys(const SbParams& p, T* lk, T* lkt, T* lv, float* lb2, int b, int g,
                                             int k0) {
  typedef SbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  const int tid = threadIdx.x;
  const T* kbase = (const T*)p.k + b * p.k_sb;
  const T* vbase = (const T*)p.v + b * p.v_sb;
  // unit = (key, 4 dims): 128 keys x 4 = 512 units, one per thread
  for (int u = tid; u < SB_KT * 4; u += SB_NW * 64) {
    const int row = u >> 2, d4 = (u & 3) * 4, key = k0 + row;
    Op4 kk, vv;
#pragma unroll
    for (int j = 0; j < 4; ++j) { kk[j] = from_f32<T>(0.f); vv[j] = from_f32<T>(0.f); }
    if (key < p.Lk) {
      kk = sb_prep4<T, RP>(kbase + (int64_t)key * p.k_sr, sb_tab_row(p.ck, key, g, p), sb_tab_row(p.sk, key, g, p),
                       g * SB_D + d4, p, 1.f);
      vv = *(const Op4*)(vbase + (int64_t)key * p.v_sr + g * SB_D + d4);
    }
    *(Op4*)(lk + row * L::RSTR + d4) = kk;
    *(Op4*)(lv + row * L::RSTR + d4) = vv;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) lkt[(d4 + j) * L::TSTR + row] = kk[j];
    }
  }
  for (int j = tid; j < SB_KT; j += SB_NW * 64) lb2[j] = sb_b2(p, b, k0 + j);
}

// Scores of the key tile for this lane's query, log2 units: x[kt][r] for key 16 kt + 4 kap + r.
template <typename T>
__device__ __forceinline__ void sb_scores(const T* lk, const float* lb2, typename OpVec<T, 4>::type qop, int l16,
                                          int kap, f32x4 (&x)[SB_KT / 16]) {
  typedef SbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
#pragma unroll
  for (int kt = 0; kt < SB_KT / 16; ++kt) {
    const Op4 a = *(const Op4*)(lk + (16 * kt + l16) * L::RSTR + 4 * kap);
    x[kt] = mfma16x16x16(a, qop, f32x4{0.f, 0.f, 0.f, 0.f});
    const f32x4 b2 = *(const f32x4*)(lb2 + 16 * kt + 4 * kap);
#pragma unroll
    for (int r = 0; r < 4; ++r) x[kt][r] = fmaf(x[kt][r], TA_LOG2E, b2[r]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// dq' l += e (dP - D) k' over the key tile, from e = exp2(x - m) = P l (the caller scales the sum by
// 1 / l): dP - D straight from the product with -D (nds) as its accumulator input, and e (dP - D)
// rounded to the input dtype as dS is. bf16: two key blocks per 32-deep product.
template <typename T>
__device__ __forceinline__ void sb_dq_tile(const T* lk, const T* lkt, const T* lv, const f32x4 (&e)[SB_KT / 16],
                                           typename OpVec<T, 4>::type dop, float nds, int l16, int kap, f32x4& acc) {
  typedef SbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  const f32x4 cnd = {nds, nds, nds, nds};
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int kt = 0; kt < SB_KT / 16; kt += 2) {
      const f32x4 dp0 = mfma16x16x16(*(const Op4*)(lv + (16 * kt + l16) * L::RSTR + 4 * kap), dop, cnd);
      const f32x4 dp1 = mfma16x16x16(*(const Op4*)(lv + (16 * kt + 16 + l16) * L::RSTR + 4 * kap), dop, cnd);
      f32x4 d0, d1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        d0[r] = e[kt][r] * dp0[r];
        d1[r] = e[kt + 1][r] * dp1[r];
      }
      acc = mfma16x16x32(sb_opT<T>(lk, lkt, 16 * kt, l16, kap), sb_opT<T>(lk, lkt, 16 * kt + 16, l16, kap),
                         cvt_bf16x4(d0), cvt_bf16x4(d1), acc);
      // two key blocks at a time: hoisting every block's dP first costs registers
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int kt = 0; kt < SB_KT / 16; ++kt) {
      const f32x4 dp = mfma16x16x16(*(const Op4*)(lv + (16 * kt + l16) * L::RSTR + 4 * kap), dop, cnd);
      Op4 ds;
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[r] = e[kt][r] * dp[r];
      acc = mfma16x16x16(sb_opT<T>(lk, lkt, 16 * kt, l16, kap), ds, acc);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// ONE_TILE: all keys fit one tile (Lk <= SB_KT).
template <typename T, bool ONE_TILE, bool RP>
__global__ __launch_bounds__(SB_NW * 64, 4) void sb_dq_kernel(SbParams p) {
  typedef SbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  constexpr int NKT = SB_KT / 16;
  __shared__ __attribute__((aligned(16))) T lk[SB_KT * L::RSTR];
  __shared__ __attribute__((aligned(16))) T lkt[L::T_ELEMS];
  __shared__ __attribute__((aligned(16))) T lv[SB_KT * L::RSTR];
  __shared__ __attribute__((aligned(16))) float lb2[SB_KT];
  __shared__ float scr[SB_NW][16 * 17];

  const int nqb = (p.Lq + SB_QB - 1) / SB_QB;
  const int nwg_q = (nqb + p.qbpw - 1) / p.qbpw;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int g = work % SB_H, qw = (work / SB_H) % nwg_q, b = work / (SB_H * nwg_q);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int d0 = g * SB_D + 4 * kap;
  const int ntiles = (p.Lk + SB_KT - 1) / SB_KT;
  if (ONE_TILE) {  // fill once for every query block of the run
    sb_fill_keys<T, RP>(p, lk, lkt, lv, lb2, b, g, 0);
    __syncthreads();
  }

  for (int qbi = 0; qbi < p.qbpw; ++qbi) {
    const int qb = qw * p.qbpw + qbi;
    if (qb >= nqb) break;  // uniform over the workgroup
    const int qi = qb * SB_QB + wave * 16 + l16;
    const bool qok = qi < p.Lq;

    // q' and dO operands of query qi (B operands of S^T = K' Q'^T and dP^T = V dO^T), D
    Op4 qop, dop;
#pragma unroll
    for (int j = 0; j < 4; ++j) { qop[j] = from_f32<T>(0.f); dop[j] = from_f32<T>(0.f); }
    float dsum = 0.f;
    if (qok) {
      qop = sb_prep4<T, RP>((const T*)p.q + b * p.q_sb + (int64_t)qi * p.q_sr, sb_tab_row(p.cq, qi, g, p),
                            sb_tab_row(p.sq, qi, g, p), d0, p, p.scale);
      const int64_t orow = ((int64_t)b * p.Lq + qi) * SB_E + d0;
      dop = *(const Op4*)((const T*)p.dout + orow);
      const Op4 ov = *(const Op4*)((const T*)p.o + orow);
#pragma unroll
      for (int j = 0; j < 4; ++j) dsum += to_f32<T>(dop[j]) * to_f32<T>(ov[j]);
    }
    dsum = xor_sum(dsum, 16);
    dsum = xor_sum(dsum, 32);

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float mq, lgl, inv;
    if (ONE_TILE) {
      // one pass: the scores stay in registers between the statistics and dq'
      f32x4 x[NKT];
      sb_scores<T>(lk, lb2, qop, l16, kap, x);
      float tm = TA_NEG_INF;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) tm = fmaxf(tm, x[kt][r]);
      mq = quad_max(tm);  // finite: the tile holds at least one key
      float l = 0.f;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[kt][r] = __builtin_amdgcn_exp2f(x[kt][r] - mq);  // e, kept for dq'
          l += x[kt][r];
        }
      l = quad_sum(l);  // >= 1
      lgl = __builtin_amdgcn_logf(l);
      inv = __builtin_amdgcn_rcpf(l);
      sb_dq_tile<T>(lk, lkt, lv, x, dop, -dsum, l16, kap, acc);
    } else {
      // sweep 1: statistics over this lane's keys (4 per 16-key block), merged over the lane quad
      float m = TA_NEG_INF, l = 0.f;
      for (int t = 0; t < ntiles; ++t) {
        __syncthreads();
        sb_fill_keys<T, RP>(p, lk, lkt, lv, lb2, b, g, t * SB_KT);
        __syncthreads();
        f32x4 x[NKT];
        sb_scores<T>(lk, lb2, qop, l16, kap, x);
        float tm = TA_NEG_INF;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) tm = fmaxf(tm, x[kt][r]);
        if (tm > TA_NEG_INF) {
          const float mn = fmaxf(m, tm);
          float s = 0.f;
#pragma unroll
          for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) s += __builtin_amdgcn_exp2f(x[kt][r] - mn);
          l = l * __builtin_amdgcn_exp2f(m - mn) + s;
          m = mn;
        }
      }
      mq = quad_max(m);
      const float lt = quad_sum(m > TA_NEG_INF ? l * __builtin_amdgcn_exp2f(m - mq) : 0.f);  // >= 1
      lgl = __builtin_amdgcn_logf(lt);
      inv = __builtin_amdgcn_rcpf(lt);
      // sweep 2: dq'
      for (int t = 0; t < ntiles; ++t) {
        __syncthreads();
        sb_fill_keys<T, RP>(p, lk, lkt, lv, lb2, b, g, t * SB_KT);
        __syncthreads();
        f32x4 x[NKT];
        sb_scores<T>(lk, lb2, qop, l16, kap, x);
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) x[kt][r] = __builtin_amdgcn_exp2f(x[kt][r] - mq);
        sb_dq_tile<T>(lk, lkt, lv, x, dop, -dsum, l16, kap, acc);
      }
    }
    if (qok && kap == 0) {
      const int64_t s = ((int64_t)b * SB_H + g) * p.Lq + qi;
      p.mx[s] = mq;
      p.ll[s] = lgl;
      p.dd[s] = dsum;
    }

    // dq = rope_bwd(dq' scale), lane: dims 4 kap .. 4 kap + 3 of head g, query qi (acc holds dq' l)
    f32x4 y;
    const float ysc = p.scale * inv;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = acc[r] * ysc;
    const int qc = qok ? qi : 0;
    y = sb_rope_bwd<RP>(y, scr[wave], l16, kap, sb_tab_row(p.cq, qc, g, p), sb_tab_row(p.sq, qc, g, p), p);
    if (qok) {
      Op4 out;
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = from_f32<T>(y[r]);
      *(Op4*)((T*)p.dq + b * p.dq_sb + (int64_t)qi * p.dq_sr + d0) = out;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dk, dv
// ---------------------------------------------------------------------------------------------
// The query tile of the dk / dv kernel: q' and dO rows (and their transposed copies for fp32), and per
// query the statistics in the form the kernel's P takes (HB: m and log2 l apart, a key bias may sit at
// the floor; else c = -(m + log2 l) ln 2, the accumulator input of the score product, so that
// P = exp2((s + c) log2 e)) and -D (the accumulator input of the dP product). Queries past Lq: m = +inf
// or c = -inf, so P = 0.
template <typename T, bool RP, bool HB>
__device__ __forceinline__ void sb_fill_queries(const SbParams& p, T* lq, T* lqt, T* ld, T* ldt, float* lmx,
                                                float* lll, float* ldd, int b, int g, int q0) {
  typedef SbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  const int tid = threadIdx.x;
  for (int u = tid; u < SB_QT * 4; u += SB_NW * 64) {
    const int row = u >> 2, d4 = (u & 3) * 4, qi = q0 + row;
    Op4 qq, dd;
#pragma unroll
    for (int j = 0; j < 4; ++j) { qq[j] = from_f32<T>(0.f); dd[j] = from_f32<T>(0.f); }
    if (qi < p.Lq) {
      qq = sb_prep4<T, RP>((const T*)p.q + b * p.q_sb + (int64_t)qi * p.q_sr, sb_tab_row(p.cq, qi, g, p),
                           sb_tab_row(p.sq, qi, g, p), g * SB_D + d4, p, p.scale);
      dd = *(const Op4*)((const T*)p.dout + ((int64_t)b * p.Lq + qi) * SB_E + g * SB_D + d4);
    }
    *(Op4*)(lq + row * L::RSTR + d4) = qq;
    *(Op4*)(ld + row * L::RSTR + d4) = dd;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lqt[(d4 + j) * L::TSTR + row] = qq[j];
        ldt[(d4 + j) * L::TSTR + row] = dd[j];
      }
    }
  }
  for (int j = tid; j < SB_QT; j += SB_NW * 64) {
    const int qi = q0 + j;
    const int64_t s = ((int64_t)b * SB_H + g) * p.Lq + qi;
    if (HB) {
      lmx[j] = qi < p.Lq ? p.mx[s] : __builtin_inff();
      lll[j] = qi < p.Lq ? p.ll[s] : 0.f;
    } else {
      lmx[j] = qi < p.Lq ? -(p.mx[s] + p.ll[s]) * TA_LN2 : TA_NEG_INF;
    }
    ldd[j] = qi < p.Lq ? -p.dd[s] : 0.f;
  }
}

// HB: the call has a key bias (else b2 only marks keys past Lk, whose dk / dv are not stored, so the
// kernel ignores it and takes P from the score product with c as its accumulator input).
template <typename T, bool RP, bool HB>
__global__ __launch_bounds__(SB_NW * 64) void sb_dkdv_kernel(SbParams p) {
  typedef SbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  __shared__ __attribute__((aligned(16))) T lq[SB_QT * L::RSTR];
  __shared__ __attribute__((aligned(16))) T lqt[L::T_ELEMS];
  __shared__ __attribute__((aligned(16))) T ld[SB_QT * L::RSTR];
  __shared__ __attribute__((aligned(16))) T ldt[L::T_ELEMS];
  __shared__ __attribute__((aligned(16))) float lmx[SB_QT];
  __shared__ __attribute__((aligned(16))) float lll[SB_QT];
  __shared__ __attribute__((aligned(16))) float ldd[SB_QT];
  __shared__ float scr[SB_NW][16 * 17];

  const int nkb = (p.Lk + SB_KB - 1) / SB_KB;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int g = work % SB_H, kb = (work / SB_H) % nkb, b = work / (SB_H * nkb);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int kj = kb * SB_KB + wave * 16 + l16;
  const bool kok = kj < p.Lk;
  const int d0 = g * SB_D + 4 * kap;

  // k' and V operands of key kj (B operands of S = Q' K'^T and dP = dO V^T) and its b2
  Op4 kop, vop;
#pragma unroll
  for (int j = 0; j < 4; ++j) { kop[j] = from_f32<T>(0.f); vop[j] = from_f32<T>(0.f); }
  if (kok) {
    kop = sb_prep4<T, RP>((const T*)p.k + b * p.k_sb + (int64_t)kj * p.k_sr, sb_tab_row(p.ck, kj, g, p),
                          sb_tab_row(p.sk, kj, g, p), d0, p, 1.f);
    vop = *(const Op4*)((const T*)p.v + b * p.v_sb + (int64_t)kj * p.v_sr + d0);
  }
  const float b2 = HB ? sb_b2(p, b, kj) : 0.f;

  f32x4 dk = {0.f, 0.f, 0.f, 0.f}, dv = {0.f, 0.f, 0.f, 0.f};
  const int ntiles = (p.Lq + SB_QT - 1) / SB_QT;
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    sb_fill_queries<T, RP, HB>(p, lq, lqt, ld, ldt, lmx, lll, ldd, b, g, t * SB_QT);
    __syncthreads();
    // P and dS of query block qs against this wave's keys: S[query 16 qs + 4 kap + r][key kj], dP - D
    // likewise
    auto pds = [&](int qs, Op4& pt, Op4& ds) {
      const Op4 aq = *(const Op4*)(lq + (16 * qs + l16) * L::RSTR + 4 * kap);
      const Op4 ad = *(const Op4*)(ld + (16 * qs + l16) * L::RSTR + 4 * kap);
      const f32x4 ms = *(const f32x4*)(lmx + 16 * qs + 4 * kap);
      const f32x4 dp = mfma16x16x16(ad, vop, *(const f32x4*)(ldd + 16 * qs + 4 * kap));
      f32x4 pr;
      if constexpr (HB) {
        const f32x4 s = mfma16x16x16(aq, kop, f32x4{0.f, 0.f, 0.f, 0.f});
        const f32x4 ls = *(const f32x4*)(lll + 16 * qs + 4 * kap);
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f((fmaf(s[r], TA_LOG2E, b2) - ms[r]) - ls[r]);
      } else {
        const f32x4 s = mfma16x16x16(aq, kop, ms);  // s - (m + log2 l) ln 2
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f(s[r] * TA_LOG2E);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pt[r] = from_f32<T>(pr[r]);
        ds[r] = from_f32<T>(pr[r] * dp[r]);
      }
    };
    if constexpr (sizeof(T) == 2) {
      // query blocks in pairs: one 32-deep product each for dv and dk
#pragma unroll
      for (int qs = 0; qs < SB_QT / 16; qs += 2) {
        Op4 pa, da, pb, db;
        pds(qs, pa, da);
        pds(qs + 1, pb, db);
        dv = mfma16x16x32(sb_opT<T>(ld, ldt, 16 * qs, l16, kap), sb_opT<T>(ld, ldt, 16 * qs + 16, l16, kap), pa, pb, dv);
        dk = mfma16x16x32(sb_opT<T>(lq, lqt, 16 * qs, l16, kap), sb_opT<T>(lq, lqt, 16 * qs + 16, l16, kap), da, db, dk);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll 2
      for (int qs = 0; qs < SB_QT / 16; ++qs) {
        Op4 pt, ds;
        pds(qs, pt, ds);
        dv = mfma16x16x16(sb_opT<T>(ld, ldt, 16 * qs, l16, kap), pt, dv);
        dk = mfma16x16x16(sb_opT<T>(lq, lqt, 16 * qs, l16, kap), ds, dk);
      }
    }
  }

  const int kc = kok ? kj : 0;
  const f32x4 y = sb_rope_bwd<RP>(dk, scr[wave], l16, kap, sb_tab_row(p.ck, kc, g, p), sb_tab_row(p.sk, kc, g, p), p);
  if (kok) {
    Op4 ok, ov;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ok[r] = from_f32<T>(y[r]);
      ov[r] = from_f32<T>(dv[r]);
    }
    *(Op4*)((T*)p.dk + b * p.dk_sb + (int64_t)kj * p.dk_sr + d0) = ok;
    *(Op4*)((T*)p.dv + b * p.dv_sb + (int64_t)kj * p.dv_sr + d0) = ov;
  }
}

// ---------------------------------------------------------------------------------------------
// Short sequences (1 <= Lq, Lk <= 128, bf16): one fused kernel, workgroup = (batch element, group of
// 4 heads), wave = (head of the group, parity of the 16-row blocks it takes). The group's 64 merged
// dims of every query and key row are loaded once, with full-row coalesced reads, into LDS (q', k',
// V, dO; D per query and head from dO and O on the way). Phase 1: per query block the scores of all
// keys stay in registers (statistics, P, dP, dS, dq'); the statistics go to LDS. Phase 2: per key
// block, dk' and dv over all query blocks from those statistics. Two workgroups fit one CU.
// RM: RoPE form, 0 none, 1 pairs over all 16 dims, 2 halves over all 16 dims (rot = 16).
// ---------------------------------------------------------------------------------------------
constexpr int SS_HG = 4;               // heads per workgroup
constexpr int SS_W = SS_HG * SB_D;     // merged dims per workgroup
constexpr int SS_STR = SS_W + 4;       // LDS row stride, elements
constexpr int SS_ROWS = 128;
constexpr int SS_NT = 8 * 64;          // threads

struct SsLds {
  bf16 q[SS_ROWS * SS_STR];  // q' = cast(rope(q) scale)
  bf16 k[SS_ROWS * SS_STR];  // k' = cast(rope(k))
  bf16 v[SS_ROWS * SS_STR];
  bf16 d[SS_ROWS * SS_STR];  // dO
  float mx[SS_HG][SS_ROWS];  // per head and query: row maximum (log2 units), +inf past Lq
  float lg[SS_HG][SS_ROWS];  // log2 of the row sum (with a key bias; else mx holds -(m + lg), -inf past Lq)
  float nd[SS_HG][SS_ROWS];  // -D: the accumulator input of the dP products, which then give dP - D
  float b2[SS_ROWS];         // per key: additive term, log2 units, -inf past Lk
};


// RoPE of a 4-dim chunk (chunk index c4 = (dim within the head) / 4) in the fill: pairs in-lane,
// halves from the partner chunk c4 ^ 2, held by lane ^ 2.
template <int RM>
__device__ __forceinline__ f32x4 ss_rope_fwd(bf16x4 x, float4 c, float4 s, int c4) {
  f32x4 y;
  const float cv[4] = {c.x, c.y, c.z, c.w};
  const float sv[4] = {s.x, s.y, s.z, s.w};
  if constexpr (RM == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = (float)x[r];
  } else if constexpr (RM == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float xp = (float)x[r ^ 1];
      y[r] = (float)x[r] * cv[r] + ((r & 1) ? xp : -xp) * sv[r];
    }
  } else {
    const uint2 u = __builtin_bit_cast(uint2, x);
    const uint2 w = {(uint32_t)__shfl_xor((int)u.x, 2, 64), (uint32_t)__shfl_xor((int)u.y, 2, 64)};
    const bf16x4 xp = __builtin_bit_cast(bf16x4, w);
    const float sg = (c4 & 2) ? 1.f : -1.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = (float)x[r] * cv[r] + sg * (float)xp[r] * sv[r];
  }
  return y;
}

// rope_bwd of dims 4 kap .. 4 kap + 3 of one head row in the MFMA result layout; cs / sn point at
// dim 0 of the head in the row's table row. Halves: the partner dims sit in lane ^ 32.
template <int RM>
__device__ __forceinline__ f32x4 ss_rope_bwd(f32x4 y, const float* cs, const float* sn, int kap) {
  if constexpr (RM == 0) return y;
  const float4 c = *(const float4*)(cs + 4 * kap);
  const float cv[4] = {c.x, c.y, c.z, c.w};
  f32x4 out;
  if constexpr (RM == 1) {
    const float4 s = *(const float4*)(sn + 4 * kap);
    const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float sg = (r & 1) ? 1.f : -1.f;
      out[r] = y[r] * cv[r] - sg * y[r ^ 1] * sv[r ^ 1];
    }
  } else {
    const float4 s = *(const float4*)(sn + 4 * (kap ^ 2));
    const float sv[4] = {s.x, s.y, s.z, s.w};
    const float sg = (kap & 2) ? 1.f : -1.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] = y[r] * cv[r] - sg * __shfl_xor(y[r], 32, 64) * sv[r];
  }
  return out;
}

// Transposed operand from a row-major LDS tile: A[i][4 kap + j] = tile[row0 + 4 kap + j][col0 + i]
// for lane (i = l16, kap), with ds_read_b64_tr_b16.
__device__ __forceinline__ bf16x4 ss_opT(const bf16* tile, int row0, int col0, int l16, int kap) {
  const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)(tile + (row0 + 4 * kap + (l16 >> 2)) * SS_STR + col0 + 4 * (l16 & 3)));
  return __builtin_bit_cast(bf16x4, t);
}

__device__ __forceinline__ bf16x4 ss_row4(const bf16* tile, int row, int col) {
  return *(const bf16x4*)(tile + row * SS_STR + col);
}

template <int RM, bool HB>
__global__ __launch_bounds__(SS_NT, 4) void ss_bwd_kernel(SbParams p) {
  __shared__ __attribute__((aligned(16))) SsLds sh;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int hg = work % (SB_H / SS_HG), b = work / (SB_H / SS_HG);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nqb = (p.Lq + 15) >> 4, nkb = (p.Lk + 15) >> 4;
  const int nq16 = nqb * 16, nk16 = nkb * 16;

  // ---- fill: thread = (row of a 32-row pass, 4-dim chunk c); two passes per round for loads in
  // flight. Rows past Lq / Lk hold the last valid row (clamped): a padded query gets P = 0 in phase 2
  // (its statistic is +inf), a padded key gets P = 0 in phase 1 (b2 = -inf) and is not stored, so
  // their finite values contribute nothing. Buffer loads with 32-bit byte offsets from the batch
  // element's base (the launcher checks that every offset fits).
  {
    const int c = tid & 15, r0 = tid >> 4;
    const int dl = 4 * c, dg = hg * SS_W + dl;
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.q + b * p.q_sb, 0, p.Lq * (int)p.q_sr * 2, TA_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.k + b * p.k_sb, 0, p.Lk * (int)p.k_sr * 2, TA_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.v + b * p.v_sb, 0, p.Lk * (int)p.v_sr * 2, TA_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.o + (int64_t)b * p.Lq * SB_E, 0, p.Lq * SB_E * 2, TA_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.dout + (int64_t)b * p.Lq * SB_E, 0, p.Lq * SB_E * 2, TA_BUF_WORD3);
    const int nmax = nq16 > nk16 ? nq16 : nk16;
    for (int i0 = 0; 32 * i0 < nmax; i0 += 2) {
      bf16x4 qx[2], ox[2], dx[2], kx[2], vx[2];
      float4 qc[2], qs[2], kc[2], ks[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {  // loads only
        const int row = r0 + 32 * (i0 + u);
        const int rq = row < p.Lq ? row : p.Lq - 1, rk = row < p.Lk ? row : p.Lk - 1;
        const int oq = (rq * SB_E + dg) * 2;
        qx[u] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(qrs, (rq * (int)p.q_sr + dg) * 2, 0, 0));
        ox[u] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(ors, oq, 0, 0));
        dx[u] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(drs, oq, 0, 0));
        kx[u] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(krs, (rk * (int)p.k_sr + dg) * 2, 0, 0));
        vx[u] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(vrs, (rk * (int)p.v_sr + dg) * 2, 0, 0));
        if constexpr (RM != 0) {
          const int tc = dg & p.tab_cm;
          qc[u] = *(const float4*)(p.cq + (rq << p.tab_ss) + tc);
          qs[u] = *(const float4*)(p.sq + (rq << p.tab_ss) + tc);
          kc[u] = *(const float4*)(p.ck + (rk << p.tab_ss) + tc);
          ks[u] = *(const float4*)(p.sk + (rk << p.tab_ss) + tc);
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = r0 + 32 * (i0 + u);  // < 128: the loop covers at most 128 rows
        const f32x4 yq = ss_rope_fwd<RM>(qx[u], qc[u], qs[u], c & 3);
        float part = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) part += (float)dx[u][r] * (float)ox[u][r];
        part += __shfl_xor(part, 1, 64);  // the 4 chunks of one head: lanes c ^ 1, c ^ 2
        part += __shfl_xor(part, 2, 64);
        *(bf16x4*)(sh.q + row * SS_STR + dl) = cvt_bf16x4(yq * p.scale);
        *(bf16x4*)(sh.d + row * SS_STR + dl) = dx[u];
        if ((c & 3) == 0) sh.nd[c >> 2][row] = -part;
        if constexpr (RM != 0)
          *(bf16x4*)(sh.k + row * SS_STR + dl) = cvt_bf16x4(ss_rope_fwd<RM>(kx[u], kc[u], ks[u], c & 3));
        else
          *(bf16x4*)(sh.k + row * SS_STR + dl) = kx[u];
        *(bf16x4*)(sh.v + row * SS_STR + dl) = vx[u];
      }
    }
    for (int j = tid; j < nk16; j += SS_NT) sh.b2[j] = sb_b2(p, b, j);
  }
  __syncthreads();

  const int gl = wave & (SS_HG - 1), par = wave / SS_HG;  // head within the group, block parity
  const int l16 = lane & 15, kap = lane >> 4;
  const int hd = gl * SB_D;                    // the head's first dim in the group
  const int dglob = hg * SS_W + hd + 4 * kap;  // merged dim of this lane's 4 output dims

  // ---- phase 1: per query block, statistics, dq. Without a key bias the scores are reduced raw
  // (b2 only masks the padded keys of the last block) and the log2e factor goes into the exponent's fma.
  // dq' = (1 / l) sum_k e_k (dP_k - D) k' with e = exp2(x - m): the products take e (dP - D), rounded
  // to bf16 as dS is, and 1 / l scales their sum (one multiply per query instead of one per score).
  for (int qb = par; qb < nqb; qb += 2) {
    const int qr = 16 * qb + l16;
    const bf16x4 qop = ss_row4(sh.q, qr, hd + 4 * kap);
    const bf16x4 dop = ss_row4(sh.d, qr, hd + 4 * kap);
    const float nds = sh.nd[gl][qr];
    f32x4 x[8];
    float tm = TA_NEG_INF;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      if (kt < nkb) {
        x[kt] = mfma16x16x16(ss_row4(sh.k, 16 * kt + l16, hd + 4 * kap), qop, f32x4{0.f, 0.f, 0.f, 0.f});
        if (HB || kt == nkb - 1) {
          const f32x4 b2 = *(const f32x4*)(sh.b2 + 16 * kt + 4 * kap);
#pragma unroll
          for (int r = 0; r < 4; ++r) x[kt][r] = HB ? fmaf(x[kt][r], TA_LOG2E, b2[r]) : x[kt][r] + b2[r];
        }
        tm = fmaxf(tm, fmaxf(fmaxf(x[kt][0], x[kt][1]), fmaxf(x[kt][2], x[kt][3])));
      }
    }
    // m: row maximum in log2 units; x -> exp2(x log2e - m) (no bias) or exp2(x - m)
    const float mraw = quad_max(tm);  // finite: key 0 exists
    const float m = HB ? mraw : mraw * TA_LOG2E;
    float l = 0.f;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      if (kt < nkb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[kt][r] = __builtin_amdgcn_exp2f(HB ? x[kt][r] - m : fmaf(x[kt][r], TA_LOG2E, -m));
          l += x[kt][r];
        }
      }
    }
    l = quad_sum(l);  // >= 1
    const float inv = __builtin_amdgcn_rcpf(l);
    const f32x4 cnd = {nds, nds, nds, nds};
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // key tiles in pairs: one 32-deep product per pair (a lone last tile: a 16-deep one)
#pragma unroll
    for (int kt = 0; kt < 8; kt += 2) {
      if (kt < nkb) {
        const f32x4 dp0 = mfma16x16x16(ss_row4(sh.v, 16 * kt + l16, hd + 4 * kap), dop, cnd);  // dP - D
        f32x4 e0;
#pragma unroll
        for (int r = 0; r < 4; ++r) e0[r] = x[kt][r] * dp0[r];
        if (kt + 1 < nkb) {
          const f32x4 dp1 = mfma16x16x16(ss_row4(sh.v, 16 * kt + 16 + l16, hd + 4 * kap), dop, cnd);
          f32x4 e1;
#pragma unroll
          for (int r = 0; r < 4; ++r) e1[r] = x[kt + 1][r] * dp1[r];
          acc = mfma16x16x32(ss_opT(sh.k, 16 * kt, hd, l16, kap), ss_opT(sh.k, 16 * kt + 16, hd, l16, kap),
                             cvt_bf16x4(e0), cvt_bf16x4(e1), acc);
        } else {
          acc = mfma16x16x16(ss_opT(sh.k, 16 * kt, hd, l16, kap), cvt_bf16x4(e0), acc);
        }
      }
    }
    const float lg = __builtin_amdgcn_logf(l);
    if (kap == 0) {
      if (HB) {
        sh.mx[gl][qr] = qr < p.Lq ? m : __builtin_inff();
        sh.lg[gl][qr] = lg;
      } else {
        sh.mx[gl][qr] = qr < p.Lq ? -(m + lg) : TA_NEG_INF;
      }
    }
    f32x4 y;
    const float ysc = p.scale * inv;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = acc[r] * ysc;
    const int qc = qr < p.Lq ? qr : 0;
    y = ss_rope_bwd<RM>(y, p.cq + ((int64_t)qc << p.tab_ss) + ((hg * SS_W + hd) & p.tab_cm),
                        p.sq + ((int64_t)qc << p.tab_ss) + ((hg * SS_W + hd) & p.tab_cm),
                        kap);
    if (qr < p.Lq) *(bf16x4*)((bf16*)p.dq + b * p.dq_sb + (int64_t)qr * p.dq_sr + dglob) = cvt_bf16x4(y);
  }
  __syncthreads();

  // ---- phase 2: per key block, dk and dv over every query block. P = exp2(s log2e + b2 - m - lg);
  // without a key bias one fma against -(m + lg) (padded keys: not stored, their P is not used).
  // The query blocks go in pairs, each pair's dv and dk in one 32-deep product (a lone last block: a
  // 16-deep one); the loop is unrolled over the at most 8 blocks, so the LDS offsets are constants.
  for (int kb = par; kb < nkb; kb += 2) {
    const int kr = 16 * kb + l16;
    const bf16x4 kop = ss_row4(sh.k, kr, hd + 4 * kap);
    const bf16x4 vop = ss_row4(sh.v, kr, hd + 4 * kap);
    const float b2 = HB ? sh.b2[kr] : 0.f;
    // bf16 P and dS of query block qs against this key block: S[query 16 qs + 4 kap + r][key kr],
    // dP - D likewise (the accumulator input is -D of those queries)
    auto pds = [&](int qs, bf16x4& pb, bf16x4& db) {
      const f32x4 s = mfma16x16x16(ss_row4(sh.q, 16 * qs + l16, hd + 4 * kap), kop, f32x4{0.f, 0.f, 0.f, 0.f});
      const f32x4 dp = mfma16x16x16(ss_row4(sh.d, 16 * qs + l16, hd + 4 * kap), vop,
                                    *(const f32x4*)(&sh.nd[gl][16 * qs + 4 * kap]));
      const f32x4 ms = *(const f32x4*)(&sh.mx[gl][16 * qs + 4 * kap]);
      f32x4 pr, dsf;
      if constexpr (HB) {
        const f32x4 ls = *(const f32x4*)(&sh.lg[gl][16 * qs + 4 * kap]);
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f((fmaf(s[r], TA_LOG2E, b2) - ms[r]) - ls[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f(fmaf(s[r], TA_LOG2E, ms[r]));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) dsf[r] = pr[r] * dp[r];
      pb = cvt_bf16x4(pr);
      db = cvt_bf16x4(dsf);
    };
    f32x4 dk = {0.f, 0.f, 0.f, 0.f}, dv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int qs = 0; qs < 8; qs += 2) {
      if (qs < nqb) {
        bf16x4 pa, da;
        pds(qs, pa, da);
        if (qs + 1 < nqb) {
          bf16x4 pb, db;
          pds(qs + 1, pb, db);
          dv = mfma16x16x32(ss_opT(sh.d, 16 * qs, hd, l16, kap), ss_opT(sh.d, 16 * qs + 16, hd, l16, kap), pa, pb, dv);
          dk = mfma16x16x32(ss_opT(sh.q, 16 * qs, hd, l16, kap), ss_opT(sh.q, 16 * qs + 16, hd, l16, kap), da, db, dk);
        } else {
          dv = mfma16x16x16(ss_opT(sh.d, 16 * qs, hd, l16, kap), pa, dv);
          dk = mfma16x16x16(ss_opT(sh.q, 16 * qs, hd, l16, kap), da, dk);
        }
      }
    }
    const int kc = kr < p.Lk ? kr : 0;
    const f32x4 y = ss_rope_bwd<RM>(dk, p.ck + ((int64_t)kc << p.tab_ss) + ((hg * SS_W + hd) & p.tab_cm),
                                    p.sk + ((int64_t)kc << p.tab_ss) + ((hg * SS_W + hd) & p.tab_cm), kap);
    if (kr < p.Lk) {
      *(bf16x4*)((bf16*)p.dk + b * p.dk_sb + (int64_t)kr * p.dk_sr + dglob) = cvt_bf16x4(y);
      *(bf16x4*)((bf16*)p.dv + b * p.dv_sb + (int64_t)kr * p.dv_sr + dglob) = cvt_bf16x4(dv);
    }
  }
}

// The fused short kernel's RoPE form for these parameters, or -1 when it does not cover them.
int ss_mode(const SbParams& p) {
  if (p.rope == 0) return 0;
  if (p.rope == 1 && p.rot == 16) return 1;
  if (p.rope == 2 && p.half == 8 && p.rot == 16) return 2;
  return -1;
}

template <typename T, bool RP>
void launch_sb(const SbParams& p, int64_t nwg_q, int64_t nkb, hipStream_t stream) {
  const dim3 block(SB_NW * 64);
  if (nwg_q > 0 && p.Lk <= SB_KT)
    hipLaunchKernelGGL((sb_dq_kernel<T, true, RP>), dim3((unsigned)(p.B * nwg_q * SB_H)), block, 0, stream, p);
  else if (nwg_q > 0)
    hipLaunchKernelGGL((sb_dq_kernel<T, false, RP>), dim3((unsigned)(p.B * nwg_q * SB_H)), block, 0, stream, p);
  if (p.bias)
    hipLaunchKernelGGL((sb_dkdv_kernel<T, RP, true>), dim3((unsigned)(p.B * nkb * SB_H)), block, 0, stream, p);
  else
    hipLaunchKernelGGL((sb_dkdv_kernel<T, RP, false>), dim3((unsigned)(p.B * nkb * SB_H)), block, 0, stream, p);
}

template <typename T>
void launch_bwd(SbParams p, hipStream_t stream) {
  if constexpr (sizeof(T) == 2) {
    const int rm = ss_mode(p);
    // byte offsets within a batch element fit 32 bits (buffer loads)
    const bool fits = (int64_t)p.Lq * p.q_sr * 2 < INT32_MAX && (int64_t)p.Lk * p.k_sr * 2 < INT32_MAX &&
                      (int64_t)p.Lk * p.v_sr * 2 < INT32_MAX && p.q_sr >= 0 && p.k_sr >= 0 && p.v_sr >= 0;
    if (p.Lq >= 1 && p.Lk >= 1 && p.Lq <= SS_ROWS && p.Lk <= SS_ROWS && rm >= 0 && fits) {
      const dim3 grid((unsigned)(p.B * (SB_H / SS_HG)));
      const bool hb = p.bias != nullptr;
      if (rm == 0 && hb)
        hipLaunchKernelGGL((ss_bwd_kernel<0, true>), grid, dim3(SS_NT), 0, stream, p);
      else if (rm == 0)
        hipLaunchKernelGGL((ss_bwd_kernel<0, false>), grid, dim3(SS_NT), 0, stream, p);
      else if (rm == 1 && hb)
        hipLaunchKernelGGL((ss_bwd_kernel<1, true>), grid, dim3(SS_NT), 0, stream, p);
      else if (rm == 1)
        hipLaunchKernelGGL((ss_bwd_kernel<1, false>), grid, dim3(SS_NT), 0, stream, p);
      else if (hb)
        hipLaunchKernelGGL((ss_bwd_kernel<2, true>), grid, dim3(SS_NT), 0, stream, p);
      else
        hipLaunchKernelGGL((ss_bwd_kernel<2, false>), grid, dim3(SS_NT), 0, stream, p);
      return;
    }
  }
  const int64_t nqb = (p.Lq + SB_QB - 1) / SB_QB, nkb = (p.Lk + SB_KB - 1) / SB_KB;
  // keys in one tile: runs of query blocks per workgroup (one fill each), still >= ~16 workgroups
  // per CU over the grid
  int64_t qbpw = 1;
  if (p.Lk <= SB_KT) {
    qbpw = (p.B * nqb * SB_H + 4095) / 4096;
    qbpw = qbpw < 1 ? 1 : (qbpw > nqb ? nqb : qbpw);
  }
  p.qbpw = (int)qbpw;
  const int64_t nwg_q = nqb > 0 ? (nqb + qbpw - 1) / qbpw : 0;
  // no query (Lq = 0): only the dk/dv kernel runs, and writes zeros
  if (p.rope)
    launch_sb<T, true>(p, nwg_q, nkb, stream);
  else
    launch_sb<T, false>(p, nwg_q, nkb, stream);
}

}  // namespace

int64_t tabicl_launch_smallhead_bwd_ws_bytes(int64_t B, int64_t Lq) {
  const int64_t n = B * SB_H * Lq;
  return 3 * ((n * 4 + 255) / 256 * 256);
}

int tabicl_launch_smallhead_bwd(const void* q, int64_t q_sb, int64_t q_sr, const void* k, int64_t k_sb,
                                int64_t k_sr, const void* v, int64_t v_sb, int64_t v_sr, const void* o,
                                const void* dout, void* dq, int64_t dq_sb, int64_t dq_sr, void* dk,
                                int64_t dk_sb, int64_t dk_sr, void* dv, int64_t dv_sb, int64_t dv_sr,
                                const float* bias, int64_t bias_sb, const float* cq, const float* sq,
                                const float* ck, const float* sk, int rope, int half, int rot, float scale,
                                int64_t B, int64_t Lq, int64_t Lk, int dtype, void* ws, int64_t ws_bytes,
                                hipStream_t stream) {
  if (ws_bytes < tabicl_launch_smallhead_bwd_ws_bytes(B, Lq)) return (int)hipErrorInvalidValue;
  SbParams p;
  p.q = q; p.q_sb = q_sb; p.q_sr = q_sr;
  p.k = k; p.k_sb = k_sb; p.k_sr = k_sr;
  p.v = v; p.v_sb = v_sb; p.v_sr = v_sr;
  p.o = o; p.dout = dout;
  p.dq = dq; p.dq_sb = dq_sb; p.dq_sr = dq_sr;
  p.dk = dk; p.dk_sb = dk_sb; p.dk_sr = dk_sr;
  p.dv = dv; p.dv_sb = dv_sb; p.dv_sr = dv_sr;
  p.bias = bias; p.bias_sb = bias_sb;
  p.cq = cq; p.sq = sq; p.ck = ck; p.sk = sk;
  const bool shared = (rope & TA_ROPE_SHARED) != 0;
  p.rope = rope & ~TA_ROPE_SHARED; p.half = half; p.rot = rot;
  p.tab_ss = shared ? 4 : 7;
  static_assert(SB_D == 16 && SB_E == 128, "table row strides as shifts");
  p.tab_cm = shared ? SB_D - 1 : SB_E - 1;
  p.scale = scale;
  p.B = (int)B; p.Lq = (int)Lq; p.Lk = (int)Lk;
  const int64_t part = tabicl_launch_smallhead_bwd_ws_bytes(B, Lq) / 3;
  p.mx = (float*)ws;
  p.ll = (float*)((char*)ws + part);
  p.dd = (float*)((char*)ws + 2 * part);
  if (dtype == 0)
    launch_bwd<bf16>(p, stream);
  else
    launch_bwd<float>(p, stream);
  return (int)hipGetLastError();
}
