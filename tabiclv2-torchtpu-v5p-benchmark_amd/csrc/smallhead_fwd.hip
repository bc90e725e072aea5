// Fused small-head attention (8 heads x 16 dims, merged width E = 128) for gfx950.
//
// The kernels here serve the four small-head ops of the reference (hx, hxq, pk_self, pk_cross;
// scripts/tabicl_tpu_pallas_attn.py): q/k/v are read straight from their merged-head rows
// (separate [B, L, E], packed K|V [B, L, 2E] or packed Q|K|V [B, L, 3E]) and the output is
// written merged [B, Lq, E]. Per (batch, head):
//   O = softmax(q' k'^T + bias [+ -inf past valid]) V,
//   q' = cast(rope(q) * scale), k' = cast(rope(k)) (RoPE and scale in fp32; no RoPE = identity),
// fp32 scores/softmax, probabilities cast to the value dtype before PV. tabicl_launch_smallhead
// picks by shape: sh_resident_kernel (bf16, all keys in LDS), sf_kernel (fp32), the streaming
// kernel of smallhead_stream.hip (bf16, long keys) or smallhead_fwd_kernel below (bf16 with RoPE or
// a key bias and long keys, partial-rotary RoPE).
//
// smallhead_fwd_kernel: a workgroup of 8 waves owns one batch element and a block of 128 queries
// (wave w: queries 16w..16w+15, all 8 heads; per-head online-softmax state in registers).
// Keys stream through LDS in tiles of KT keys x all heads (K row-major, V transposed to
// [E][KT], per-key bias pre-multiplied by log2(e), -inf past the valid length). When all keys
// fit one tile the workgroup keeps them resident and walks several query blocks.
// MFMA 16x16x16 (bf16) or 4 x 16x16x4 (fp32), in the orientation
//   S^T (16 keys x 16 queries) = K Q^T,  O^T (16 dims x 16 queries) += V^T P^T
// so that the S^T accumulator is already the B operand of the PV product and every softmax
// statistic of a query lives in the four lanes l%16 + 16j.
#include <atomic>

#include "common.h"
#include "launch.h"

namespace {

constexpr int SH_E = 128;
constexpr int SH_H = 8;
constexpr int SH_D = 16;
constexpr int SH_NW = 8;
constexpr int SH_QB = 16 * SH_NW;
constexpr float SH_LAZY = 8.0f;
constexpr float SH_BIAS_FLOOR = -1e37f;

struct ShParams {
  const void* q;
  int64_t q_sb, q_sr;
  const void* k;
  int64_t k_sb, k_sr;
  const void* v;
  int64_t v_sb, v_sr;
  void* o;
  int64_t o_sb, o_sr;
  const float* bias;
  int64_t bias_sb;
  const int32_t* valid;
  int valid_n;
  const float* cq;
  const float* sq;
  const float* ck;
  const float* sk;
  int rope, half, rot;
  float scale;
  int B, Lq, Lk;
  int nqb, qbpw, nwg_b;
  int exact_scale;  // fold scale and log2e into the K operand: scale is a power of two (bf16(q * scale)
                    // needs no rounding) and the runs are long enough to amortise the K split
  int pow2_scale;   // scale is a power of two
  float qc;         // scale * log2e (exact for a power-of-two scale)
  int half_last;    // the last 32-key group's upper 16 keys are all past Lk (resident kernel, 4 groups)
  // RoPE tables: element (position, dim d) at position * tab_sr + (d & tab_cm); [L, E] tables give
  // (E, E - 1), tables of one head's columns shared by every head give (16, 15)
  int tab_sr, tab_cm;
  // query rows needed per batch element (qlen[b], or qlen[0] for all; null: all Lq rows): the
  // resident kernel neither computes nor writes the rows at or past it
  const int32_t* qlen;
  int qlen_n;
  // batch elements computed by another kernel of the same call (skip[b], or skip[0] for all; null:
  // none): smallhead_fwd_kernel returns for them
  const int32_t* skip;
  int skip_n;
  // persistent resident kernel: the q RoPE tables are staged in LDS rows of their own (cross
  // attention with q tables other than the key tables) instead of reading the key rows' tables
  int rp_qsep;
};

template <typename T, int KT> struct ShLds {
  static constexpr int PAD = 16 / sizeof(T);
  static constexpr int KSTR = SH_E + PAD;
  static constexpr int VSTR = KT + PAD;
  static constexpr int K_ELEMS = KT * KSTR;
  static constexpr int V_ELEMS = SH_E * VSTR;
};

template <typename T, int KT>
__device__ __forceinline__ void sh_fill(const ShParams& p, T* lds_k, T* lds_vt, float* lds_b2,
                                        int b, int k0, int lk) {
  typedef ShLds<T, KT> L;
  const int tid = threadIdx.x, nt = blockDim.x;
  const T* kbase = (const T*)p.k + b * p.k_sb;
  const T* vbase = (const T*)p.v + b * p.v_sb;
  // K: unit = (key row, 4 dims); RoPE applied in fp32 then cast
#pragma unroll 1
  for (int u = tid; u < KT * (SH_E / 4); u += nt) {
    const int row = u >> 5, d0 = (u & 31) * 4, key = k0 + row;
    typedef typename OpVec<T, 4>::type Op4;
    Op4 val;
    if (key < lk) {
      const T* src = kbase + (int64_t)key * p.k_sr;
      if (p.rope) {
        const f32x4 y = rope4<T>(src, p.ck + (int64_t)key * p.tab_sr, p.sk + (int64_t)key * p.tab_sr, d0,
                                 p.rope, p.half, p.rot, d0 & p.tab_cm);
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = from_f32<T>(y[r]);
      } else {
        val = *(const Op4*)(src + d0);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) val[r] = from_f32<T>(0.f);
    }
    *(Op4*)(lds_k + row * L::KSTR + d0) = val;
  }
  // V: unit = (key pair, head), transposed store [E][KT]
#pragma unroll 1
  for (int u = tid; u < (KT / 2) * SH_H; u += nt) {
    const int pr = u >> 3, g = u & 7, key = k0 + 2 * pr;
    constexpr int EPC = 16 / sizeof(T);
    union { uint4 u4[SH_D / EPC]; T e[SH_D]; } a, c;
#pragma unroll
    for (int i = 0; i < SH_D / EPC; ++i) {
      a.u4[i] = make_uint4(0, 0, 0, 0);
      c.u4[i] = make_uint4(0, 0, 0, 0);
    }
    if (key < lk) {
#pragma unroll
      for (int i = 0; i < SH_D / EPC; ++i)
        a.u4[i] = ldg16(vbase + (int64_t)key * p.v_sr + g * SH_D + i * EPC);
    }
    if (key + 1 < lk) {
#pragma unroll
      for (int i = 0; i < SH_D / EPC; ++i)
        c.u4[i] = ldg16(vbase + (int64_t)(key + 1) * p.v_sr + g * SH_D + i * EPC);
    }
    typedef T T2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int j = 0; j < SH_D; ++j) {
      T2 pair;
      pair[0] = a.e[j];
      pair[1] = c.e[j];
      *(T2*)(lds_vt + (g * SH_D + j) * L::VSTR + 2 * pr) = pair;
    }
  }
  // per-key additive term in log2 units
  for (int j = tid; j < KT; j += nt) {
    const int key = k0 + j;
    float b2 = TA_NEG_INF;
    if (key < lk) {
      b2 = 0.f;
      if (p.bias) b2 = fmaxf(p.bias[b * p.bias_sb + key] * TA_LOG2E, SH_BIAS_FLOOR);
    }
    lds_b2[j] = b2;
  }
}

template <typename T, int KT>
__global__ __launch_bounds__(SH_NW * 64) void smallhead_fwd_kernel(ShParams p) {
  typedef ShLds<T, KT> L;
  typedef typename OpVec<T, 4>::type Op4;
  constexpr int NKT = KT / 16;
  __shared__ __attribute__((aligned(16))) T lds_k[L::K_ELEMS];
  __shared__ __attribute__((aligned(16))) T lds_vt[L::V_ELEMS];
  __shared__ __attribute__((aligned(16))) float lds_b2[KT];

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int b = work / p.nwg_b;
  const int qb0 = (work % p.nwg_b) * p.qbpw;
  if (p.skip && p.skip[p.skip_n == 1 ? 0 : b]) return;

  int lk = p.Lk;
  if (p.valid) {
    int vl = p.valid[p.valid_n == 1 ? 0 : b];
    vl = vl < 0 ? 0 : vl;
    lk = vl < lk ? vl : lk;
  }
  const int ntiles = (lk + KT - 1) / KT;
  const bool resident = ntiles <= 1;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const T* qbase = (const T*)p.q + b * p.q_sb;
  T* obase = (T*)p.o + b * p.o_sb;

  for (int qbi = 0; qbi < p.qbpw; ++qbi) {
    const int qb = qb0 + qbi;
    if (qb >= p.nqb) break;
    const int qw0 = qb * SH_QB + wave * 16;
    const int qi = qw0 + l16;
    const bool qok = qi < p.Lq;
    const bool wave_active = qw0 < p.Lq;

    Op4 qop[SH_H];
    f32x4 o[SH_H];
    float m_run[SH_H], l_run[SH_H];
#pragma unroll
    for (int g = 0; g < SH_H; ++g) {
      m_run[g] = TA_NEG_INF;
      l_run[g] = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) { o[g][r] = 0.f; qop[g][r] = from_f32<T>(0.f); }
    }
    if (qok) {
      const T* qrow = qbase + (int64_t)qi * p.q_sr;
      if (p.rope) {
#pragma unroll
        for (int g = 0; g < SH_H; ++g) {
          const f32x4 y = rope4<T>(qrow, p.cq + (int64_t)qi * p.tab_sr, p.sq + (int64_t)qi * p.tab_sr,
                                   g * SH_D + 4 * kap, p.rope, p.half, p.rot, (g * SH_D + 4 * kap) & p.tab_cm);
#pragma unroll
          for (int r = 0; r < 4; ++r) qop[g][r] = from_f32<T>(y[r] * p.scale);
        }
      } else {
#pragma unroll
        for (int g = 0; g < SH_H; ++g) {
          const Op4 raw = *(const Op4*)(qrow + g * SH_D + 4 * kap);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            qop[g][r] = p.scale == 1.f ? raw[r] : from_f32<T>(to_f32<T>(raw[r]) * p.scale);
        }
      }
    }

    for (int t = 0; t < ntiles; ++t) {
      if (!(resident && qbi > 0)) {
        __syncthreads();
        sh_fill<T, KT>(p, lds_k, lds_vt, lds_b2, b, t * KT, lk);
        __syncthreads();
      }
      if (!wave_active) continue;
#pragma unroll
      for (int g = 0; g < SH_H; ++g) {
        f32x4 s[NKT];
        float mx = TA_NEG_INF;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
          const Op4 a = *(const Op4*)(lds_k + (16 * kt + l16) * L::KSTR + g * SH_D + 4 * kap);
          f32x4 z = {0.f, 0.f, 0.f, 0.f};
          s[kt] = mfma16x16x16(a, qop[g], z);
          const f32x4 b2 = *(const f32x4*)(lds_b2 + 16 * kt + 4 * kap);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            s[kt][r] = fmaf(s[kt][r], TA_LOG2E, b2[r]);
            mx = fmaxf(mx, s[kt][r]);
          }
        }
        mx = xor_max(mx, 16);
        mx = xor_max(mx, 32);
        const float m_new = fmaxf(m_run[g], mx);
        if (wave_any(m_new - m_run[g] > SH_LAZY)) {
          const float alpha = __builtin_amdgcn_exp2f(m_run[g] - m_new);
          l_run[g] *= alpha;
#pragma unroll
          for (int r = 0; r < 4; ++r) o[g][r] *= alpha;
          m_run[g] = m_new;
        }
        const float mr = m_run[g];
        float lsum = 0.f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
          Op4 pv;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pr = __builtin_amdgcn_exp2f(s[kt][r] - mr);
            lsum += pr;
            pv[r] = from_f32<T>(pr);
          }
          const Op4 a = *(const Op4*)(lds_vt + (g * SH_D + l16) * L::VSTR + 16 * kt + 4 * kap);
          o[g] = mfma16x16x16(a, pv, o[g]);
        }
        l_run[g] += lsum;
        // keep the per-head bodies apart: interleaving heads only raises register pressure
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    if (qok) {
      T* orow = obase + (int64_t)qi * p.o_sr;
#pragma unroll
      for (int g = 0; g < SH_H; ++g) {
        float lt = xor_sum(l_run[g], 16);
        lt = xor_sum(lt, 32);
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        Op4 ov;
#pragma unroll
        for (int r = 0; r < 4; ++r) ov[r] = from_f32<T>(o[g][r] * inv);
        *(Op4*)(orow + g * SH_D + 4 * kap) = ov;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Resident-keys kernel (bf16, Lk <= 128: row self attention over 104 tokens, CLS, ISAB-2 over the
// 128 inducing points, hxq over short key sets). A workgroup of 8 waves takes one batch element and a
// run of 16-query blocks. It loads all keys once into LDS (K with RoPE, row-major V, per-key additive
// term b2 = bias*log2e, 0 without bias, -inf past the valid length); wave g then copies head g's K
// and V^T MFMA operands into registers and walks the run's query blocks, each one pass over all keys:
//   x = K (q' log2e) + b2         16x16x32 MFMAs: q' log2e as a bf16 high part and the bf16
//                                 remainder in the two k-halves, b2 as the accumulator input (a zero
//                                 accumulator for key groups that need no b2)
//   p = bf16(exp2(x)), l = 1 p    (ones-operand MFMA)
//   O^T = V^T P^T / l             V^T read once with ds_read_b64_tr_b16 from the row-major V tile
// q is read with buffer loads two blocks ahead of its use and O written with range-checked buffer
// stores, so the main loop reads no LDS except b2 of masked groups.
// exp2 takes x without the row maximum subtracted; only when l falls outside [2^-64, 2^64] (or is
// not finite) is the block recomputed with the exact maximum subtracted. Otherwise every p lies
// below 2^64 and every p that matters above the fp32 floor, and fp32 / bf16 relative precision does
// not depend on scale, so both give the softmax to rounding.
// ---------------------------------------------------------------------------------------------
constexpr int RS_LK = 128;
constexpr int RS_KSTR = SH_E + 8;   // K rows of 272 B: a 16-row b128 operand read covers all banks
constexpr int RS_VSTR = SH_E + 16;  // V rows of 288 B: the transposed reads of 8 rows cover all banks
constexpr float RS_L_HI = 0x1p64f;
constexpr float RS_L_LO = 0x1p-64f;

// One rotated K element, x cos + x' sin with x' the signed partner dim, in one fixed rounding order
// (both resident kernels use it, so they give the same bits).
__device__ __forceinline__ float rs_rot(float x, float xp, float c, float s) { return __builtin_fmaf(xp, s, x * c); }

// This lane's 8 dims of q (those of its B-operand k-slots) at byte offset off of the workgroup's q
// rows. A buffer load: rows past Lq lie outside the resource and read as zero, and the compiler
// keeps a load issued ahead of its use where it is (it does not merge these into the loop's phi).
__device__ __forceinline__ bf16x8 rs_qraw(__amdgpu_buffer_rsrc_t qrsrc, int off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(qrsrc, off, 0, 0));
}

// Four fp32 table values (cos or sin of 4 dims) at byte offset off, likewise.
__device__ __forceinline__ f32x4 rs_tab(__amdgpu_buffer_rsrc_t rsrc, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
}

// Lanes l and l ^ 32 (G and G ^ 2) share the 8 dims d8..d8+7 of their operand k-slots; each has
// computed 4 of them (G < 2: d8..d8+3, G >= 2: d8+4..d8+7). One v_permlane32_swap per word trades
// the upper lanes' vdst with the lower lanes' vsrc; with both operands = the lane's own 4, the
// swapped vdst holds dims d8..d8+3 and the swapped vsrc dims d8+4..d8+7 in every lane.
__device__ __forceinline__ bf16x8 rs_pair8(bf16x4 mine, int G) {
  (void)G;
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
  const u32x2 sw = __builtin_bit_cast(u32x2, mine);
  u32x4v w;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(sw[k], sw[k], false, false);
    w[k] = r[0];
    w[2 + k] = r[1];
  }
  return __builtin_bit_cast(bf16x8, w);
}

// K operand with c = scale * log2e folded in: k c as a bf16 high part (G < 2, k-slots 0..15) and
// the bf16 remainder (G >= 2, k-slots 16..31), so that a raw q' operand in both halves gives
// x = q' k c to ~2^-17 relative.
__device__ __forceinline__ bf16x8 rs_ksplit(bf16x8 k, float c, int G) {
  bf16x8 op;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = (float)k[j] * c;
    const bf16 hi = (bf16)x;
    op[j] = G < 2 ? hi : (bf16)(x - (float)hi);
  }
  return op;
}

// q' log2e operand from this lane's 4 values v (v c = q' log2e: v = q' = bf16(rope(q) * scale) and c =
// log2e, or, for a power-of-two scale, v = bf16(rope(q)) and c = scale log2e, the same product
// exactly; the reference's packed kernels, :498-502). Each lane splits its 4 values of x = v c into
// bf16 high parts (vdst) and bf16 remainders fma(v, c, -hi) (vsrc); one v_permlane32_swap per word
// (upper lanes' vdst <-> lower lanes' vsrc) leaves lanes G < 2 with the 8 high parts and lanes
// G >= 2 with the 8 remainders of the shared dims, in k-slot order, with no selects.
__device__ __forceinline__ bf16x8 rs_qsplit(f32x4 v, float c, int G) {
  (void)G;
  f32x4 x, rem;
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = v[j] * c;
  const bf16x4 hi = cvt_bf16x4(x);
#pragma unroll
  for (int j = 0; j < 4; ++j) rem[j] = __builtin_fmaf(v[j], c, -(float)hi[j]);
  const bf16x4 lo = cvt_bf16x4(rem);
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
  const u32x2 hw = __builtin_bit_cast(u32x2, hi), lw = __builtin_bit_cast(u32x2, lo);
  u32x4v w;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(hw[k], lw[k], false, false);
    w[k] = r[0];
    w[2 + k] = r[1];
  }
  return __builtin_bit_cast(bf16x8, w);
}

// Scores of the 32-key group kg, x = K (q' log2e) + b2: lane (l16, G) holds keys 32kg + 4G + r (x0)
// and 32kg + 16 + 4G + r (x1) of query l16 (the k-slot order 8G + j of the 16x16x32 B operand).
// Groups below MF have b2 = 0 for every key (no bias, all keys valid): a zero accumulator.
// skip1: keys 32kg+16.. do not exist (x1 is not computed).
template <int MF>
__device__ __forceinline__ void rs_scores(bf16x8 ka0, bf16x8 ka1, bf16x8 qop, const float* lds_b2, int kg,
                                          int G, f32x4& x0, f32x4& x1, bool skip1 = false) {
  f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
  if (kg >= MF) {
    c0 = *(const f32x4*)(lds_b2 + 32 * kg + 4 * G);
    if (!skip1) c1 = *(const f32x4*)(lds_b2 + 32 * kg + 16 + 4 * G);
  }
  x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka0, qop, c0, 0, 0, 0);
  if (!skip1) x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka1, qop, c1, 0, 0, 0);
}

__device__ __forceinline__ float rs_sum(bf16x8 ones, bf16x8 pv) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pv, zero, 0, 0, 0)[0];
}

// One (16 queries, head) unit over all keys: p = bf16(exp2(x - sub)), l = sum p (ones-operand
// MFMA), o = V^T p^T, accumulated group by group in key order.
// HALF: the last group's keys 32(NG-1)+16.. are all past Lk, so its second score product and
// their probabilities are skipped (zero).
template <int NG, int MF, bool SUB, bool HALF>
__device__ __forceinline__ void rs_unit(const bf16x8 (&ka)[NG][2], const bf16x8 (&va)[NG], bf16x8 ones,
                                        bf16x8 qop, const float* lds_b2, int G, float sub, f32x4& o, float& l) {
  o = f32x4{0.f, 0.f, 0.f, 0.f};
  l = 0.f;
#pragma unroll
  for (int kg = 0; kg < NG; ++kg) {
    const bool half = HALF && kg == NG - 1;
    f32x4 x0, x1;
    rs_scores<MF>(ka[kg][0], ka[kg][1], qop, lds_b2, kg, G, x0, x1, half);
    bf16x8 pv;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pv[r] = (bf16)__builtin_amdgcn_exp2f(SUB ? x0[r] - sub : x0[r]);
      pv[4 + r] = half ? (bf16)0.f : (bf16)__builtin_amdgcn_exp2f(SUB ? x1[r] - sub : x1[r]);
    }
    const float sk = rs_sum(ones, pv);
    l = kg == 0 ? sk : l + sk;  // sums are >= +0: the first needs no add
    o = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[kg], pv, o, 0, 0, 0);
    // keep the groups apart: hoisting every group's scores first costs registers
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Largest x of query l16 over all keys (keys past the valid length hold -inf).
template <int NG, int MF, bool HALF>
__device__ __forceinline__ float rs_max(const bf16x8 (&ka)[NG][2], bf16x8 qop, const float* lds_b2, int G) {
  float m = TA_NEG_INF;
#pragma unroll
  for (int kg = 0; kg < NG; ++kg) {
    const bool half = HALF && kg == NG - 1;
    f32x4 x0, x1;
    rs_scores<MF>(ka[kg][0], ka[kg][1], qop, lds_b2, kg, G, x0, x1, half);
#pragma unroll
    for (int r = 0; r < 4; ++r) m = fmaxf(m, half ? x0[r] : fmaxf(x0[r], x1[r]));
  }
  return quad_max(m);
}

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// RoPE of this lane's 4 dims of q (d4..d4+3, `own`; rs_rope_q takes them from the raw 8 dims qr of its
// k-slots, the lane's 4 at positions 4 (G >> 1)) and the prefetched cos / sin of those 4 dims, for the
// two full-width forms
// (rot = 16) this kernel takes: pairs in-lane; halves with the partner dims d4 ^ 8 from lane l ^ 16,
// whose qr holds the other 8 dims of the head at the same positions (v_permlane16_swap).
// y = fma(x, cos, partner sin): RF = 0 takes the form from p.rope and signs the partner (pairs: -x[d+1]
// on even dims, +x[d-1] on odd; halves: -x[d+8] on dims 0..7, +x[d-8] on 8..15); RF = 1 (pairs) / 2
// (halves) take tables whose sin already carries that sign (the same products exactly).
template <int RF = 0>
__device__ __forceinline__ f32x4 rs_rope_own(const ShParams& p, bf16x4 own, f32x4 cs, f32x4 sn, int G) {
  typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
  f32x4 y;
  if (RF == 1 || (RF == 0 && p.rope == 1)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float xp = (float)own[r ^ 1];
      y[r] = __builtin_fmaf((float)own[r], cs[r], (RF != 0 || (r & 1) ? xp : -xp) * sn[r]);
    }
  } else {
    const u32x2v ow = __builtin_bit_cast(u32x2v, own);
    u32x2v pw;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const auto r = __builtin_amdgcn_permlane16_swap(ow[k], ow[k], false, false);
      pw[k] = (G & 1) ? r[0] : r[1];
    }
    const bf16x4 pt = __builtin_bit_cast(bf16x4, pw);
    const float sg = (RF != 0 || (G & 1)) ? 1.f : -1.f;  // dims 8..15 of the head: +x[jd - 8]; 0..7: -x[jd + 8]
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = __builtin_fmaf((float)own[r], cs[r], sg * (float)pt[r] * sn[r]);
  }
  return y;
}

// The lane's own 4 dims of its 8 k-slot dims qr.
__device__ __forceinline__ bf16x4 rs_own4(bf16x8 qr, int G) {
  typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
  typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
  const u32x4v w = __builtin_bit_cast(u32x4v, qr);
  const bool upper = (G >> 1) != 0;
  const u32x2v ow = {upper ? w[2] : w[0], upper ? w[3] : w[1]};
  return __builtin_bit_cast(bf16x4, ow);
}

template <int RF = 0>
__device__ __forceinline__ f32x4 rs_rope_q(const ShParams& p, bf16x8 qr, f32x4 cs, f32x4 sn, int G) {
  return rs_rope_own<RF>(p, rs_own4(qr, G), cs, sn, G);
}

// q' log2e operand for scales that are not folded into K (or short runs): q' = bf16(rope(q) scale)
// rounded here from the raw q (with RoPE: this block's cos / sin of the lane's 4 dims), split over
// the two k-halves. FOLD (a power-of-two scale): bf16(rope(q)) (pairs rounded together) times
// scale log2e, the same operand with one multiply per value less.
template <bool ROPE, int RF = 0, bool FOLD = false>
__device__ __forceinline__ bf16x8 rs_qop_split(const ShParams& p, bf16x8 qr, f32x4 cs, f32x4 sn, int G) {
  f32x4 y;
  if constexpr (!ROPE) {
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = (float)qr[(G >> 1) * 4 + j];
  } else {
    y = rs_rope_q<RF>(p, qr, cs, sn, G);
  }
  f32x4 v;
  if constexpr (FOLD) {
    if constexpr (ROPE) {
      const bf16x4 yb = cvt_bf16x4(y);  // raw q needs no rounding
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = (float)yb[j];
    }
    return rs_qsplit(y, p.qc, G);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (float)(bf16)(y[j] * p.scale);
    return rs_qsplit(v, TA_LOG2E, G);
  }
}

// The folded q' log2e operand from the lane's q dims (a power-of-two scale; sin tables signed, RF 1
// or 2): bf16(rope(q)) (pairs of values rounded together; raw q needs no rounding) times scale log2e,
// split.
// Halves form: the partner dims d4 ^ 8 are the own dims of lane l ^ 16, taken with ds_swizzle (xor 16
// within each 32 lanes; the LDS crossbar, no VALU).
template <int RF>
__device__ __forceinline__ bf16x8 rs_qop_own(const ShParams& p, bf16x4 q, f32x4 cs, f32x4 sn, int G) {
  f32x4 y;
  if constexpr (RF == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = (float)q[j];
  } else {
    f32x4 r;
    if constexpr (RF == 1) {
      r = rs_rope_own<1>(p, q, cs, sn, G);
    } else {
      typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
      const u32x2v ow = __builtin_bit_cast(u32x2v, q);
      u32x2v pw;
#pragma unroll
      for (int k = 0; k < 2; ++k) pw[k] = (unsigned)__builtin_amdgcn_ds_swizzle((int)ow[k], 0x401F);
      const bf16x4 pt = __builtin_bit_cast(bf16x4, pw);
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = __builtin_fmaf((float)q[j], cs[j], (float)pt[j] * sn[j]);
    }
    const bf16x4 yb = cvt_bf16x4(r);
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = (float)yb[j];
  }
  return rs_qsplit(y, p.qc, G);
}

// The sweep of one 16-query block over all keys from its q' operand, the exact-maximum recompute
// when l is out of range, and the normalised output (this lane's 4 dims, bf16).
template <int NG, int MF, bool HALF>
__device__ __forceinline__ u32x2 rs_finish(const bf16x8 (&ka)[NG][2], const bf16x8 (&va)[NG], bf16x8 ones,
                                          const float* lds_b2, bf16x8 qop, int G) {
  f32x4 o;
  float l;
  rs_unit<NG, MF, false, HALF>(ka, va, ones, qop, lds_b2, G, 0.f, o, l);
  if (wave_any(!(l >= RS_L_LO && l <= RS_L_HI))) {
    // rare: recompute with the exact maximum subtracted (queries in range keep theirs)
    const float mx = rs_max<NG, MF, HALF>(ka, qop, lds_b2, G);
    const float sub = (l >= RS_L_LO && l <= RS_L_HI) || !(mx > TA_NEG_INF) ? 0.f : mx;
    rs_unit<NG, MF, true, HALF>(ka, va, ones, qop, lds_b2, G, sub, o, l);
  }
  const float inv = l == 0.f ? 0.f : __builtin_amdgcn_rcpf(l);
  bf16x4 ov;
#pragma unroll
  for (int r = 0; r < 4; ++r) ov[r] = (bf16)(o[r] * inv);
  return __builtin_bit_cast(u32x2, ov);
}

// One 16-query block of head g: q' operand from the raw q (and, with RoPE, its prefetched cos / sin),
// one sweep over all keys, the exact-maximum recompute when l is out of range; returns the
// normalised output (this lane's 4 dims, bf16).
// With RoPE, cs / sn hold this block's cos / sin on entry and the next block's (table byte offset
// cnext) on return: reloaded as soon as the q' operand is built, a block of work ahead of their use.
template <int NG, int MF, bool ROPE, bool EXACT, bool HALF>
__device__ __forceinline__ u32x2 rs_block(const ShParams& p, const bf16x8 (&ka)[NG][2], const bf16x8 (&va)[NG],
                                         bf16x8 ones, const float* lds_b2, bf16x8 qr, f32x4& cs, f32x4& sn,
                                         __amdgpu_buffer_rsrc_t crsrc, __amdgpu_buffer_rsrc_t srsrc, int cnext, int G) {
  bf16x8 qop;
  if (EXACT && !ROPE) {
    qop = qr;  // q' = q scale exactly: scale and log2e ride on the K operand
  } else if (EXACT) {
    const f32x4 y = rs_rope_q(p, qr, cs, sn, G);
    bf16x4 y4;
#pragma unroll
    for (int j = 0; j < 4; ++j) y4[j] = (bf16)y[j];  // bf16(rope(q) scale) = bf16(rope(q)) scale
    qop = rs_pair8(y4, G);
  } else {
    qop = rs_qop_split<ROPE>(p, qr, cs, sn, G);
  }
  if constexpr (ROPE) {
    cs = rs_tab(crsrc, cnext);
    sn = rs_tab(srsrc, cnext);
  }
  return rs_finish<NG, MF, HALF>(ka, va, ones, lds_b2, qop, G);
}

// Every lane stores (the buffer range check drops rows past Lq): an unconditional store keeps the
// compiler's count of pending memory operations exact, so the waits for q stay partial.
__device__ __forceinline__ void rs_store(__amdgpu_buffer_rsrc_t orsrc, u32x2 ov, int off) {
  __builtin_amdgcn_raw_buffer_store_b64(ov, orsrc, off, 0, 0);
}

// NG = 32-key groups swept (ceil(Lk / 32)); b2 is read from LDS for groups kg >= MF only; ROPE:
// q and k take the rotary embedding; EXACT: the scale is a power of two (scale and log2e folded
// into the K operand, raw q as the B operand).
template <int NG, int MF, bool ROPE, bool EXACT, bool HALF = false>
__global__ __launch_bounds__(SH_H * 64, 4) void sh_resident_kernel(ShParams p) {
  constexpr int NT = SH_H * 64;
  __shared__ __attribute__((aligned(16))) bf16 lds_k[RS_LK * RS_KSTR];
  __shared__ __attribute__((aligned(16))) bf16 lds_v[RS_LK * RS_VSTR];
  __shared__ __attribute__((aligned(16))) float lds_b2[RS_LK];

  // Work order. Ragged calls (per-element row counts): run-major (all batch elements' first runs,
  // then their second runs, ...) in the hardware's dispatch order. Their runs differ in work (any
  // run past an element's rows is empty), and interleaving them element by element (or by
  // XCD-contiguous ranges of elements) left part of the CUs with the heavy runs: measured on the
  // 2k-row ISAB-2 shape with every element's rows cut to its first run, 3.41 ms element-major
  // against 2.04 ms run-major (4.11 ms uncut); C5's ragged ISAB-2 leg 44.3 -> 36.3 ms.
  // Dense calls: element-major in XCD-contiguous ranges, so an element's runs share its K / V
  // through one XCD's L2 (run-major spread them over the XCDs: C3 ISAB-2 read its 64 KB of K / V
  // once per run from HBM, 2.5 GB more traffic, 1.13x the algorithmic bytes).
  int b, qb0;
  if (p.qlen) {
    b = blockIdx.x % p.B;
    qb0 = (blockIdx.x / p.B) * p.qbpw;
  } else {
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    b = work / p.nwg_b;
    qb0 = (work % p.nwg_b) * p.qbpw;
  }
  int lk = p.Lk;
  if (p.valid) {
    const int vl = p.valid[p.valid_n == 1 ? 0 : b];
    lk = vl < 0 ? 0 : (vl < lk ? vl : lk);
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = tid >> 6;
  const int l16 = lane & 15, G = lane >> 4;

  // live query rows: the rows at or past `live` are neither computed nor written
  int live = p.Lq;
  if (p.qlen) {
    const int r = p.qlen[p.qlen_n == 1 ? 0 : b];
    live = r < 0 ? 0 : (r < live ? r : live);
  }
  const int orow = qb0 * 16;
  if (live <= orow) return;  // uniform over the workgroup: before the fill and its barrier

  // fill: K rows with RoPE (fp32 math, cast), V rows as they are, b2 per key; keys past lk (up to
  // NG 32-key groups) get zero K/V (the buffer loads' range check) and b2 = -inf. Thread units: whole
  // 16-dim head rows of K (the RoPE partner dims in registers) and 16-byte chunks of V; every load of
  // the fill is issued before the first LDS store.
  {
    constexpr int NK = NG * 32;
    constexpr int KU = (NK * SH_H + NT - 1) / NT;  // K head rows per thread
    constexpr int VU = (NK * 16 + NT - 1) / NT;    // V chunks per thread
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.k + b * p.k_sb, 0, lk * (int)p.k_sr * 2, TA_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.v + b * p.v_sb, 0, lk * (int)p.v_sr * 2, TA_BUF_WORD3);
    __amdgpu_buffer_rsrc_t crs, srs;
    if constexpr (ROPE) {
      crs = __builtin_amdgcn_make_buffer_rsrc((float*)p.ck, 0, lk * p.tab_sr * 4, TA_BUF_WORD3);
      srs = __builtin_amdgcn_make_buffer_rsrc((float*)p.sk, 0, lk * p.tab_sr * 4, TA_BUF_WORD3);
    }
    typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
    u32x4v kx[KU][2], vx[VU];
    f32x4 kc[KU][4], ks[KU][4];
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      const int u = tid + j * NT, key = u >> 3, hh = u & 7;  // key row, head
      const int off = (key * (int)p.k_sr + hh * SH_D) * 2;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) kx[j][h2] = __builtin_amdgcn_raw_buffer_load_b128(krs, off + 16 * h2, 0, 0);
      if constexpr (ROPE) {
        const int toff = (key * p.tab_sr + ((hh * SH_D) & p.tab_cm)) * 4;
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          kc[j][c4] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(crs, toff + 16 * c4, 0, 0));
          ks[j][c4] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, toff + 16 * c4, 0, 0));
        }
      }
    }
#pragma unroll
    for (int j = 0; j < VU; ++j) {
      const int u = tid + j * NT, key = u >> 4, c8 = (u & 15) * 8;
      vx[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (key * (int)p.v_sr + c8) * 2, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      const int u = tid + j * NT, key = u >> 3, hh = u & 7;
      if (u < NK * SH_H) {  // uniform per wave
        if constexpr (ROPE) {
          const bf16x8 lo = __builtin_bit_cast(bf16x8, kx[j][0]), hi = __builtin_bit_cast(bf16x8, kx[j][1]);
          float x[SH_D], y[SH_D];
#pragma unroll
          for (int d = 0; d < 8; ++d) {
            x[d] = (float)lo[d];
            x[8 + d] = (float)hi[d];
          }
#pragma unroll
          for (int d = 0; d < SH_D; ++d) {
            // full-width forms only (the launcher sends others to smallhead_fwd_kernel)
            const float xp = p.rope == 1 ? ((d & 1) ? x[d - 1] : -x[d + 1]) : (d < 8 ? -x[d + 8] : x[d - 8]);
            y[d] = rs_rot(x[d], xp, kc[j][d >> 2][d & 3], ks[j][d >> 2][d & 3]);
          }
          bf16x8 o0, o1;
#pragma unroll
          for (int d = 0; d < 8; ++d) {
            o0[d] = (bf16)y[d];
            o1[d] = (bf16)y[8 + d];
          }
          *(bf16x8*)(lds_k + key * RS_KSTR + hh * SH_D) = o0;
          *(bf16x8*)(lds_k + key * RS_KSTR + hh * SH_D + 8) = o1;
        } else {
          *(u32x4v*)(lds_k + key * RS_KSTR + hh * SH_D) = kx[j][0];
          *(u32x4v*)(lds_k + key * RS_KSTR + hh * SH_D + 8) = kx[j][1];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < VU; ++j) {
      const int u = tid + j * NT, key = u >> 4, c8 = (u & 15) * 8;
      if (u < NK * 16) *(u32x4v*)(lds_v + key * RS_VSTR + c8) = vx[j];
    }
    for (int j = tid; j < NK; j += NT) {
      float b2 = TA_NEG_INF;
      if (j < lk) b2 = p.bias ? fmaxf(p.bias[b * p.bias_sb + j] * TA_LOG2E, SH_BIAS_FLOOR) : 0.f;
      lds_b2[j] = b2;
    }
  }
  __syncthreads();

  // wave g owns head g: its K operands (the 16 dims twice, for the high and remainder halves of q)
  // and V^T operands stay in registers for the whole query range
  const int kcol = g * SH_D + 8 * (G & 1);
  // transposed-read lane roles: lane 4j + c of group G points at key 4G + j, dims 4c..4c+3
  const int tr_key = 4 * G + (l16 >> 2), tr_col = 4 * (l16 & 3);
  bf16x8 ka[NG][2], va[NG];
#pragma unroll
  for (int kg = 0; kg < NG; ++kg) {
    ka[kg][0] = *(const bf16x8*)(lds_k + (32 * kg + l16) * RS_KSTR + kcol);
    ka[kg][1] = *(const bf16x8*)(lds_k + (32 * kg + 16 + l16) * RS_KSTR + kcol);
    if (EXACT) {
      ka[kg][0] = rs_ksplit(ka[kg][0], p.scale * TA_LOG2E, G);
      ka[kg][1] = rs_ksplit(ka[kg][1], p.scale * TA_LOG2E, G);
    }
    const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(lds_v + (32 * kg + tr_key) * RS_VSTR + g * SH_D + tr_col));
    const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(lds_v + (32 * kg + 16 + tr_key) * RS_VSTR + g * SH_D + tr_col));
    const bf16x4 a0 = __builtin_bit_cast(bf16x4, t0), a1 = __builtin_bit_cast(bf16x4, t1);
    va[kg] = bf16x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
  }

  const bf16* qbase = (const bf16*)p.q + b * p.q_sb;
  // 16-query blocks of this workgroup that hold a live row
  const int nb = (live - orow + 15) / 16 < p.qbpw ? (live - orow + 15) / 16 : p.qbpw;
  // live output rows orow .. orow + nrow - 1 as a buffer resource (byte offsets, range checked: the
  // stores of rows past them are dropped by the hardware)
  const int nrow = nb * 16 < live - orow ? nb * 16 : live - orow;
  const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
      (bf16*)p.o + b * p.o_sb + (int64_t)orow * p.o_sr, 0, nrow * p.o_sr * 2, TA_BUF_WORD3);
  const int ooff = (l16 * p.o_sr + g * SH_D + 4 * G) * 2, ostep = 16 * p.o_sr * 2;
  const int d4 = kcol + 4 * (G >> 1);  // this lane's 4 dims of q
  // q rows orow .. orow + nrow - 1 likewise; two q buffers, each loaded two blocks ahead of its use
  const __amdgpu_buffer_rsrc_t qrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (bf16*)qbase + (int64_t)orow * p.q_sr, 0, nrow * p.q_sr * 2, TA_BUF_WORD3);
  const int qoff = (l16 * p.q_sr + kcol) * 2, qstep = 16 * p.q_sr * 2;
  // the ones operand of the row-sum MFMA, kept in registers (not rebuilt per key group)
  bf16x8 ones = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f};
  asm volatile("" : "+v"(ones));
  // q loads are issued before the previous block's store and waited for one block later, and the
  // loop is entered with the pending memory operations in the order of its back edge (q, store, q,
  // store): each wait for q then leaves the younger stores and q loads in flight. The two zero
  // stores go to blocks 0 and 1, which their units rewrite later, in order, from this wave (block 1
  // lies outside the resource when the run has one block, and that store is dropped).
  // RoPE: cos / sin of the lane's 4 dims at its query's position (tables [Lq][E] fp32; rows past Lq
  // read as zero), one buffer refilled inside each block for the next one
  __amdgpu_buffer_rsrc_t crsrc, srsrc;
  const int coff = (l16 * p.tab_sr + (d4 & p.tab_cm)) * 4, cstep = 16 * p.tab_sr * 4;
  f32x4 cs = {0.f, 0.f, 0.f, 0.f}, sn = cs;
  if constexpr (ROPE) {
    crsrc = __builtin_amdgcn_make_buffer_rsrc((float*)p.cq + (int64_t)orow * p.tab_sr, 0, nrow * p.tab_sr * 4,
                                              TA_BUF_WORD3);
    srsrc = __builtin_amdgcn_make_buffer_rsrc((float*)p.sq + (int64_t)orow * p.tab_sr, 0, nrow * p.tab_sr * 4,
                                              TA_BUF_WORD3);
    cs = rs_tab(crsrc, coff);
    sn = rs_tab(srsrc, coff);
  }
  bf16x8 qa = rs_qraw(qrsrc, qoff);
  rs_store(orsrc, u32x2{0u, 0u}, ooff);
  bf16x8 qb = rs_qraw(qrsrc, qoff + qstep);
  rs_store(orsrc, u32x2{0u, 0u}, ooff + ostep);
  int i = 0;
#pragma unroll 1
  for (; i + 1 < nb; i += 2) {
    u32x2 ov = rs_block<NG, MF, ROPE, EXACT, HALF>(p, ka, va, ones, lds_b2, qa, cs, sn, crsrc, srsrc,
                                              coff + (i + 1) * cstep, G);
    qa = rs_qraw(qrsrc, qoff + (i + 2) * qstep);
    rs_store(orsrc, ov, ooff + i * ostep);
    ov = rs_block<NG, MF, ROPE, EXACT, HALF>(p, ka, va, ones, lds_b2, qb, cs, sn, crsrc, srsrc,
                                       coff + (i + 2) * cstep, G);
    qb = rs_qraw(qrsrc, qoff + (i + 3) * qstep);
    rs_store(orsrc, ov, ooff + (i + 1) * ostep);
  }
  if (i < nb)
    rs_store(orsrc,
             rs_block<NG, MF, ROPE, EXACT, HALF>(p, ka, va, ones, lds_b2, qa, cs, sn, crsrc, srsrc,
                                           coff + (i + 1) * cstep, G),
             ooff + i * ostep);
}

// ---------------------------------------------------------------------------------------------
// Persistent resident-keys kernel (bf16, 97..112 keys: four 32-key groups, the last one half; NB = 1
// or 7 query blocks per batch element; no per-batch row counts; RoPE only from the shared one-head
// tables): the row stage's 104-token self attention and the CLS cross attention over many batch
// elements. The one-element-per-workgroup
// kernel above waits for every element's K / V fill before it computes; here each workgroup stays
// resident (two per CU) and walks the batch elements blockIdx.x, + gridDim.x, ...: the load unit
// copies the next element's K and V rows global -> LDS (global_load_lds_dwordx4, no registers)
// while the current element is computed from the register operands, which were read from LDS
// before the copies were issued. Per element:
//   wait for its copies, b2 into one of two LDS rows, barrier; with RoPE, rotate its K rows in LDS
//   (tables staged once per workgroup), barrier; read head g's K and V^T operands; barrier; issue
//   the next element's copies; then the same per-block sweep as the kernel above.
// LDS (dynamic): K and V rows of 256 bytes with 16-byte chunks XOR-swizzled per row (K: by r & 7,
// for the b128 operand reads of 8 rows; V: by 2 (r & 3), for the transposed reads of 4 rows x 2
// chunks), b2 [2][NK], then the tables (16 cos + 16 sin floats per key row, and per query row when
// the q tables are other tensors). Rows past the valid length are copied from the last valid row (so
// they hold finite values) and masked by b2 = -inf; an element without valid keys writes zeros.
// q comes by buffer loads two blocks ahead along the workgroup's stream of (element, block)
// pairs, so the first two blocks of an element are loaded during the previous one.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int rp_kchunk(int r, int c) { return r * 16 + (c ^ (r & 7)); }
__device__ __forceinline__ int rp_vchunk(int r, int c) { return r * 16 + (c ^ ((r & 3) << 1)); }

// LDS bytes of the persistent kernel for NK key rows (the tables only with RoPE).
// Chunk c (0..7) of a staged table row: c < 4 cos of dims 4c..4c+3, else sin of dims 4(c-4)..; the
// sin values carry the sign of the rotation's partner term for form RF (1 pairs, 2 halves).
template <int RF>
__device__ __forceinline__ f32x4 rp_sign_tab(f32x4 t, int c) {
  if (c >= 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 4 * (c - 4) + j;
      if (RF == 1 ? (d & 1) == 0 : d < 8) t[j] = -t[j];
    }
  }
  return t;
}

__host__ __device__ inline int rp_lds_bytes(int NK, bool rope, int Lk, int Lq, bool qsep) {
  return 2 * NK * 256 + 2 * NK * 4 + (rope ? 128 * (Lk + (qsep ? Lq : 0)) : 0);
}

template <int NG, int MF, int RF, bool HALF, int NB>
__global__ __launch_bounds__(SH_H * 64, 4) void sh_persist_kernel(ShParams p) {
  constexpr int NT = SH_H * 64;
  constexpr int NK = NG * 32;
  constexpr bool ROPE = RF != 0;
  extern __shared__ __attribute__((aligned(16))) unsigned char rp_lds[];
  bf16* const lds_k = (bf16*)rp_lds;
  bf16* const lds_v = (bf16*)(rp_lds + NK * 256);
  float* const lds_b2 = (float*)(rp_lds + 2 * NK * 256);
  float* const lds_tk = lds_b2 + 2 * NK;
  float* const lds_tq = p.rp_qsep ? lds_tk + 32 * p.Lk : lds_tk;

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = tid >> 6;
  const int l16 = lane & 15, G = lane >> 4;
  const int stride = gridDim.x;
  const int nitems = (p.B - (int)blockIdx.x + stride - 1) / stride;  // >= 1 (grid <= B)
  constexpr int nb = NB;  // query blocks per element (p.nqb)

  // valid keys of element bb: a scalar load (the lengths do not change while the kernel runs), so
  // that no wait for it also waits for the copies in flight
  auto klen = [&](int bb) {
    int lk = p.Lk;
    if (p.valid) {
      const int vl = ((const __attribute__((address_space(4))) int32_t*)p.valid)[p.valid_n == 1 ? 0 : bb];
      lk = vl < 0 ? 0 : (vl < lk ? vl : lk);
    }
    return lk;
  };
  // the copies of element bb's NK K and V rows (rows >= lk from row lk - 1; lk >= 1): wave g copies
  // the 4-row slabs g, g + 8, ...; lane: row 4 slab + lane / 16, LDS chunk lane % 16
  auto issue = [&](int bb, int lk) {
    const bf16* kb = (const bf16*)p.k + (int64_t)bb * p.k_sb;
    const bf16* vb = (const bf16*)p.v + (int64_t)bb * p.v_sb;
#pragma unroll
    for (int s4 = 0; s4 < NG; ++s4) {
      const int slab = g + 8 * s4, r = 4 * slab + (lane >> 4), pos = lane & 15;
      const int rs = r < lk ? r : lk - 1;
      lds_dma16_s((uint32_t)((rs * (int)p.k_sr + 8 * (pos ^ (r & 7))) * 2), kb, lds_addr(lds_k) + slab * 1024);
      lds_dma16_s((uint32_t)((rs * (int)p.v_sr + 8 * (pos ^ ((r & 3) << 1))) * 2), vb,
                  lds_addr(lds_v) + slab * 1024);
    }
  };
  // this thread's key bias of element bb (threads < NK; keys past Lk read as zero through the
  // buffer range check), loaded ahead of the element
  auto bias_raw = [&](int bb) -> float {
    if (!p.bias) return 0.f;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (float*)p.bias + (int64_t)bb * p.bias_sb, 0, p.Lk * 4, TA_BUF_WORD3);
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (tid & (NK - 1)) * 4, 0, 0));
  };
  const int kcol = g * SH_D + 8 * (G & 1);
  const int d4 = kcol + 4 * (G >> 1);
  const int qoff = (l16 * (int)p.q_sr + d4) * 2, qstep = 16 * (int)p.q_sr * 2;
  const int ooff = (l16 * (int)p.o_sr + g * SH_D + 4 * G) * 2, ostep = 16 * (int)p.o_sr * 2;
  // the lane's own 4 dims of q in block m of the workgroup's element it (the callers' it and m are
  // compile-time offsets from the current element, so the resource is shared by its blocks); past
  // the last element the resource is empty and the load reads zeros
  auto qload = [&](int it, int m) {
    const int bb = (int)blockIdx.x + it * stride;
    const int rows = it < nitems ? p.Lq : 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (bf16*)p.q + (int64_t)(it < nitems ? bb : 0) * p.q_sb, 0, rows * (int)p.q_sr * 2, TA_BUF_WORD3);
    int so = m * qstep;
    asm volatile("" : "+s"(so));  // formed at the load, not hoisted into a register per block
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rs, qoff + so, 0, 0));
  };

  int b = blockIdx.x;
  int lk = klen(b);
  if (lk > 0) issue(b, lk);
  if constexpr (ROPE) {
    // tables of the key rows (and of the query rows when they are other tensors), once per workgroup
    // the sin columns take the sign of the partner term (pairs: - on even dims; halves: - on dims
    // 0..7), so that the rotations multiply the unsigned partner (the same products exactly)
    for (int u = tid; u < 8 * p.Lk; u += NT) {
      const int r = u >> 3, c = u & 7;
      const float* src = (c < 4 ? p.ck : p.sk) + (int64_t)r * p.tab_sr + 4 * (c & 3);
      *(f32x4*)(lds_tk + 32 * r + 4 * c) = rp_sign_tab<RF>(*(const f32x4*)src, c);
    }
    if (p.rp_qsep) {
      for (int u = tid; u < 8 * p.Lq; u += NT) {
        const int r = u >> 3, c = u & 7;
        const float* src = (c < 4 ? p.cq : p.sq) + (int64_t)r * p.tab_sr + 4 * (c & 3);
        *(f32x4*)(lds_tq + 32 * r + 4 * c) = rp_sign_tab<RF>(*(const f32x4*)src, c);
      }
    }
  }
  float braw = bias_raw(b);
  bf16x4 qa = qload(0, 0), qb = NB >= 2 ? qload(0, 1) : qload(1, 0);
  __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc((bf16*)p.o + (int64_t)b * p.o_sb, 0,
                                                                 p.Lq * (int)p.o_sr * 2, TA_BUF_WORD3);
  // a zero store to the first element's block 0 (which this wave rewrites later, in order): the
  // element loop is then entered with the pending memory operations of its back edge (q, q, store)
  rs_store(ors, u32x2{0u, 0u}, ooff);
  bf16x8 ones = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f};
  asm volatile("" : "+v"(ones));
  const int tr_key = 4 * G + (l16 >> 2);
  const int tr_c = 2 * g + ((l16 & 3) >> 1), tr_e = 4 * (l16 & 1);
  bf16x8 ka[NG][2], va[NG];
  int b2off = 0;  // the element's b2 row: lds_b2 + b2off

  // Element set-up: its copies have landed (first element: everything; later ones: the copies are
  // older than the previous element's last q load and output store, so all but the two youngest
  // memory operations), b2, RoPE on K, operands, then the next element's copies.
  auto setup = [&](int it, bf16x4& q0, bf16x4& q1) {
    if (it == 0)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    float* b2 = lds_b2 + (it & 1) * NK;
    if (tid < NK)
      b2[tid] = tid < lk ? (p.bias ? fmaxf(braw * TA_LOG2E, SH_BIAS_FLOOR) : 0.f) : TA_NEG_INF;
    b2off = (it & 1) * NK;
    TA_JOIN_LDS();
    if constexpr (ROPE) {
      for (int u = tid; u < lk * SH_H; u += NT) {
        const int r = u >> 3, hh = u & 7;
        bf16x8* c0 = (bf16x8*)lds_k + rp_kchunk(r, 2 * hh);
        bf16x8* c1 = (bf16x8*)lds_k + rp_kchunk(r, 2 * hh + 1);
        const bf16x8 lo = *c0, hi = *c1;
        const float* tc = lds_tk + 32 * r;
        float x[SH_D], y[SH_D];
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          x[d] = (float)lo[d];
          x[8 + d] = (float)hi[d];
        }
#pragma unroll
        for (int d = 0; d < SH_D; ++d) {
          const float xp = RF == 1 ? ((d & 1) ? x[d - 1] : x[d + 1]) : (d < 8 ? x[d + 8] : x[d - 8]);
          y[d] = rs_rot(x[d], xp, tc[d], tc[16 + d]);  // signed sin
        }
        bf16x8 o0, o1;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          o0[d] = (bf16)y[d];
          o1[d] = (bf16)y[8 + d];
        }
        *c0 = o0;
        *c1 = o1;
      }
      TA_JOIN_LDS();
    }
#pragma unroll
    for (int kg = 0; kg < NG; ++kg) {
      ka[kg][0] = *((const bf16x8*)lds_k + rp_kchunk(32 * kg + l16, 2 * g + (G & 1)));
      ka[kg][1] = *((const bf16x8*)lds_k + rp_kchunk(32 * kg + 16 + l16, 2 * g + (G & 1)));
      const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(lds_v + 8 * rp_vchunk(32 * kg + tr_key, tr_c) + tr_e));
      const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(lds_v + 8 * rp_vchunk(32 * kg + 16 + tr_key, tr_c) + tr_e));
      const bf16x4 a0 = __builtin_bit_cast(bf16x4, t0), a1 = __builtin_bit_cast(bf16x4, t1);
      va[kg] = bf16x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    }
    ors = __builtin_amdgcn_make_buffer_rsrc((bf16*)p.o + (int64_t)b * p.o_sb, 0, p.Lq * (int)p.o_sr * 2,
                                            TA_BUF_WORD3);
    // the element's first two q blocks (one with a single block per element) were loaded during the
    // previous ones: waited for here, before the next copies are issued (a wait after them would also
    // wait for the copies)
    if constexpr (NB >= 2)
      asm volatile("" : "+v"(q0), "+v"(q1));
    else
      asm volatile("" : "+v"(q0));
    TA_JOIN_LDS();  // every wave holds its operands: the K / V rows may be overwritten
    const int bn = b + stride;
    if (bn < p.B) {
      const int lkn = klen(bn);
      if (lkn > 0) issue(bn, lkn);
      braw = bias_raw(bn);
    }
  };

  // one block of the stream: q' operand (RoPE tables from LDS), sweep, store
  auto block = [&](bf16x4 qr, int m) -> u32x2 {
    if (lk == 0) return u32x2{0u, 0u};
    f32x4 cs = {0.f, 0.f, 0.f, 0.f}, sn = cs;
    if constexpr (ROPE) {
      const int row = 16 * m + l16 < p.Lq ? 16 * m + l16 : p.Lq - 1;
      cs = *(const f32x4*)(lds_tq + 32 * row + (d4 & 15));
      sn = *(const f32x4*)(lds_tq + 32 * row + 16 + (d4 & 15));
    }
    const bf16x8 qop = rs_qop_own<RF>(p, qr, cs, sn, G);
    // b2 is read inside each block, not hoisted over the element's blocks (registers)
    int bo = b2off;
    asm volatile("" : "+s"(bo));
    return rs_finish<NG, MF, HALF>(ka, va, ones, lds_b2 + bo, qop, G);
  };

  // One element: set-up, then its blocks, each computing with q0 / q1 alternately and loading the
  // block two ahead into the same register. After an odd block count the next element's block 0 is in
  // q1 and block 1 in q0, so elements alternate the roles of qa and qb (no register moves).
  auto element = [&](int it, bf16x4& q0, bf16x4& q1) {
    setup(it, q0, q1);
#pragma unroll
    for (int m = 0; m < NB; ++m) {
      bf16x4& qr = (m & 1) ? q1 : q0;
      const u32x2 ov = block(qr, m);
      qr = qload(it + (m + 2) / NB, (m + 2) % NB);
      int so = m * ostep;
      asm volatile("" : "+s"(so));
      rs_store(ors, ov, ooff + so);
    }
  };
  auto next = [&]() {
    b += stride;
    lk = klen(b);
  };
#pragma unroll 1
  for (int it = 0;; it += 2) {
    element(it, qa, qb);
    if (it + 1 == nitems) break;
    next();
    if constexpr (NB & 1)
      element(it + 1, qb, qa);
    else
      element(it + 1, qa, qb);
    if (it + 2 == nitems) break;
    next();
  }
}

// mode 0: b2 read for every group (key bias or per-batch valid lengths); 1: last group only (Lk not
// a multiple of 32); 2: none.
template <int NG, bool ROPE, bool EXACT>
void launch_resident_mode(const ShParams& p, int mode, int64_t nblk, hipStream_t stream) {
  const dim3 grid((unsigned)nblk), block(SH_H * 64);
  if constexpr (NG == 4) {
    // the row stage's 104 keys: the last group's upper half holds no key
    if (p.half_last && mode == 0) {
      hipLaunchKernelGGL((sh_resident_kernel<NG, 0, ROPE, EXACT, true>), grid, block, 0, stream, p);
      return;
    }
    if (p.half_last && mode == 1) {
      hipLaunchKernelGGL((sh_resident_kernel<NG, NG - 1, ROPE, EXACT, true>), grid, block, 0, stream, p);
      return;
    }
  }
  if (mode == 0)
    hipLaunchKernelGGL((sh_resident_kernel<NG, 0, ROPE, EXACT>), grid, block, 0, stream, p);
  else if (mode == 1)
    hipLaunchKernelGGL((sh_resident_kernel<NG, NG - 1, ROPE, EXACT>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((sh_resident_kernel<NG, NG, ROPE, EXACT>), grid, block, 0, stream, p);
}

// The K split (EXACT) serves RoPE-free long runs; with RoPE, and for three key groups (whose K-split
// build needs more than 128 VGPRs), q carries the split.
template <int NG, bool ROPE>
void launch_resident_ng(const ShParams& p, int mode, int64_t nblk, hipStream_t stream) {
  if constexpr (!ROPE && NG != 3) {
    if (p.exact_scale) {
      launch_resident_mode<NG, false, true>(p, mode, nblk, stream);
      return;
    }
  }
  launch_resident_mode<NG, ROPE, false>(p, mode, nblk, stream);
}

template <bool ROPE>
void launch_resident_rope(const ShParams& p, int ngrp, int mode, int64_t nblk, hipStream_t stream) {
  switch (ngrp) {
    case 1: launch_resident_ng<1, ROPE>(p, mode, nblk, stream); break;
    case 2: launch_resident_ng<2, ROPE>(p, mode, nblk, stream); break;
    case 3: launch_resident_ng<3, ROPE>(p, mode, nblk, stream); break;
    default: launch_resident_ng<4, ROPE>(p, mode, nblk, stream); break;
  }
}

// Compute units of device dev (cached per device; 0 if the query fails).
constexpr int RP_DEV_CACHE = 64;
int rp_cus(int dev) {
  static std::atomic<int> cache[RP_DEV_CACHE];
  if (dev >= 0 && dev < RP_DEV_CACHE) {
    const int hit = cache[dev].load(std::memory_order_relaxed);
    if (hit > 0) return hit;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
  if (dev >= 0 && dev < RP_DEV_CACHE) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// LDS bytes that still let two persistent workgroups share a CU (160 KB of LDS per CU).
constexpr int RP_LDS_MAX = 80 * 1024;

template <int MF, int RF, int NB>
int launch_persist_inst(const ShParams& p, int dev, int nwg, int lds, hipStream_t stream) {
  // the dynamic-LDS limit of this instance, raised once per device
  static std::atomic<bool> raised[RP_DEV_CACHE];
  if (dev >= 0 && dev < RP_DEV_CACHE && !raised[dev].load(std::memory_order_relaxed)) {
    (void)hipFuncSetAttribute((const void*)sh_persist_kernel<4, MF, RF, true, NB>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, RP_LDS_MAX);
    raised[dev].store(true, std::memory_order_relaxed);
  }
  hipLaunchKernelGGL((sh_persist_kernel<4, MF, RF, true, NB>), dim3((unsigned)nwg), dim3(SH_H * 64),
                     (unsigned)lds, stream, p);
  return (int)hipGetLastError();
}

template <int RF, int NB>
int launch_persist_nb(const ShParams& p, int dev, int mode, int nwg, int lds, hipStream_t stream) {
  return mode == 0 ? launch_persist_inst<0, RF, NB>(p, dev, nwg, lds, stream)
                   : launch_persist_inst<3, RF, NB>(p, dev, nwg, lds, stream);
}

template <int NB>
int launch_persist_rf(const ShParams& p, int dev, int mode, int nwg, int lds, hipStream_t stream) {
  switch (p.rope) {
    case 0: return launch_persist_nb<0, NB>(p, dev, mode, nwg, lds, stream);
    case 1: return launch_persist_nb<1, NB>(p, dev, mode, nwg, lds, stream);
    default: return launch_persist_nb<2, NB>(p, dev, mode, nwg, lds, stream);
  }
}

// The persistent kernel for a resident-keys call, or -1 when the call does not suit it (then the
// one-element-per-workgroup kernel runs): 97..112 keys (the row stage's 104 tokens), 1 or 7 query
// blocks per element (CLS queries, the row stage's self attention), no per-batch row counts, the
// shared one-head RoPE tables (q tables equal to the key tables, or staged separately), a
// power-of-two scale (folded into the q' operand's log2e factor), 16-byte aligned K / V rows, LDS for
// two workgroups per CU and at least two elements per workgroup.
int launch_persist(ShParams& p, int ngrp, int mode, hipStream_t stream) {
  if (ngrp != 4 || !p.half_last || mode == 2 || (p.nqb != 1 && p.nqb != 7) || p.qlen != nullptr ||
      p.exact_scale || !p.pow2_scale)
    return -1;
  if (p.rope && p.tab_sr != SH_D) return -1;
  if ((p.k_sr & 7) || (p.v_sr & 7) || ((uintptr_t)p.k & 15) || ((uintptr_t)p.v & 15)) return -1;
  p.rp_qsep = p.rope && !(p.cq == p.ck && p.sq == p.sk && p.Lq <= p.Lk);
  const int lds = rp_lds_bytes(128, p.rope != 0, p.Lk, p.Lq, p.rp_qsep != 0);
  if (lds > RP_LDS_MAX) return -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  const int cus = rp_cus(dev);
  if (cus <= 0) return -1;
  const int nwg = 2 * cus;
  if (p.B < 2 * nwg) return -1;
  return p.nqb == 1 ? launch_persist_rf<1>(p, dev, mode, nwg, lds, stream)
                    : launch_persist_rf<7>(p, dev, mode, nwg, lds, stream);
}

void launch_resident(const ShParams& p, int ngrp, int mode, int64_t nblk, hipStream_t stream) {
  if (p.rope)
    launch_resident_rope<true>(p, ngrp, mode, nblk, stream);
  else
    launch_resident_rope<false>(p, ngrp, mode, nblk, stream);
}

// ---------------------------------------------------------------------------------------------
// fp32 kernel (every fp32 call: the C1 column ISAB in the reference's fp32 precision). A workgroup of
// 8 waves takes (batch element, group of 4 heads, run of 16-query blocks); wave = (head of the group,
// parity of the blocks it takes). Keys go through LDS in tiles of 128 (the group's 64 dims of K
// row-major and of V transposed: 69 KB, two workgroups per CU). Per block and 16-key group, fp32
// MFMA (4 x 16x16x4 per 16x16x16 product):
//   x = K (q' log2e) - m     S^T with the accumulator initialised to -m (m: the softmax reference,
//                            fixed by the block's first 16 keys), plus b2 on masked tiles
//   p = exp2(x), l += p, O^T += V^T P^T
// so the VALU work per score is one v_exp_f32 and one add. A row sum outside [2^-64, 2^96] or a
// non-finite O (a score far above the reference, all keys masked, NaN / inf inputs) sends the block
// (RESIDENT: the wave's blocks, keys still in LDS) or the workgroup (streaming: its keys streamed
// again) through the exact online softmax: x = S log2e + b2 per tile, running maximum rescaled only
// when it grows by more than SH_LAZY.
// RESIDENT (all keys in one tile): each block in one pass, nothing carried between blocks, any run
// length; otherwise up to SF_SB blocks per wave carry (o, m, l) across the tiles.
// ---------------------------------------------------------------------------------------------
constexpr int SF_HG = 4;
constexpr int SF_W = SF_HG * SH_D;   // merged dims per workgroup
constexpr int SF_KT = 128;           // keys per tile
constexpr int SF_KSTR = SF_W + 4;    // K tile row stride (floats)
constexpr int SF_VSTR = SF_KT + 4;   // V^T tile row stride (floats)
constexpr int SF_SB = 2;             // blocks per wave carried across tiles (streaming)

// One tile for one block: online-softmax update of (o, m, l) (l: this lane's partial sum).
__device__ __forceinline__ void sf_tile(const float* lkt, const float* lvt, const float* lb2, int nkb, f32x4 qop,
                                        int hd, int l16, int kap, f32x4& o, float& m, float& l) {
  f32x4 x[SF_KT / 16];
  float tm = TA_NEG_INF;
#pragma unroll
  for (int kt = 0; kt < SF_KT / 16; ++kt) {
    if (kt < nkb) {
      const f32x4 a = *(const f32x4*)(lkt + (16 * kt + l16) * SF_KSTR + hd + 4 * kap);
      x[kt] = mfma16x16x16(a, qop, f32x4{0.f, 0.f, 0.f, 0.f});
      const f32x4 b2 = *(const f32x4*)(lb2 + 16 * kt + 4 * kap);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[kt][r] = fmaf(x[kt][r], TA_LOG2E, b2[r]);
        tm = fmaxf(tm, x[kt][r]);
      }
    }
  }
  const float m_new = fmaxf(m, quad_max(tm));  // finite: every tile holds a valid key
  if (wave_any(m_new - m > SH_LAZY)) {
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    l *= alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] *= alpha;
    m = m_new;
  }
#pragma unroll
  for (int kt = 0; kt < SF_KT / 16; ++kt) {
    if (kt < nkb) {
      f32x4 pv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[r] = __builtin_amdgcn_exp2f(x[kt][r] - m);
        l += pv[r];
      }
      const f32x4 a = *(const f32x4*)(lvt + (hd + l16) * SF_VSTR + 16 * kt + 4 * kap);
      o = mfma16x16x16(a, pv, o);
    }
  }
}

// One tile against a fixed softmax reference m (log2 units; the fast pass): x = K q'' - m comes
// straight from the MFMA (q'' = q' log2e, the accumulator initialised to -m), plus b2 on tiles with
// masked keys (addb), p = exp2(x), l += p, O^T += V^T P^T, one 16-key group at a time (no score
// array). FIRST: the first tile of the sweep, whose first 16 keys set m (their ceiled maximum,
// clamped to [-1e4, 1e4]; -inf and NaN give 0). p may exceed 1; the caller's trust test (l <= 2^96,
// O finite) decides whether the exact pass must redo the block. Even and odd 16-key groups
// accumulate O into separate registers (summed at the end): the PV products of consecutive groups
// do not wait on each other.
// NG: 16-key groups of the tile (8: a 128-key tile; 4: one half of it, the streaming sweep's tiles).
template <bool FIRST, int NG = SF_KT / 16>
__device__ __forceinline__ void sf_tile_fix(const float* lkt, const float* lvt, const float* lb2, int nkb,
                                            f32x4 qop, int hd, int l16, int kap, bool addb, f32x4& o, float& m,
                                            float& l) {
  f32x4 o1 = {0.f, 0.f, 0.f, 0.f};  // odd groups: two independent PV accumulation chains
#pragma unroll
  for (int kt = 0; kt < NG; ++kt) {
    if (kt < nkb) {
      const bool first = FIRST && kt == 0;
      const f32x4 a = *(const f32x4*)(lkt + (16 * kt + l16) * SF_KSTR + hd + 4 * kap);
      const f32x4 init = first ? f32x4{0.f, 0.f, 0.f, 0.f} : f32x4{-m, -m, -m, -m};
      f32x4 x = mfma16x16x16(a, qop, init);
      if (addb) {
        const f32x4 b2 = *(const f32x4*)(lb2 + 16 * kt + 4 * kap);
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] += b2[r];
      }
      if (first) {
        const float tm = quad_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
        m = tm > -1e4f ? fminf(ceilf(tm), 1e4f) : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] -= m;
      }
      f32x4 pv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[r] = __builtin_amdgcn_exp2f(x[r]);
        l += pv[r];
      }
      const f32x4 va = *(const f32x4*)(lvt + (hd + l16) * SF_VSTR + 16 * kt + 4 * kap);
      if (kt & 1)
        o1 = mfma16x16x16(va, pv, o1);
      else
        o = mfma16x16x16(va, pv, o);
    }
    __builtin_amdgcn_sched_barrier(0);  // one 16-key group at a time: hoisted operand reads cost registers
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) o[r] += o1[r];
}

// True when a fast-pass result may not be trusted: the row sum outside [2^-64, 2^96] or not finite,
// or O not finite. Above: a score ~66 nats above the first 16 keys' maximum, or NaN / inf in the
// inputs. Below: the first 16 keys' maximum was clamped (every score far below any finite reference,
// e.g. all keys under a -1e30 bias, whose softmax is uniform) or no key is visible; a trusted row
// has l >= 1/2 from its first 16 keys on.
__device__ __forceinline__ bool sf_suspect(f32x4 o, float l) {
  bool bad = !(l >= 0x1p-64f && l <= 0x1p96f);
#pragma unroll
  for (int r = 0; r < 4; ++r) bad |= !(__builtin_fabsf(o[r]) <= 0x1p127f);
  return bad;
}

// q' = rope(q) scale (fp32) of query qi, this lane's 4 dims d0..d0+3; zero past Lq.
__device__ __forceinline__ f32x4 sf_qop(const ShParams& p, int b, int qi, int d0) {
  if (qi >= p.Lq) return f32x4{0.f, 0.f, 0.f, 0.f};
  const float* row = (const float*)p.q + b * p.q_sb + (int64_t)qi * p.q_sr;
  f32x4 y = p.rope ? rope4<float>(row, p.cq + (int64_t)qi * p.tab_sr, p.sq + (int64_t)qi * p.tab_sr, d0, p.rope,
                                  p.half, p.rot, d0 & p.tab_cm)
                   : *(const f32x4*)(row + d0);
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] *= p.scale;
  return y;
}

__device__ __forceinline__ void sf_store(const ShParams& p, int b, int qi, int d0, f32x4 o, float l) {
  const float lt = quad_sum(l);
  if (qi >= p.Lq) return;
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) out[r] = o[r] * inv;
  *(f32x4*)((float*)p.o + b * p.o_sb + (int64_t)qi * p.o_sr + d0) = out;
}

// Tile t of keys (rows past lk: zero K / V, b2 = -inf); the group's 64 dims, K with RoPE.
__device__ __forceinline__ void sf_fill(const ShParams& p, float* lkt, float* lvt, float* lb2, int b, int hg, int t,
                                        int lk) {
  const int tid = threadIdx.x, k0 = t * SF_KT;
  const float* kbase = (const float*)p.k + b * p.k_sb;
  const float* vbase = (const float*)p.v + b * p.v_sb;
#pragma unroll 2
  for (int i = 0; i < SF_KT * (SF_W / 4) / 512; ++i) {
    const int u = tid + 512 * i, key = u >> 4, c = u & 15, d = hg * SF_W + 4 * c;
    const int gk = k0 + key, gc = gk < lk ? gk : lk - 1;
    const float* krow = kbase + (int64_t)gc * p.k_sr;
    f32x4 kv = p.rope ? rope4<float>(krow, p.ck + (int64_t)gc * p.tab_sr, p.sk + (int64_t)gc * p.tab_sr, d, p.rope,
                                     p.half, p.rot, d & p.tab_cm)
                      : *(const f32x4*)(krow + d);
    f32x4 vv = *(const f32x4*)(vbase + (int64_t)gc * p.v_sr + d);
    if (gk >= lk) kv = vv = f32x4{0.f, 0.f, 0.f, 0.f};
    *(f32x4*)(lkt + key * SF_KSTR + 4 * c) = kv;
#pragma unroll
    for (int j = 0; j < 4; ++j) lvt[(4 * c + j) * SF_VSTR + key] = vv[j];
  }
  for (int j = tid; j < SF_KT; j += 512) {
    const int gk = k0 + j;
    float b2 = TA_NEG_INF;
    if (gk < lk) b2 = p.bias ? fmaxf(p.bias[b * p.bias_sb + gk] * TA_LOG2E, SH_BIAS_FLOOR) : 0.f;
    lb2[j] = b2;
  }
}

template <bool RESIDENT>
__global__ __launch_bounds__(512, 4) void sf_kernel(ShParams p) {
  __shared__ __attribute__((aligned(16))) float lkt[SF_KT * SF_KSTR];
  __shared__ __attribute__((aligned(16))) float lvt[SF_W * SF_VSTR];
  __shared__ __attribute__((aligned(16))) float lb2[SF_KT];
  __shared__ int sf_bad;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int hg = work % (SH_H / SF_HG), rest = work / (SH_H / SF_HG);
  const int b = rest / p.nwg_b, qb0 = (rest % p.nwg_b) * p.qbpw;
  int lk = p.Lk;
  if (p.valid) {
    const int vl = p.valid[p.valid_n == 1 ? 0 : b];
    lk = vl < 0 ? 0 : (vl < lk ? vl : lk);
  }
  const int ntiles = (lk + SF_KT - 1) / SF_KT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int gl = wave & (SF_HG - 1), par = wave / SF_HG;
  const int hd = gl * SH_D, d0 = hg * SF_W + hd + 4 * kap;
  const int nb = p.nqb - qb0 < p.qbpw ? p.nqb - qb0 : p.qbpw;

  if constexpr (RESIDENT) {
    if (ntiles == 1) {
      sf_fill(p, lkt, lvt, lb2, b, hg, 0, lk);
      __syncthreads();
    }
    const int nkb = (lk + 15) >> 4;
    const bool addb = p.bias != nullptr || (lk & 15) != 0;
    for (int bi = par; bi < nb; bi += 2) {
      const int qi = (qb0 + bi) * 16 + l16;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      float m = 0.f, l = 0.f;
      if (ntiles == 1) {
        const f32x4 q = sf_qop(p, b, qi, d0);
        f32x4 q2;
#pragma unroll
        for (int r = 0; r < 4; ++r) q2[r] = q[r] * TA_LOG2E;
        sf_tile_fix<true>(lkt, lvt, lb2, nkb, q2, hd, l16, kap, addb, o, m, l);
        if (wave_any(sf_suspect(o, l))) {
          // rare: the exact online softmax over the same keys (still in LDS)
          o = f32x4{0.f, 0.f, 0.f, 0.f};
          m = TA_NEG_INF;
          l = 0.f;
          sf_tile(lkt, lvt, lb2, nkb, q, hd, l16, kap, o, m, l);
        }
      }
      sf_store(p, b, qi, d0, o, l);
    }
  } else {
    f32x4 qop[SF_SB], o[SF_SB];
    float m[SF_SB], l[SF_SB];
    // fast pass: a softmax reference fixed by each block's first 16 keys
#pragma unroll
    for (int j = 0; j < SF_SB; ++j) {
      const f32x4 q = sf_qop(p, b, (qb0 + par + 2 * j) * 16 + l16, d0);
#pragma unroll
      for (int r = 0; r < 4; ++r) qop[j][r] = q[r] * TA_LOG2E;
      o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      m[j] = 0.f;
      l[j] = 0.f;
    }
    if (threadIdx.x == 0) sf_bad = 0;
    if (!p.rope) {
      // 64-key tiles in the two halves of the LDS tile: the next tile's K / V rows and b2 are loaded
      // into registers before the current one is computed and stored to the other half after it,
      // so the loads are in flight during the products (one barrier per tile). With RoPE the fill
      // rotates K at the store: the unpipelined 128-key sweep below.
      constexpr int HK = SF_KT / 2;
      constexpr int HU = HK * (SF_W / 4) / 512;  // 16-byte K / V chunks per thread and tile
      const int nt = (lk + HK - 1) / HK;
      const int tid = threadIdx.x;
      const float* kbase = (const float*)p.k + b * p.k_sb;
      const float* vbase = (const float*)p.v + b * p.v_sb;
      f32x4 rk[HU], rv[HU];
      float rb = TA_NEG_INF;
      auto fetch = [&](int t) {
#pragma unroll
        for (int i = 0; i < HU; ++i) {
          const int u = tid + 512 * i, key = u >> 4, c = u & 15;
          const int gk = t * HK + key, gc = gk < lk ? gk : lk - 1;
          rk[i] = *(const f32x4*)(kbase + (int64_t)gc * p.k_sr + hg * SF_W + 4 * c);
          rv[i] = *(const f32x4*)(vbase + (int64_t)gc * p.v_sr + hg * SF_W + 4 * c);
          if (gk >= lk) rk[i] = rv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if (tid < HK) {
          const int gk = t * HK + tid;
          rb = TA_NEG_INF;
          if (gk < lk) rb = p.bias ? fmaxf(p.bias[b * p.bias_sb + gk] * TA_LOG2E, SH_BIAS_FLOOR) : 0.f;
        }
      };
      auto put = [&](int h) {
#pragma unroll
        for (int i = 0; i < HU; ++i) {
          const int u = tid + 512 * i, key = HK * h + (u >> 4), c = u & 15;
          *(f32x4*)(lkt + key * SF_KSTR + 4 * c) = rk[i];
#pragma unroll
          for (int j = 0; j < 4; ++j) lvt[(4 * c + j) * SF_VSTR + key] = rv[i][j];
        }
        if (tid < HK) lb2[HK * h + tid] = rb;
      };
      if (nt > 0) {  // lk >= 1: the clamped row lk - 1 exists
        fetch(0);
        put(0);
      }
      __syncthreads();
      for (int t = 0; t < nt; ++t) {
        const int h = t & 1;
        if (t + 1 < nt) fetch(t + 1);
        const int rem = lk - t * HK;
        const int nkb = rem >= HK ? HK / 16 : (rem + 15) >> 4;
        const bool addb = p.bias != nullptr || (rem < HK && (rem & 15) != 0);
#pragma unroll
        for (int j = 0; j < SF_SB; ++j) {
          if (par + 2 * j < nb) {
            if (t == 0)
              sf_tile_fix<true, HK / 16>(lkt + HK * h * SF_KSTR, lvt + HK * h, lb2 + HK * h, nkb, qop[j], hd, l16,
                                         kap, addb, o[j], m[j], l[j]);
            else
              sf_tile_fix<false, HK / 16>(lkt + HK * h * SF_KSTR, lvt + HK * h, lb2 + HK * h, nkb, qop[j], hd,
                                          l16, kap, addb, o[j], m[j], l[j]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        // half h ^ 1 was last read by tile t - 1's products, which every wave finished before the
        // previous barrier
        if (t + 1 < nt) put(h ^ 1);
        __syncthreads();
      }
    } else {
      for (int t = 0; t < ntiles; ++t) {
        __syncthreads();
        sf_fill(p, lkt, lvt, lb2, b, hg, t, lk);
        __syncthreads();
        const int rem = lk - t * SF_KT;
        const int nkb = rem >= SF_KT ? SF_KT / 16 : (rem + 15) >> 4;
        const bool addb = p.bias != nullptr || (rem < SF_KT && (rem & 15) != 0);
#pragma unroll
        for (int j = 0; j < SF_SB; ++j) {
          if (par + 2 * j < nb) {
            if (t == 0)
              sf_tile_fix<true>(lkt, lvt, lb2, nkb, qop[j], hd, l16, kap, addb, o[j], m[j], l[j]);
            else
              sf_tile_fix<false>(lkt, lvt, lb2, nkb, qop[j], hd, l16, kap, addb, o[j], m[j], l[j]);
          }
          __builtin_amdgcn_sched_barrier(0);  // one block at a time: interleaving them costs registers
        }
      }
    }
    bool bad = false;
#pragma unroll
    for (int j = 0; j < SF_SB; ++j)
      if (par + 2 * j < nb) bad |= sf_suspect(o[j], l[j]);
    if (wave_any(bad) && lane == 0) sf_bad = 1;
    __syncthreads();
    if (sf_bad) {
      // rare: the whole workgroup sweeps its keys again with the exact online softmax
#pragma unroll
      for (int j = 0; j < SF_SB; ++j) {
        qop[j] = sf_qop(p, b, (qb0 + par + 2 * j) * 16 + l16, d0);
        o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        m[j] = TA_NEG_INF;
        l[j] = 0.f;
      }
      for (int t = 0; t < ntiles; ++t) {
        __syncthreads();
        sf_fill(p, lkt, lvt, lb2, b, hg, t, lk);
        __syncthreads();
        const int rem = lk - t * SF_KT;
        const int nkb = rem >= SF_KT ? SF_KT / 16 : (rem + 15) >> 4;
#pragma unroll
        for (int j = 0; j < SF_SB; ++j) {
          if (par + 2 * j < nb) sf_tile(lkt, lvt, lb2, nkb, qop[j], hd, l16, kap, o[j], m[j], l[j]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < SF_SB; ++j)
      if (par + 2 * j < nb) sf_store(p, b, (qb0 + par + 2 * j) * 16 + l16, d0, o[j], l[j]);
  }
}

// fp32: runs of query blocks sized for >= ~2048 workgroups (resident) or at most 2 SF_SB blocks
// (streaming: state carried across tiles), >= ~1024 workgroups when the batch allows.
void launch_sf(ShParams p, hipStream_t stream) {
  p.nqb = (p.Lq + 15) / 16;
  const int64_t groups = (int64_t)p.B * (SH_H / SF_HG);
  const bool resident = p.Lk <= SF_KT;
  int64_t run;
  if (resident) {
    run = (groups * p.nqb + 2047) / 2048;
    run = run < 2 ? 2 : (run > 32 ? 32 : run);
  } else {
    run = 2 * SF_SB;
    while (run > 2 && groups * ((p.nqb + run - 1) / run) < 1024) run /= 2;
  }
  p.qbpw = (int)(run > p.nqb ? p.nqb : run);
  p.nwg_b = (p.nqb + p.qbpw - 1) / p.qbpw;
  const dim3 grid((unsigned)(groups * p.nwg_b)), block(512);
  if (resident)
    hipLaunchKernelGGL((sf_kernel<true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((sf_kernel<false>), grid, block, 0, stream, p);
}

}  // namespace

int tabicl_launch_smallhead(const void* q, int64_t q_sb, int64_t q_sr, const void* k, int64_t k_sb,
                            int64_t k_sr, const void* v, int64_t v_sb, int64_t v_sr, void* o,
                            const float* bias, int64_t bias_sb, const int32_t* valid,
                            int64_t valid_n, const float* cq, const float* sq, const float* ck,
                            const float* sk, int rope, int half, int rot, float scale, int64_t B,
                            int64_t Lq, int64_t Lk, int dtype, void* ws, int64_t ws_bytes,
                            hipStream_t stream, const int32_t* qlen, int64_t qlen_n) {
  if (dtype == 0 && Lk > RS_LK && bias == nullptr && rope == 0)
    return tabicl_launch_ss(q, q_sb, q_sr, k, k_sb, k_sr, v, v_sb, v_sr, o, valid, valid_n, scale, B,
                            Lq, Lk, ws, ws_bytes, stream);
  // bf16, long keys, a key mask and a workspace with room for its prefix view: the batch elements
  // whose mask is a prefix mask run on the streaming kernel with that valid length, the others on
  // smallhead_fwd_kernel with the mask added term by term
  const int64_t pref = (B * 8 + 255) / 256 * 256;
  const bool gated = dtype == 0 && Lk > RS_LK && bias != nullptr && rope == 0 && ws != nullptr && ws_bytes >= pref;
  const int64_t pn = (bias_sb == 0 && valid_n <= 1) ? 1 : B;
  int32_t* pvalid = gated ? (int32_t*)ws : nullptr;
  if (gated) {
    int st = tabicl_launch_key_prefix(bias, bias_sb, bias_sb == 0 ? 1 : B, Lk, valid, valid ? valid_n : 0, pn,
                                      pvalid, pvalid + pn, stream);
    if (st == 0)
      st = tabicl_launch_ss(q, q_sb, q_sr, k, k_sb, k_sr, v, v_sb, v_sr, o, pvalid, pn, scale, B, Lq, Lk,
                            (char*)ws + pref, ws_bytes - pref, stream, pvalid + pn, pn);
    if (st != 0) return st;
  }
  ShParams p;
  p.q = q; p.q_sb = q_sb; p.q_sr = q_sr;
  p.k = k; p.k_sb = k_sb; p.k_sr = k_sr;
  p.v = v; p.v_sb = v_sb; p.v_sr = v_sr;
  p.o = o; p.o_sb = Lq * SH_E; p.o_sr = SH_E;
  p.bias = bias; p.bias_sb = bias_sb;
  p.valid = valid; p.valid_n = (int)valid_n;
  p.cq = cq; p.sq = sq; p.ck = ck; p.sk = sk;
  // rope: the form (none / pairs / halves) plus TA_ROPE_SHARED when the tables hold one head's 16
  // columns for every head
  p.tab_sr = (rope & TA_ROPE_SHARED) ? SH_D : SH_E;
  p.tab_cm = p.tab_sr - 1;
  rope &= ~TA_ROPE_SHARED;
  p.rope = rope; p.half = half; p.rot = rot;
  p.scale = scale;
  {
    int e = 0;
    p.exact_scale = scale > 0.f && frexpf(scale, &e) == 0.5f;
    p.pow2_scale = p.exact_scale;
    p.qc = scale * TA_LOG2E;
  }
  p.half_last = 0;
  p.qlen = qlen; p.qlen_n = (int)qlen_n;
  p.skip = gated ? pvalid + pn : nullptr; p.skip_n = (int)pn;
  p.rp_qsep = 0;
  p.B = (int)B; p.Lq = (int)Lq; p.Lk = (int)Lk;
  const bool fast_rope = rope == 0 || (rope == 1 && rot == 16) || (rope == 2 && half == 8 && rot == 16);
  // the resident kernel's buffer loads take 32-bit byte offsets within a batch element (query runs
  // are at most 64 blocks of 16 rows)
  const bool offsets_fit = k_sr >= 0 && v_sr >= 0 && q_sr >= 0 && Lk * k_sr * 2 < INT32_MAX &&
                           Lk * v_sr * 2 < INT32_MAX && 64 * 16 * q_sr * 2 < INT32_MAX;
  if (dtype == 0 && Lk <= RS_LK && fast_rope && offsets_fit) {
    // all keys resident: one workgroup per (batch element, run of 16-query blocks), one head per wave
    p.nqb = (int)((Lq + 15) / 16);
    // long enough runs to amortise the key fill, while keeping >= ~32 workgroups per CU for the grid
    const int64_t target_wgs = 256 * 32;
    int64_t qbpw = (B * (int64_t)p.nqb + target_wgs - 1) / target_wgs;
    qbpw = qbpw < 1 ? 1 : (qbpw > 64 ? 64 : qbpw);
    p.qbpw = (int)(qbpw > p.nqb ? p.nqb : qbpw);
    p.nwg_b = (p.nqb + p.qbpw - 1) / p.qbpw;
    // short runs: splitting q' log2e per block (a few VALU per block) costs less than splitting every
    // key of the head once per workgroup (~320 VALU per wave); same product to ~2^-17 either way
    if (p.qbpw <= 8) p.exact_scale = 0;
    if (rope) p.exact_scale = 0;
    const int64_t nblk = B * (int64_t)p.nwg_b;
    const int ngrp = (int)((Lk + 31) / 32);  // 32-key groups every batch element sweeps
    p.half_last = Lk - 32 * (ngrp - 1) <= 16;
    const int mode = (bias || valid) ? 0 : (Lk == 32 * ngrp ? 2 : 1);
    p.rp_qsep = 0;
    const int st = launch_persist(p, ngrp, mode, stream);
    if (st >= 0) return st;
    launch_resident(p, ngrp, mode, nblk, stream);
    return (int)hipGetLastError();
  }
  p.nqb = (int)((Lq + SH_QB - 1) / SH_QB);
  const int kt = 64;
  // all keys in one tile: keep them resident and walk up to 8 query blocks per workgroup
  p.qbpw = Lk <= kt ? (p.nqb < 8 ? p.nqb : 8) : 1;
  p.nwg_b = (p.nqb + p.qbpw - 1) / p.qbpw;
  const int64_t nblk = B * (int64_t)p.nwg_b;
  if (dtype == 0)
    hipLaunchKernelGGL((smallhead_fwd_kernel<bf16, 64>), dim3((unsigned)nblk), dim3(SH_NW * 64), 0,
                       stream, p);
  else
    launch_sf(p, stream);
  return (int)hipGetLastError();
}

int64_t tabicl_launch_smallhead_ws_bytes(int64_t B, int64_t Lq, int64_t Lk, int dtype, bool bias,
                                         int rope) {
  if (dtype == 0 && Lk > RS_LK && rope == 0)
    return tabicl_launch_ss_ws_bytes(B, Lq, Lk) + (bias ? (B * 8 + 255) / 256 * 256 : 0);
  return 0;
}
