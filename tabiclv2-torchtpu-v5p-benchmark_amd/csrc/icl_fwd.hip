// Dataset-wise in-context attention over cached train-row K/V, head_dim 64 (gfx950).
//
// Math (the Splash hook of the reference, results/tpu_patch.diff:123-155, 95-102): per (n, h),
//   O = softmax(scale * Q K^T + mask) V,  mask[j] = -inf for key j >= valid,
// fp32 scores and softmax, probabilities cast to the value dtype before the PV product.
//
// Work decomposition (both kernels): one workgroup = (n, h, key split, block of NW * QW queries);
// each wave owns QW = 32 * QC queries (QC column blocks of 32). Two kernels share it:
//  * icl_pipe_kernel (bf16, when the caller gives a workspace): tiles copied global -> LDS by the
//    load unit several tiles ahead, a softmax reference fixed per query, MFMA and softmax VALU
//    interleaved per half tile; it flags the work items whose scores leave the reference's range.
//  * icl_fwd_kernel (fp32; bf16 without a workspace; the flagged bf16 items): keys stream through
//    LDS in tiles of KT = 64, double buffered (the global loads of tile t+1 are issued into
//    registers before tile t is computed and written to the other LDS buffer afterwards), K
//    row-major, V transposed with the key order permuted inside each 16-key group so that every
//    MFMA operand is one 16-byte LDS read; per tile and wave
//      S^T (keys x queries) = K Q^T      v_mfma_f32_32x32x16_bf16, 2 key blocks x 4 d-slices x QC
//      online softmax in registers       lane l owns query l%32 of each column block; the two lanes
//                                        l, l^32 holding a query are combined with v_permlane32_swap
//      O^T (d x queries)   += V^T P^T    2 d-blocks x 4 key-slices x QC; P^T is the S^T accumulator
//                                        layout converted to bf16 in place (no shuffles)
//    with the running max updated lazily (accumulators rescaled only when the tile max exceeds the
//    running max by more than 2^8; exact because O and l always share the same reference max).
#include <atomic>
#include <cmath>
#include <mutex>

#include "common.h"
#include "launch.h"

namespace {

constexpr int ICL_D = 64;
constexpr int ICL_KT = 64;
constexpr float ICL_LAZY = 8.0f;  // log2 units

struct IclParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* valid;
  int valid_n;
  // query rows computed per batch element n (qlen[n], or qlen[0] for all; null: all Tq rows); rows
  // at or past it are neither computed nor written, work items holding none of them skip the sweep
  const int32_t* qlen;
  int qlen_n;
  int N, H, Tq, Tkv, nqb;
  int64_t q_sn, q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st;
  float sc;  // scale * log2(e)
  // key split: nsplit > 1 writes unnormalised partials (O, m, l) per split to the workspace
  int nsplit;
  float* ws_o;   // [nsplit][N*H][Tq][64]
  float* ws_ml;  // [nsplit][N*H][Tq][2], m in log2 units
  // per workgroup: 1 = the fast kernel's result must be recomputed exactly (null: no fast kernel)
  int* flags;
  // additive key mask: fp32 [bias_n][Tkv], row stride bias_sn, added to the scaled scores by
  // icl_fwd_kernel<..., BIAS = true>; bias_inv_scale = 1 / scale puts it in raw score units
  const float* bias;
  int64_t bias_sn;
  int bias_n;
  float bias_inv_scale;
  float scale;  // the score scale itself
  // prefix view of that mask for the pipelined kernel (pvalid / pok [pn], pn in {1, N}): rows whose
  // mask is a prefix mask run with valid length pvalid; the others run on icl_pipe_kernel<true> (a
  // power-of-two scale) or are flagged for icl_fwd_kernel
  const int32_t* pvalid;
  const int32_t* pok;
  int pn;
  // ragged calls of the pipelined kernel: [count, work items...] of the work items that hold a live
  // query row, in work-item order (written by icl_live_list_kernel; null: every work item is run)
  const int32_t* live;
  // optional, calls without a key mask: per query row [N * H][Tq][2] the softmax statistics (m, l) of
  // the final result, m in log2 units and l the sum of exp2(x - m) (the backward's normalisation),
  // written by whichever kernel writes the row's output
  float* stat;
};

__device__ __forceinline__ int icl_live_rows(const IclParams& p, int n) {
  if (!p.qlen) return p.Tq;
  const int r = p.qlen[p.qlen_n == 1 ? 0 : n];
  return r < 0 ? 0 : (r > p.Tq ? p.Tq : r);
}

// LDS tiles of the generic kernel for head dim D (64: ICL; 128: the folded ISAB-1 attention).
template <typename T, int D = ICL_D> struct IclLds {
  static constexpr int EPC = 16 / sizeof(T);      // elements per 16-byte chunk
  static constexpr int CPR = D / EPC;              // chunks per row
  static constexpr int KSTR = D + EPC;             // padded row strides (elements)
  static constexpr int VSTR = ICL_KT + EPC;
  static constexpr int K_ELEMS = ICL_KT * KSTR;
  static constexpr int V_ELEMS = D * VSTR;
};

// Position of key r (0..15) inside its 16-key group in the transposed V tile: bits 2 and 3
// swapped, so that lane half hh finds keys {4hh..4hh+3, 8+4hh..8+4hh+3} at 8hh..8hh+7.
__device__ __forceinline__ int vperm(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

__device__ __forceinline__ float lane_pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane_pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Physical element offset of logical key position `pos` in row `d` of the transposed V tile: the
// 8-element chunks of a row are XOR-swizzled by (d / 8) % 8, so that the transposing stores (eight
// rows d, d+8, ... at one key position) and the operand reads (32 rows at one chunk) both spread
// over all LDS banks.
__device__ __forceinline__ int vt_off(int d, int pos, int vstr) {
  return d * vstr + ((((pos >> 3) ^ (d >> 3)) & 7) << 3) + (pos & 7);
}

// Register staging of one K/V tile: each thread owns KREP 16-byte chunks of K rows and VREP pairs
// of 16-byte chunks of two consecutive V rows. Rows past `valid` are read from row valid-1 (always
// in bounds and finite whenever the visible rows are), so the masked keys of the last tile meet
// p = 0 times a finite value and nothing from the unused cache tail is ever read.
template <typename T, int NT, int D = ICL_D> struct Stage {
  static constexpr int EPC = IclLds<T, D>::EPC, CPR = IclLds<T, D>::CPR;
  static constexpr int KREP = ICL_KT * CPR / NT;
  static constexpr int VREP = (ICL_KT / 2) * CPR / NT;
  uint4 k[KREP];
  uint4 va[VREP], vb[VREP];

  __device__ __forceinline__ void load(const T* kbase, const T* vbase, int64_t k_st, int64_t v_st,
                                       int k0, int valid) {
    const int tid = threadIdx.x, last = valid - 1;
#pragma unroll
    for (int i = 0; i < KREP; ++i) {
      const int c = tid + i * NT, row = c / CPR, cc = c % CPR;
      const int key = min(k0 + row, last);
      k[i] = ldg16(kbase + (int64_t)key * k_st + cc * EPC);
    }
#pragma unroll
    for (int i = 0; i < VREP; ++i) {
      const int c = tid + i * NT, pr = c / CPR, cc = c % CPR;
      const int key0 = min(k0 + 2 * pr, last), key1 = min(k0 + 2 * pr + 1, last);
      va[i] = ldg16(vbase + (int64_t)key0 * v_st + cc * EPC);
      vb[i] = ldg16(vbase + (int64_t)key1 * v_st + cc * EPC);
    }
  }

  __device__ __forceinline__ void store(T* lds_k, T* lds_vt) const {
    typedef IclLds<T, D> L;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < KREP; ++i) {
      const int c = tid + i * NT, row = c / CPR, cc = c % CPR;
      *(uint4*)(lds_k + row * L::KSTR + cc * EPC) = k[i];
    }
#pragma unroll
    for (int i = 0; i < VREP; ++i) {
      const int c = tid + i * NT, pr = c / CPR, cc = c % CPR;
      const int pos = (2 * pr & ~15) | vperm(2 * pr & 15);
      const uint32_t a[4] = {va[i].x, va[i].y, va[i].z, va[i].w};
      const uint32_t b[4] = {vb[i].x, vb[i].y, vb[i].z, vb[i].w};
      if (sizeof(T) == 2) {
        // element e of a row is the low (e even) or high (e odd) half of word e/2
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d0 = cc * EPC + 2 * w;
          *(uint32_t*)(lds_vt + vt_off(d0, pos, L::VSTR)) = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);
          *(uint32_t*)(lds_vt + vt_off(d0 + 1, pos, L::VSTR)) = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);
        }
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w)
          *(uint2*)(lds_vt + vt_off(cc * EPC + w, pos, L::VSTR)) = make_uint2(a[w], b[w]);
      }
    }
  }
};

// Row-sum of the probabilities of one 16-value accumulator: bf16 pairs through v_dot2 against
// (1, 1) (the values the PV product uses), fp32 values by plain adds.
__device__ __forceinline__ float psum8(const bf16x8& p, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16x2 pr = {p[2 * i], p[2 * i + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
  }
  return acc;
}
__device__ __forceinline__ float psum8(const f32x8& p, float acc) {
#pragma unroll
  for (int i = 0; i < 8; ++i) acc += p[i];
  return acc;
}

template <typename T, int QC, int D = ICL_D> struct IclState {
  typedef typename OpVec<T, 8>::type Op8;
  Op8 qop[QC][D / 16];
  f32x16 o[QC][D / 32];
  float m_run[QC], l_run[QC];
};

// The key mask of one tile in LDS: thread t < ICL_KT stages key k0 + t of its row, in raw score
// units and clamped at -1e30 (so that every score stays finite: a row whose keys all carry the
// floor gets equal weights, as the reference's softmax over finfo.min terms does). Keys past `valid`
// (masked by the kernel anyway) read row entry valid - 1.
struct BiasStage {
  float b;
  __device__ __forceinline__ void load(const float* row, int k0, int valid, float inv_scale) {
    const int t = threadIdx.x;
    if (t < ICL_KT) b = fmaxf(row[min(k0 + t, valid - 1)] * inv_scale, -1e30f);
  }
  __device__ __forceinline__ void store(float* lds) const {
    if (threadIdx.x < ICL_KT) lds[threadIdx.x] = b;
  }
};

// One 32-key half kb of a key tile with the tile's key mask lb: S^T = K Q^T + mask, the online softmax
// update (the running max moves per half), O^T += V^T P^T. The masked instance of the kernel takes a
// tile in two such halves: only one half's scores and probabilities are live at a time, which keeps it
// within 256 VGPRs (two waves per SIMD; a whole-tile pass needed 264 registers, one wave per SIMD).
template <typename T, int QC, bool MASK, int D>
__device__ __forceinline__ void icl_half_bias(IclState<T, QC, D>& st, const T* lk, const T* lv, const float* lb,
                                              int k0, int valid, float sc, int lr, int hh, int kb) {
  typedef IclLds<T, D> L;
  typedef typename OpVec<T, 8>::type Op8;
  f32x16 s[QC];
#pragma unroll
  for (int qc = 0; qc < QC; ++qc)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[qc][r] = 0.f;
#pragma unroll
  for (int sl = 0; sl < D / 16; ++sl) {
    const Op8 a = *(const Op8*)(lk + (kb * 32 + lr) * L::KSTR + 16 * sl + 8 * hh);
#pragma unroll
    for (int qc = 0; qc < QC; ++qc) s[qc] = mfma32x32x16(a, st.qop[qc][sl], s[qc]);
  }
  // S^T row of reg r = key 8 (r / 4) + 4 hh + r % 4 of the 32-key block
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 bb = *(const float4*)(lb + kb * 32 + 8 * g + 4 * hh);
#pragma unroll
    for (int qc = 0; qc < QC; ++qc) {
      s[qc][4 * g] += bb.x;
      s[qc][4 * g + 1] += bb.y;
      s[qc][4 * g + 2] += bb.z;
      s[qc][4 * g + 3] += bb.w;
    }
  }
  if (MASK) {
#pragma unroll
    for (int qc = 0; qc < QC; ++qc)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (k0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3) >= valid) s[qc][r] = TA_NEG_INF;
  }
  Op8 pop[QC][2];
#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    float mx = s[qc][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[qc][r]);
    mx = lane_pair_max(mx);
    const float m_new = fmaxf(st.m_run[qc], mx);
    if (wave_any((m_new - st.m_run[qc]) * sc > ICL_LAZY)) {
      const float alpha = __builtin_amdgcn_exp2f((st.m_run[qc] - m_new) * sc);
      st.l_run[qc] *= alpha;
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.o[qc][db][r] *= alpha;
      st.m_run[qc] = m_new;
    }
    const float mr = st.m_run[qc];
    float lsum = 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
      for (int j = 0; j < 8; ++j)  // the difference first: scores reach the -1e30 floor (see icl_tile)
        pop[qc][m][j] = from_f32<T>(__builtin_amdgcn_exp2f((s[qc][8 * m + j] - mr) * sc));
      lsum = psum8(pop[qc][m], lsum);
    }
    st.l_run[qc] += lsum;
  }
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const Op8 a = *(const Op8*)(lv + vt_off(db * 32 + lr, kb * 32 + 16 * m + 8 * hh, L::VSTR));
#pragma unroll
      for (int qc = 0; qc < QC; ++qc) st.o[qc][db] = mfma32x32x16(a, pop[qc][m], st.o[qc][db]);
    }
}

// One key tile: S^T = K Q^T (+ the tile's key mask lb when BIAS), online softmax, O^T += V^T P^T.
// MASK: the tile crosses `valid`. With BIAS the tile goes through icl_half_bias twice.
template <typename T, int QC, bool MASK, int D, bool BIAS = false>
__device__ __forceinline__ void icl_tile(IclState<T, QC, D>& st, const T* lk, const T* lv, const float* lb,
                                         int k0, int valid, float sc, int lr, int hh) {
  if constexpr (BIAS) {
    icl_half_bias<T, QC, MASK, D>(st, lk, lv, lb, k0, valid, sc, lr, hh, 0);
    __builtin_amdgcn_sched_barrier(0);  // the second half's products start after the first half's PV
    icl_half_bias<T, QC, MASK, D>(st, lk, lv, lb, k0, valid, sc, lr, hh, 1);
    return;
  }
  typedef IclLds<T, D> L;
  typedef typename OpVec<T, 8>::type Op8;
  f32x16 s[QC][2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int qc = 0; qc < QC; ++qc)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[qc][kb][r] = 0.f;
#pragma unroll
    for (int sl = 0; sl < D / 16; ++sl) {
      const Op8 a = *(const Op8*)(lk + (kb * 32 + lr) * L::KSTR + 16 * sl + 8 * hh);
#pragma unroll
      for (int qc = 0; qc < QC; ++qc) s[qc][kb] = mfma32x32x16(a, st.qop[qc][sl], s[qc][kb]);
    }
  }
  if (BIAS) {
    // S^T row of reg r = key 8 (r / 4) + 4 hh + r % 4 of the 32-key block
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 bb = *(const float4*)(lb + kb * 32 + 8 * g + 4 * hh);
#pragma unroll
        for (int qc = 0; qc < QC; ++qc) {
          s[qc][kb][4 * g] += bb.x;
          s[qc][kb][4 * g + 1] += bb.y;
          s[qc][kb][4 * g + 2] += bb.z;
          s[qc][kb][4 * g + 3] += bb.w;
        }
      }
  }
  if (MASK) {
#pragma unroll
    for (int qc = 0; qc < QC; ++qc)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= valid) s[qc][kb][r] = TA_NEG_INF;
        }
  }

  Op8 pop[QC][2][2];
#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    float mx = s[qc][0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qc][kb][r]);
    mx = lane_pair_max(mx);
    const float m_new = fmaxf(st.m_run[qc], mx);
    if (wave_any((m_new - st.m_run[qc]) * sc > ICL_LAZY)) {
      const float alpha = __builtin_amdgcn_exp2f((st.m_run[qc] - m_new) * sc);
      st.l_run[qc] *= alpha;
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.o[qc][db][r] *= alpha;
      st.m_run[qc] = m_new;
    }
    const float nm = -st.m_run[qc] * sc;
    const float mr = st.m_run[qc];
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          // with a key mask the scores can be huge (down to the -1e30 floor); there fma(s, sc, -m sc)
          // would turn the rounding of m sc into the exponent, so the difference is taken first
          const float x = BIAS ? (s[qc][kb][8 * m + j] - mr) * sc : fmaf(s[qc][kb][8 * m + j], sc, nm);
          pop[qc][kb][m][j] = from_f32<T>(__builtin_amdgcn_exp2f(x));
        }
        lsum = psum8(pop[qc][kb][m], lsum);
      }
    st.l_run[qc] += lsum;
  }

#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Op8 a = *(const Op8*)(lv + vt_off(db * 32 + lr, kb * 32 + 16 * m + 8 * hh, L::VSTR));
#pragma unroll
        for (int qc = 0; qc < QC; ++qc) st.o[qc][db] = mfma32x32x16(a, pop[qc][kb][m], st.o[qc][db]);
      }
}

template <typename T, int NW, int QC, int D = ICL_D, bool BIAS = false>
__global__ __launch_bounds__(NW * 64) void icl_fwd_kernel(IclParams p) {
  typedef IclLds<T, D> L;
  typedef typename OpVec<T, 8>::type Op8;
  constexpr int NT = NW * 64;
  constexpr int QW = 32 * QC;
  __shared__ __attribute__((aligned(16))) T lds_k[2][L::K_ELEMS];
  __shared__ __attribute__((aligned(16))) T lds_vt[2][L::V_ELEMS];
  __shared__ __attribute__((aligned(16))) float lds_b[BIAS ? 2 : 1][BIAS ? ICL_KT : 4];

  // work item = (n, h, split, query block); consecutive items share (n, h) and stay on one XCD
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  // behind the pipelined kernel: only the work items it flagged
  if (p.flags && p.flags[work] == 0) return;
  const int qb = work % p.nqb;
  const int rest = work / p.nqb;
  const int split = rest % p.nsplit;
  const int nh = rest / p.nsplit;
  const int h = nh % p.H, n = nh / p.H;

  int valid = p.Tkv;
  if (p.valid) {
    valid = p.valid[p.valid_n == 1 ? 0 : n];
    valid = valid < 0 ? 0 : (valid > p.Tkv ? p.Tkv : valid);
  }
  // a row whose key mask is a prefix mask ends at its prefix here too (the mask is 0 below it), so
  // the keys past it are never read, as in the pipelined kernel
  if (p.pok && p.pok[p.pn == 1 ? 0 : n]) valid = p.pvalid[p.pn == 1 ? 0 : n];

  const int live = icl_live_rows(p, n);
  if (qb * (QW * NW) >= live) return;  // no live query row: nothing to compute or write

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 31, hh = lane >> 5;
  const int qw0 = qb * (QW * NW) + wave * QW;

  const T* qbase = (const T*)p.q + n * p.q_sn + h * p.q_sh;
  const T* kbase = (const T*)p.k + n * p.k_sn + h * p.k_sh;
  const T* vbase = (const T*)p.v + n * p.v_sn + h * p.v_sh;

  IclState<T, QC, D> st;
#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    const int qi = qw0 + qc * 32 + lr;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      Op8 z = {};
      st.qop[qc][s] = qi < p.Tq ? *(const Op8*)(qbase + (int64_t)qi * p.q_st + 16 * s + 8 * hh) : z;
    }
    st.m_run[qc] = TA_NEG_INF;
    st.l_run[qc] = 0.f;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.o[qc][db][r] = 0.f;
  }
  const float sc = p.sc;

  // this split's tiles [t0, t1) of the ceil(valid / KT) key tiles
  const int ntiles = (valid + ICL_KT - 1) / ICL_KT;
  const int per = (ntiles + p.nsplit - 1) / p.nsplit;
  const int t0 = min(split * per, ntiles), t1 = min(t0 + per, ntiles);
  if (t1 > t0) {
    const float* brow = BIAS ? p.bias + (p.bias_n == 1 ? 0 : (int64_t)n * p.bias_sn) : nullptr;
    Stage<T, NT, D> stg;
    BiasStage bst;
    stg.load(kbase, vbase, p.k_st, p.v_st, t0 * ICL_KT, valid);
    if (BIAS) bst.load(brow, t0 * ICL_KT, valid, p.bias_inv_scale);
    stg.store(lds_k[0], lds_vt[0]);
    if (BIAS) bst.store(lds_b[0]);
    __syncthreads();
    // all tiles but the last one of the range: no key past `valid`
    for (int t = t0; t + 1 < t1; ++t) {
      const int k0 = t * ICL_KT, buf = (t - t0) & 1;
      stg.load(kbase, vbase, p.k_st, p.v_st, k0 + ICL_KT, valid);
      if (BIAS) bst.load(brow, k0 + ICL_KT, valid, p.bias_inv_scale);
      icl_tile<T, QC, false, D, BIAS>(st, lds_k[buf], lds_vt[buf], lds_b[BIAS ? buf : 0], k0, valid, sc, lr, hh);
      stg.store(lds_k[buf ^ 1], lds_vt[buf ^ 1]);
      if (BIAS) bst.store(lds_b[BIAS ? buf ^ 1 : 0]);
      __syncthreads();
    }
    const int tl = t1 - 1, bl = (tl - t0) & 1;
    if (t1 == ntiles)
      icl_tile<T, QC, true, D, BIAS>(st, lds_k[bl], lds_vt[bl], lds_b[BIAS ? bl : 0], tl * ICL_KT, valid, sc, lr, hh);
    else
      icl_tile<T, QC, false, D, BIAS>(st, lds_k[bl], lds_vt[bl], lds_b[BIAS ? bl : 0], tl * ICL_KT, valid, sc, lr,
                                      hh);
  }

  if (p.nsplit > 1) {
    // unnormalised partial result of this key range: O (fp32), running max m and sum l
#pragma unroll
    for (int qc = 0; qc < QC; ++qc) {
      const float lt = lane_pair_sum(st.l_run[qc]);
      const int qi = qw0 + qc * 32 + lr;
      if (qi < live) {
        const int64_t row = ((int64_t)split * p.N * p.H + nh) * p.Tq + qi;
        float* orow = p.ws_o + row * D;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 ov = make_float4(st.o[qc][db][4 * j], st.o[qc][db][4 * j + 1], st.o[qc][db][4 * j + 2],
                                    st.o[qc][db][4 * j + 3]);
            *(float4*)(orow + 32 * db + 8 * j + 4 * hh) = ov;
          }
        if (hh == 0) *(float2*)(p.ws_ml + row * 2) = make_float2(st.m_run[qc] * sc, lt);
      }
    }
    return;
  }

#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    const float lt = lane_pair_sum(st.l_run[qc]);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int qi = qw0 + qc * 32 + lr;
    if (qi < live) {
      if (p.stat && hh == 0) *(float2*)(p.stat + ((int64_t)nh * p.Tq + qi) * 2) = make_float2(st.m_run[qc] * sc, lt);
      T* orow = (T*)p.o + n * p.o_sn + h * p.o_sh + (int64_t)qi * p.o_st;
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          typename OpVec<T, 4>::type ov;
#pragma unroll
          for (int r = 0; r < 4; ++r) ov[r] = from_f32<T>(st.o[qc][db][4 * j + r] * inv);
          *(typename OpVec<T, 4>::type*)(orow + 32 * db + 8 * j + 4 * hh) = ov;
        }
    }
  }
}

// Combines the per-split partials (m in log2 units): m* = max_s m_s, w_s = 2^(m_s - m*),
// O = sum_s w_s O_s / sum_s w_s l_s (0 when no split saw a valid key). One thread per 4 outputs.
template <typename T, int D = ICL_D>
__global__ __launch_bounds__(256) void icl_merge_kernel(IclParams p) {
  const int64_t rows = (int64_t)p.N * p.H * p.Tq;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * (D / 4)) return;
  const int64_t row = idx / (D / 4);
  const int c4 = (int)(idx % (D / 4)) * 4;
  const int64_t nh = row / p.Tq;
  const int qi = (int)(row % p.Tq);
  const int n = (int)(nh / p.H), h = (int)(nh % p.H);
  if (qi >= icl_live_rows(p, n)) return;  // not computed: no partials to merge, nothing written
  float mstar = TA_NEG_INF;
  for (int s = 0; s < p.nsplit; ++s) {
    const float2 ml = *(const float2*)(p.ws_ml + ((int64_t)s * rows + row) * 2);
    if (ml.y > 0.f) mstar = fmaxf(mstar, ml.x);
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float l = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const float2 ml = *(const float2*)(p.ws_ml + ((int64_t)s * rows + row) * 2);
    if (!(ml.y > 0.f)) continue;
    const float w = __builtin_amdgcn_exp2f(ml.x - mstar);
    const float4 o = *(const float4*)(p.ws_o + ((int64_t)s * rows + row) * D + c4);
    acc.x += w * o.x; acc.y += w * o.y; acc.z += w * o.z; acc.w += w * o.w;
    l += w * ml.y;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (p.stat && c4 == 0) *(float2*)(p.stat + row * 2) = make_float2(mstar, l);
  T* dst = (T*)p.o + n * p.o_sn + h * p.o_sh + (int64_t)qi * p.o_st + c4;
  typename OpVec<T, 4>::type ov;
  ov[0] = from_f32<T>(acc.x * inv); ov[1] = from_f32<T>(acc.y * inv);
  ov[2] = from_f32<T>(acc.z * inv); ov[3] = from_f32<T>(acc.w * inv);
  *(typename OpVec<T, 4>::type*)dst = ov;
}

// ---------------------------------------------------------------------------------------------
// Pipelined bf16 kernel (the bf16 path whenever the caller gives a workspace). Same work items and
// results as icl_fwd_kernel<bf16, 4, 2>, with three changes that let one wave keep the MFMA pipe
// and the VALU busy at the same time:
//  * K and V tiles are copied global -> LDS by the load unit (global_load_lds_dwordx4) three tiles
//    ahead, row-major [key][d] with 128-byte rows whose 16-byte chunks are XOR-swizzled by the key;
//    the V^T operands of the PV product come from ds_read_b64_tr_b16.
//  * the softmax reference m (per query) is the ceiled maximum over the first 32 keys of the work
//    item's key range and then stays fixed: no running max, no rescale, p = exp2(s sc - m) may
//    exceed 1. At the end, l <= 2^96 and a finite O show that every p stayed far inside the
//    bf16/fp32 range, so the result is the max-subtracted softmax to rounding (fp32/bf16 relative
//    precision does not depend on scale). Otherwise the work item is flagged in the workspace and
//    icl_fwd_kernel, launched right after on the same stream, recomputes exactly those items.
//  * per 32-key half tile a wave runs 16 MFMAs (S of the next half, PV of the previous half), each
//    followed by the VALU work of two probabilities of the current half (fma, exp2, convert, dot2
//    row sum), in one basic block ordered with sched_barrier.
// ---------------------------------------------------------------------------------------------
constexpr int IP_NW = 4;
constexpr int IP_QW = 64;
constexpr int IP_NBUF = 4;
constexpr int IP_TILE = 2 * ICL_KT * ICL_D;  // bf16 elements per buffer: K tile then V tile (16 KB)
constexpr float IP_L_HI = 0x1p96f;
constexpr float IP_L_LO = 0x1p-64f;  // with a key mask: below it the fixed reference lost the row

// 16-byte chunk swizzle of a 128-byte tile row: a bijection on key % 8 that keeps (a) any 8
// consecutive rows at one chunk and (b) the chunk pairs {c, c^1} of 4 consecutive rows on distinct
// banks.
__device__ __forceinline__ int ip_swz(int key) { return ((key & 3) << 1) | ((key >> 2) & 1); }

struct IpState {
  bf16x8 qop[2][4];
  f32x16 o[2][2];
  float nm[2];      // -m (log2 units) of this lane's query in column block qc
  f32x4 lacc[2];    // row sums of column block qc: element 0 of lanes 0..31 (query lane % 32)
  bf16x8 rs_ones;   // A operand of the row-sum product
};

// The row sums come from the matrix core: a 16x16x32 MFMA reads a PV operand pop[qc][m] (lane l:
// keys 8(l/32)+j of query l%32) as its B operand, i.e. lane group g = l/16 as k rows 8g..8g+7 of
// column l%16, which hold keys 8(g>>1)+j of query 16(g&1) + l%16. With A row 0 = 1 on the groups
// g = 0, 2 and A row 4 = 1 on g = 1, 3, D[0][n] is the sum over the 16 keys of query n and D[4][n]
// that of query 16 + n; lane l < 32 receives D[4(l/16)][l%16], its own query's sum, in element 0,
// and lanes 32..63 receive zero rows. A lane holds A[l%16][8(l/16)+j].
__device__ __forceinline__ bf16x8 ip_rs_ones(int lane) {
  const bool one = ((lane & 15) == 0 && !((lane >> 4) & 1)) || ((lane & 15) == 4 && ((lane >> 4) & 1));
  const bf16 v = (bf16)(one ? 1.0f : 0.0f);
  const bf16x8 a = {v, v, v, v, v, v, v, v};
  return a;
}
__device__ __forceinline__ void ip_rowsum(IpState& st, const bf16x8 (&pop)[2][2], int qc, int m) {
  st.lacc[qc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.rs_ones, pop[qc][m], st.lacc[qc], 0, 0, 0);
}


// K operand of the S product: d-slice sl of rows kr..kr+31 of the K tile.
__device__ __forceinline__ bf16x8 ip_kop(const bf16* lk, int kr, int sl, int lr, int hh) {
  const int row = kr + lr;
  return *(const bf16x8*)(lk + row * ICL_D + (((2 * sl + hh) ^ ip_swz(row)) << 3));
}

// V^T operand of one PV MFMA (d-block db, keys kr + 16m .. kr + 16m + 15): two transposed reads.
// Lane l holds V[key][32 db + l % 32] for the keys of k-slots 8 (l / 32) .. +7, in the order the
// S^T accumulator puts the probabilities: keys 4 hh + j and 8 + 4 hh + j (j = 0..3).
__device__ __forceinline__ bf16x8 ip_vop(const bf16* lv, int kr, int m, int db, int lane) {
  const int g = lane >> 4;
  const int key = kr + 16 * m + 4 * (g >> 1) + ((lane & 15) >> 2);
  const int lc = 4 * db + 2 * (g & 1) + ((lane & 3) >> 1);
  const int half = (lane & 1) * 4;
  const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)(lv + key * ICL_D + ((lc ^ ip_swz(key)) << 3) + half));
  const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)(lv + (key + 8) * ICL_D + ((lc ^ ip_swz(key + 8)) << 3) + half));
  // reassembled through whole-vector bit casts (per-element casts of a transposed-read result are
  // folded to element 0 by this compiler)
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
  const u32x2 xw = __builtin_bit_cast(u32x2, x);
  const u32x2 yw = __builtin_bit_cast(u32x2, y);
  const u32x4v w = {xw[0], xw[1], yw[0], yw[1]};
  return __builtin_bit_cast(bf16x8, w);
}

// Key mask of keys kr..kr+31 of a tile in the S^T accumulator's order (reg r = key kr + 8 (r / 4) +
// 4 hh + r % 4), from this wave's copy of the tile's mask row.
__device__ __forceinline__ f32x16 ip_bias(const float* lb, int kr, int hh) {
  f32x16 b;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 v = *(const float4*)(lb + kr + 8 * g + 4 * hh);
    b[4 * g] = v.x;
    b[4 * g + 1] = v.y;
    b[4 * g + 2] = v.z;
    b[4 * g + 3] = v.w;
  }
  return b;
}

// S^T of keys kr..kr+31 of the K tile for both column blocks (KB: started from the keys' mask, lb).
template <bool KB = false>
__device__ __forceinline__ void ip_s(f32x16 (&s)[2], const IpState& st, const bf16* lk, const float* lb, int kr, int lr,
                                     int hh) {
  if constexpr (KB) {
    const f32x16 b = ip_bias(lb, kr, hh);
    s[0] = b;
    s[1] = b;
  } else {
#pragma unroll
    for (int qc = 0; qc < 2; ++qc)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[qc][r] = 0.f;
  }
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) {
    const bf16x8 a = ip_kop(lk, kr, sl, lr, hh);
#pragma unroll
    for (int qc = 0; qc < 2; ++qc) s[qc] = mfma32x32x16(a, st.qop[qc][sl], s[qc]);
  }
}

// O^T += V^T P^T for keys kr..kr+31 of the V tile, and the row sums of P.
__device__ __forceinline__ void ip_pv(IpState& st, const bf16x8 (&pop)[2][2], const bf16* lv, int kr, int lane) {
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const bf16x8 a = ip_vop(lv, kr, m, db, lane);
#pragma unroll
      for (int qc = 0; qc < 2; ++qc) {
        st.o[qc][db] = mfma32x32x16(a, pop[qc][m], st.o[qc][db]);
        if (db == 0) ip_rowsum(st, pop, qc, m);
      }
    }
}

// Keys at or past `valid` out of S^T (keys k0 + 8(r/4) + 4hh + r%4).
__device__ __forceinline__ void ip_mask(f32x16 (&s)[2], int k0, int valid, int hh) {
#pragma unroll
  for (int qc = 0; qc < 2; ++qc)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (k0 + 8 * (r >> 2) + 4 * hh + (r & 3) >= valid) s[qc][r] = TA_NEG_INF;
}

// Probabilities 2k, 2k+1 of column block qc: exp2(s sc - m), one packed convert for the PV product
// (their row sums are taken with the PV product, on the matrix core).
__device__ __forceinline__ void ip_exp2(const f32x16 (&s)[2], const IpState& st, float sc, bf16x8 (&pop)[2][2],
                                        int qc, int k) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const float p0 = __builtin_amdgcn_exp2f(fmaf(s[qc][2 * k], sc, st.nm[qc]));
  const float p1 = __builtin_amdgcn_exp2f(fmaf(s[qc][2 * k + 1], sc, st.nm[qc]));
  const bf16x2 pr = {(bf16)p0, (bf16)p1};
  pop[qc][k >> 2][(2 * k) & 7] = pr[0];
  pop[qc][k >> 2][(2 * k + 1) & 7] = pr[1];
}

// One half-tile phase: probabilities of `cur` (keys k0..k0+31) into `pcur`; if DO_S, S^T of the
// next half tile (rows kr_next.. of lk_next) into `nxt`; if DO_PV, the PV product of the previous
// half tile's probabilities `pprev` (rows kr_prev.. of lv_prev). Eight steps of up to two MFMAs,
// each MFMA followed by two probabilities; operands are read from LDS two steps ahead. KB: the next
// half tile's scores start from its key mask (lb_next), the first score product's accumulator input.
template <bool MASK, bool DO_S, bool DO_PV, bool KB = false>
__device__ __forceinline__ void ip_phase(IpState& st, f32x16 (&cur)[2], f32x16 (&nxt)[2], bf16x8 (&pcur)[2][2],
                                         const bf16x8 (&pprev)[2][2], const bf16* lk_next, const float* lb_next,
                                         int kr_next, const bf16* lv_prev, int kr_prev, int k0, int valid, float sc,
                                         int lane) {
  const int lr = lane & 31, hh = lane >> 5;
  if (MASK) ip_mask(cur, k0, valid, hh);
  constexpr int I0 = DO_S ? 0 : 4, I1 = DO_PV ? 8 : 4;  // operand steps [I0, I1)
  auto read_op = [&](int i) -> bf16x8 {
    if (i < 4) return ip_kop(lk_next, kr_next, i, lr, hh);
    const int j = i - 4;  // (db, m) = (j >> 1, j & 1)
    return ip_vop(lv_prev, kr_prev, j & 1, j >> 1, lane);
  };
  f32x16 bnext;
  if constexpr (DO_S && KB) {
    bnext = ip_bias(lb_next, kr_next, hh);
  } else if (DO_S) {
#pragma unroll
    for (int qc = 0; qc < 2; ++qc)
#pragma unroll
      for (int r = 0; r < 16; ++r) nxt[qc][r] = 0.f;
  }
  bf16x8 op[8];
  if (I0 < I1) op[I0] = read_op(I0);
  if (I0 + 1 < I1) op[I0 + 1] = read_op(I0 + 1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < I0 || i >= I1) {
      ip_exp2(cur, st, sc, pcur, (2 * i) >> 3, (2 * i) & 7);
      ip_exp2(cur, st, sc, pcur, (2 * i + 1) >> 3, (2 * i + 1) & 7);
      continue;
    }
    if (i + 2 < I1) op[i + 2] = read_op(i + 2);
#pragma unroll
    for (int qc = 0; qc < 2; ++qc) {
      if (i < 4) {
        nxt[qc] = mfma32x32x16(op[i], st.qop[qc][i], KB && i == 0 ? bnext : nxt[qc]);
      } else {
        const int j = i - 4;
        st.o[qc][j >> 1] = mfma32x32x16(op[i], pprev[qc][j & 1], st.o[qc][j >> 1]);
        if (j < 2) ip_rowsum(st, pprev, qc, j);
      }
      const int step = 2 * i + qc;  // 0..15, two probabilities each
      ip_exp2(cur, st, sc, pcur, step >> 3, step & 7);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

struct IpCtx {
  const bf16* kbase;
  const bf16* vbase;
  int64_t k_st, v_st;
  uint32_t koff, voff;  // byte offsets in a tile of this lane's K / V chunk in rows 16w..16w+7
  uint32_t choff;       // byte offset of that chunk within its row (the same for rows 16w+8..)
  int lrow;             // this lane's row in rows 16w..16w+7
  uint32_t lds0;
  int t0, nt, valid, wave, lane;
  float sc;
  // KB: the row's key mask (global) and this wave's copy of tile buffer 0's mask row (LDS; buffer b's
  // at + b IP_NW ICL_KT floats)
  const float* brow;
  const float* lb;
};

// Queue the copy of the tile at key k0 into tile buffer bi (LDS byte address lds0 + bi 16 KB): wave w copies K
// rows 16w..16w+15 and V rows 16w..16w+15, 8 rows (1 KB) per instruction, from the tile's
// (wave-uniform) base plus each lane's 32-bit offset. Rows 16w+8.. share the swizzle of rows 16w..
// (it depends on row & 7). Rows past `valid` are read from row valid-1 (in bounds, and finite
// whenever the visible rows are); k0 < valid always. KB: and each wave copies the tile's 64 mask
// entries into its own slot of the buffer's mask rows (entries past `valid` from entry valid-1).
// FULL: the caller knows that k0 + 64 <= valid (no row to clamp: no per-lane compare or select).
template <bool KB = false, bool FULL = false>
__device__ __forceinline__ void ip_issue(const IpCtx& c, int bi, int k0) {
  const uint32_t buf = c.lds0 + bi * IP_TILE * 2;
  const bf16* kt = c.kbase + (int64_t)k0 * c.k_st;
  const bf16* vt = c.vbase + (int64_t)k0 * c.v_st;
  const int lim = c.valid - k0;  // rows below lim are visible
  const int64_t last = lim < ICL_KT ? lim - 1 : 0;  // offsets of the clamped row, used only when lim < 64
  const uint32_t kcl = (uint32_t)(last * c.k_st * 2) + c.choff;
  const uint32_t vcl = (uint32_t)(last * c.v_st * 2) + c.choff;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = i & 1;
    const bool in = FULL || c.lrow + 8 * j < lim;
    const uint32_t off = i < 2 ? (in ? c.koff + (uint32_t)(j * 16 * c.k_st) : kcl)
                               : (in ? c.voff + (uint32_t)(j * 16 * c.v_st) : vcl);
    lds_dma16_s(off, i < 2 ? kt : vt, buf + (i < 2 ? 0 : ICL_KT * ICL_D * 2) + (16 * c.wave + 8 * j) * ICL_D * 2);
  }
  if constexpr (KB)
    lds_dma4_s((uint32_t)min(k0 + c.lane, c.valid - 1) * 4u, c.brow, lds_addr(c.lb + bi * (IP_NW * ICL_KT)));
}

// Tile copies per wave and tile (the constant vmcnt of the joins counts them).
template <bool KB> constexpr int ip_copies() { return KB ? 5 : 4; }
template <bool KB> __device__ __forceinline__ void ip_join_tile() {
  if constexpr (KB) TA_WAIT_JOIN(5);
  else TA_WAIT_JOIN(4);
}

// Sweep iteration t (tile t0 + t, buffer t % IP_NBUF, no key past `valid`): phase A = softmax of
// its first half, S of its second half, PV of the previous tile's second half; join (tile t + 1
// landed, tile t - 1 retired); queue tile t + IP_NBUF - 1 into tile t - 1's buffer; phase B =
// softmax of the second half, S of the next tile's first half (unless LAST), PV of this tile's first
// half. B = t % IP_NBUF when the caller knows it (unrolled sweep: buffer addresses become
// immediate offsets), else -1.
// FULL: tile t + IP_NBUF - 1, the one this iteration queues, lies below `valid` (the steady state).
template <bool FIRST, bool LAST, int B = -1, bool KB = false, bool FULL = false>
__device__ __forceinline__ void ip_iter(IpState& st, f32x16 (&sA)[2], f32x16 (&sB)[2], bf16x8 (&pA)[2][2],
                                        bf16x8 (&pB)[2][2], bf16 (*lds)[IP_TILE], const IpCtx& c, int t) {
  const int b = B >= 0 ? B : t % IP_NBUF;
  const bf16* lk = lds[b];
  const bf16* lv = lk + ICL_KT * ICL_D;
  const bf16* lvp = lds[(b + IP_NBUF - 1) % IP_NBUF] + ICL_KT * ICL_D;
  const bf16* lkn = lds[(b + 1) % IP_NBUF];
  const float* lb = c.lb + b * (IP_NW * ICL_KT);
  const float* lbn = c.lb + ((b + 1) % IP_NBUF) * (IP_NW * ICL_KT);
  const int k0 = (c.t0 + t) * ICL_KT;
  ip_phase<false, true, !FIRST, KB>(st, sA, sB, pA, pB, lk, lb, 32, lvp, 32, k0, c.valid, c.sc, c.lane);
  static_assert(IP_NBUF == 4, "one tile's copies may stay in flight below");
  ip_join_tile<KB>();
  ip_issue<KB, FULL>(c, (b + IP_NBUF - 1) % IP_NBUF,
                     (FULL ? c.t0 + t + IP_NBUF - 1 : min(c.t0 + t + IP_NBUF - 1, c.t0 + c.nt - 1)) * ICL_KT);
  ip_phase<false, !LAST, true, KB>(st, sB, sA, pB, pA, lkn, lbn, 0, lv, 0, k0 + 32, c.valid, c.sc, c.lane);
}

// Sweep iteration t of a wave whose query rows are all past the live count (ragged calls): the same
// join and tile copy as ip_iter, in the same order, without the products and the softmax.
template <bool KB = false>
__device__ __forceinline__ void ip_iter_idle(const IpCtx& c, int t) {
  ip_join_tile<KB>();
  ip_issue<KB>(c, (t + IP_NBUF - 1) % IP_NBUF, min(c.t0 + t + IP_NBUF - 1, c.t0 + c.nt - 1) * ICL_KT);
}

// The tile that crosses `valid` (buffer b, keys k0..): S, mask, probabilities and PV per half,
// without the MFMA/VALU interleave (once per work item at most).
template <bool KB = false>
__device__ __forceinline__ void ip_tail(IpState& st, const bf16* lk, const bf16* lv, const float* lb, int k0, int valid,
                                        float sc, int lane) {
  const int lr = lane & 31, hh = lane >> 5;
#pragma unroll 1
  for (int half = 0; half < 2; ++half) {
    f32x16 sT[2];
    bf16x8 pT[2][2];
    ip_s<KB>(sT, st, lk, lb, 32 * half, lr, hh);
    ip_mask(sT, k0 + 32 * half, valid, hh);
#pragma unroll
    for (int j = 0; j < 16; ++j) ip_exp2(sT, st, sc, pT, j >> 3, j & 7);
    ip_pv(st, pT, lv, 32 * half, lane);
  }
}

// KB (a call with a key mask and a power-of-two scale, launched after the KB = false instance, which
// took the rows whose mask is a prefix mask and flagged the others): the rows whose mask is not a prefix
// mask, adding it in raw score units as the score product's accumulator input (q is taken times the
// scale, exactly, and the exponent's factor is log2 e alone); rows whose sum then leaves [2^-64, 2^96]
// (every key masked, say) stay flagged for icl_fwd_kernel.
template <bool KB>
__global__ __launch_bounds__(IP_NW * 64, 2) void icl_pipe_kernel(IclParams p) {
  __shared__ __attribute__((aligned(1024))) bf16 lds[IP_NBUF][IP_TILE];
  __shared__ __attribute__((aligned(16))) float lbias[KB ? IP_NBUF * IP_NW * ICL_KT : 4];
  __shared__ int wg_bad;

  int work;
  if (p.live) {
    // ragged call: the listed (live) work items, each XCD its section or an equal contiguous share of
    // the list (the work items of one (n, h) stay together, for L2); workgroups past it exit. The
    // padded grid's order would interleave live and empty work items, and the dispatcher's
    // placement then leaves part of the CUs with the live ones (C5's small buckets ran 2.4x slower
    // than a call of the live rows alone).
    const int cnt = p.live[0];
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
    if (p.H % 8 == 0) {  // one section per XCD (its heads h = xcd mod 8), cnt entries each
      if (j >= cnt) return;  // no flag written: icl_fwd_kernel checks the rows first
      work = p.live[1 + xcd * cnt + j];
    } else {  // one section: each XCD an equal contiguous share
      const int q8 = cnt >> 3, r8 = cnt & 7;
      if (j >= q8 + (xcd < r8 ? 1 : 0)) return;
      work = p.live[1 + xcd * q8 + (xcd < r8 ? xcd : r8) + j];
    }
  } else {
    work = xcd_remap(blockIdx.x, gridDim.x);
  }
  const int qb = work % p.nqb;
  const int rest = work / p.nqb;
  const int split = rest % p.nsplit;
  const int nh = rest / p.nsplit;
  const int h = nh % p.H, n = nh / p.H;

  int valid = p.Tkv;
  if (p.valid) {
    valid = p.valid[p.valid_n == 1 ? 0 : n];
    valid = valid < 0 ? 0 : (valid > p.Tkv ? p.Tkv : valid);
  }

  const int live = icl_live_rows(p, n);
  if (qb * (IP_QW * IP_NW) >= live) {  // no live query row: nothing to compute or write
    if (threadIdx.x == 0) p.flags[work] = 0;
    return;
  }
  if (p.pok) {
    // key mask: a prefix mask is the valid length pvalid; any other mask is flagged here for the KB
    // instance or for icl_fwd_kernel (which adds it term by term), and added by the KB instance
    const int pr = p.pn == 1 ? 0 : n;
    if (KB == (p.pok[pr] != 0)) {
      if (!KB && threadIdx.x == 0) p.flags[work] = 1;
      return;
    }
    valid = p.pvalid[pr];  // the plain valid length for a row whose mask is not a prefix mask
  }

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, hh = lane >> 5;
  const int qw0 = qb * (IP_QW * IP_NW) + wave * IP_QW;

  const bf16* qbase = (const bf16*)p.q + n * p.q_sn + h * p.q_sh;
  IpState st;
  st.rs_ones = ip_rs_ones(lane);
#pragma unroll
  for (int qc = 0; qc < 2; ++qc) {
    const int qi = qw0 + qc * 32 + lr;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 z = {};
      st.qop[qc][s] = qi < p.Tq ? *(const bf16x8*)(qbase + (int64_t)qi * p.q_st + 16 * s + 8 * hh) : z;
      if (KB) {
#pragma unroll
        for (int j = 0; j < 8; ++j) st.qop[qc][s][j] = (bf16)((float)st.qop[qc][s][j] * p.scale);
      }
    }
    st.nm[qc] = 0.f;
    st.lacc[qc] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.o[qc][db][r] = 0.f;
  }
  // Consume the q loads here: a load the compiler still tracks inside the sweep would make it wait
  // with s_waitcnt vmcnt(n), which also counts (and so waits for) the tile copies in flight.
#pragma unroll
  for (int qc = 0; qc < 2; ++qc)
#pragma unroll
    for (int s = 0; s < 4; ++s) asm volatile("" ::"v"(st.qop[qc][s]));
  if (threadIdx.x == 0) wg_bad = 0;
  __syncthreads();

  // this split's tiles [t0, t1) of the ceil(valid / KT) key tiles (as icl_fwd_kernel)
  const int ntiles = (valid + ICL_KT - 1) / ICL_KT;
  const int per = (ntiles + p.nsplit - 1) / p.nsplit;
  const int t0 = min(split * per, ntiles), t1 = min(t0 + per, ntiles);
  const int nt = t1 - t0;
  if (nt > 0) {
    IpCtx c;
    c.kbase = (const bf16*)p.k + n * p.k_sn + h * p.k_sh;
    c.vbase = (const bf16*)p.v + n * p.v_sn + h * p.v_sh;
    c.k_st = p.k_st;
    c.v_st = p.v_st;
    c.lds0 = lds_addr(&lds[0][0]);
    c.t0 = t0;
    c.nt = nt;
    c.valid = valid;
    c.wave = wave;
    c.lane = lane;
    c.sc = KB ? TA_LOG2E : p.sc;
    c.brow = KB ? p.bias + (p.bias_n == 1 ? 0 : (int64_t)n * p.bias_sn) : nullptr;
    c.lb = &lbias[KB ? wave * ICL_KT : 0];
    {
      const int row = 16 * wave + (lane >> 3);
      const int ch = (lane & 7) ^ ip_swz(row);
      c.lrow = row;
      c.choff = (uint32_t)(ch * 16);
      c.koff = (uint32_t)((row * c.k_st + ch * 8) * 2);
      c.voff = (uint32_t)((row * c.v_st + ch * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < IP_NBUF - 1; ++i) ip_issue<KB>(c, i, min(t0 + i, t1 - 1) * ICL_KT);
    // tile t0 landed, two more tiles' copies in flight
    if constexpr (KB) TA_WAIT_JOIN(10);
    else TA_WAIT_JOIN(8);
    static_assert(ip_copies<true>() == 5 && ip_copies<false>() == 4, "the joins' vmcnt counts");
    // tiles entirely below `valid` through the pipelined sweep, the crossing one (if any) after it
    const int nfull = (t1 == ntiles && valid % ICL_KT != 0) ? nt - 1 : nt;
    if (qw0 >= live) {
      // a ragged call's wave with no live row: only its share of the tile copies and the joins
      for (int t = 0; t < nfull; ++t) ip_iter_idle<KB>(c, t);
      TA_WAIT_JOIN(0);
      goto swept;
    }

    // reference m: ceiled maximum over the first 32 keys of the range
    f32x16 sA[2], sB[2];
    bf16x8 pA[2][2], pB[2][2];
    ip_s<KB>(sA, st, lds[0], c.lb, 0, lr, hh);
    if (t0 == ntiles - 1) ip_mask(sA, t0 * ICL_KT, valid, hh);
#pragma unroll
    for (int qc = 0; qc < 2; ++qc) {
      float mx = sA[qc][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sA[qc][r]);
      mx = lane_pair_max(mx) * c.sc;
      st.nm[qc] = mx > -1e4f ? -fminf(ceilf(mx), 1e4f) : 0.f;
    }

    if (nfull > 1) {
      ip_iter<true, false, -1, KB>(st, sA, sB, pA, pB, lds, c, 0);
      int t = 1;
      // t % IP_NBUF == 1 at the top; the four iterations queue tiles t + 3 .. t + 6, all below nfull
      for (; t + IP_NBUF + 2 < nfull; t += IP_NBUF) {
        ip_iter<false, false, 1, KB, true>(st, sA, sB, pA, pB, lds, c, t);
        ip_iter<false, false, 2, KB, true>(st, sA, sB, pA, pB, lds, c, t + 1);
        ip_iter<false, false, 3, KB, true>(st, sA, sB, pA, pB, lds, c, t + 2);
        ip_iter<false, false, 0, KB, true>(st, sA, sB, pA, pB, lds, c, t + 3);
      }
      for (; t + 1 < nfull; ++t) ip_iter<false, false, -1, KB>(st, sA, sB, pA, pB, lds, c, t);
      ip_iter<false, true, -1, KB>(st, sA, sB, pA, pB, lds, c, nfull - 1);
      ip_pv(st, pB, lds[(nfull - 1) % IP_NBUF] + ICL_KT * ICL_D, 32, lane);
    } else if (nfull == 1) {
      // one full tile: the unpipelined form (the same probabilities, products and order), then the
      // join that the pipelined iteration would make (tile 1 landed; the idle waves make it too).
      // A pipelined instance for this case kept the first tile's probabilities live across the
      // sweep and made the compiler spill 25 VGPRs around it.
      ip_tail<KB>(st, lds[0], lds[0] + ICL_KT * ICL_D, c.lb, t0 * ICL_KT, valid, c.sc, lane);
      ip_join_tile<KB>();
    }
    if (nfull < nt) {
      // the crossing tile landed at the last join (or before the sweep when it is the only tile)
      const bf16* lk = lds[nfull % IP_NBUF];
      ip_tail<KB>(st, lk, lk + ICL_KT * ICL_D, c.lb + (nfull % IP_NBUF) * (IP_NW * ICL_KT), (t0 + nfull) * ICL_KT,
                  valid, c.sc, lane);
    }
    TA_WAIT_JOIN(0);  // no copy into this workgroup's LDS may outlive it
  }
swept:

  if (p.qlen) {
    // rows at or past the live count are not written: clear their state so that they cannot flag
    // the work item for the exact recompute
#pragma unroll
    for (int qc = 0; qc < 2; ++qc)
      if (qw0 + qc * 32 + lr >= live) {
        st.nm[qc] = 0.f;
        st.lacc[qc] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) st.o[qc][db][r] = 0.f;
      }
  }

  // trust test of the fixed reference; any failing lane flags the work item for exact recompute
  float lt[2];
  bool bad = false;
#pragma unroll
  for (int qc = 0; qc < 2; ++qc) {
    lt[qc] = lane_pair_sum(st.lacc[qc][0]);
    bad |= !(lt[qc] <= IP_L_HI);
    if (KB) bad |= qw0 + qc * 32 + lr < live && !(lt[qc] >= IP_L_LO);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) bad |= !(__builtin_fabsf(st.o[qc][db][r]) <= 0x1p127f);
  }
  if (wave_any(bad)) wg_bad = 1;
  __syncthreads();
  if (threadIdx.x == 0) p.flags[work] = wg_bad;

  if (p.nsplit > 1) {
#pragma unroll
    for (int qc = 0; qc < 2; ++qc) {
      const int qi = qw0 + qc * 32 + lr;
      if (qi < live) {
        const int64_t row = ((int64_t)split * p.N * p.H + nh) * p.Tq + qi;
        float* orow = p.ws_o + row * ICL_D;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 ov = make_float4(st.o[qc][db][4 * j], st.o[qc][db][4 * j + 1], st.o[qc][db][4 * j + 2],
                                    st.o[qc][db][4 * j + 3]);
            *(float4*)(orow + 32 * db + 8 * j + 4 * hh) = ov;
          }
        if (hh == 0) *(float2*)(p.ws_ml + row * 2) = make_float2(-st.nm[qc], lt[qc]);
      }
    }
    return;
  }
#pragma unroll
  for (int qc = 0; qc < 2; ++qc) {
    const float inv = lt[qc] > 0.f ? 1.f / lt[qc] : 0.f;
    const int qi = qw0 + qc * 32 + lr;
    if (qi < live) {
      if (p.stat && hh == 0) *(float2*)(p.stat + ((int64_t)nh * p.Tq + qi) * 2) = make_float2(-st.nm[qc], lt[qc]);
      bf16* orow = (bf16*)p.o + n * p.o_sn + h * p.o_sh + (int64_t)qi * p.o_st;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x4 ov;
#pragma unroll
          for (int r = 0; r < 4; ++r) ov[r] = (bf16)(st.o[qc][db][4 * j + r] * inv);
          *(bf16x4*)(orow + 32 * db + 8 * j + 4 * hh) = ov;
        }
    }
  }
}

constexpr int ICL_DEV_CACHE = 64;

// CUs of the current device and resident workgroups per CU of the kernel that carries the work (the
// pipelined one for bf16, d = 64): queried once per device and kernel, then cached (cus * 256 + per_cu).
struct Residency {
  int64_t cus, per_cu;
};
template <typename T, int NW, int QC, int D>
Residency residency() {
  static std::atomic<int64_t> cache[ICL_DEV_CACHE];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return {0, 0};
  if (dev >= 0 && dev < ICL_DEV_CACHE) {
    const int64_t hit = cache[dev].load(std::memory_order_relaxed);
    if (hit > 0) return {hit >> 8, hit & 255};
  }
  int cus = 0, n = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return {0, 0};
  const hipError_t e =
      sizeof(T) == 2 && D == ICL_D
          ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_pipe_kernel<false>, IP_NW * 64, 0)
          : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_fwd_kernel<T, NW, QC, D>, NW * 64, 0);
  const int64_t per_cu = e == hipSuccess && n > 0 ? (n < 255 ? n : 255) : 1;
  if (dev >= 0 && dev < ICL_DEV_CACHE) cache[dev].store((int64_t)cus * 256 + per_cu, std::memory_order_relaxed);
  return {cus, per_cu};
}

// Number of key splits S = 1..4 (each keeping >= 8 key tiles) with the least modelled time, in
// units of one key tile of one work item at full occupancy:
//  - W = items S work items of u = tiles / S + F tiles; F = 12 is a work item's fixed cost (q loads,
//    the first tiles in flight, the softmax reference, the epilogue);
//  - each full round of R C items (C CUs, R resident per CU) takes R u; a last partial round takes
//    R u when some CU holds R of its items, else k u / 0.9 with k = its most items on one CU: fewer
//    workgroups on a CU each run faster, at 0.9 of the CU's full-occupancy throughput for one
//    (icl_pipe_kernel at C4: 42.09 ms per query at one workgroup per CU, 38.33 ms at two);
//  - each split beyond the first adds 3.5% for its partial results and the merge.
// Measured on one box, splits pay only when the grid would leave CUs idle: C4 (703 tiles, 1280
// items) runs 38.33 ms unsplit and 38.90 / 39.13 ms at 2 / 4 splits, and every bucket of C5's ICL
// leg runs fastest unsplit (43.07 ms per step against 51.1 - 60.2 ms at 2 - 4 splits).
double split_time(int64_t W, double u, int64_t C, int64_t R) {
  const int64_t per_round = C * R, full = W / per_round, rem = W % per_round;
  double t = (double)full * R * u;
  if (rem > 0) {
    const int64_t k = (rem + C - 1) / C;
    t += k >= R ? R * u : k * u / 0.9;
  }
  return t;
}
template <typename T, int NW, int QC, int D>
int pick_splits(int64_t items, int64_t Tkv) {
  const Residency r = residency<T, NW, QC, D>();
  if (r.cus <= 0) return 1;
  const int64_t tiles = (Tkv + ICL_KT - 1) / ICL_KT;
  constexpr double fixed = 12.0;
  int best = 1;
  double best_cost = split_time(items, (double)tiles + fixed, r.cus, r.per_cu);
  for (int s = 2; s <= 4; ++s) {
    if (tiles / s < 8) break;
    const double cost = split_time(items * s, (double)tiles / s + fixed, r.cus, r.per_cu) * (1.0 + 0.035 * (s - 1));
    if (cost < best_cost - 1e-9) { best = s; best_cost = cost; }
  }
  return best;
}

constexpr int ICL_LIST_MAXN = 8192;  // batch elements the live list takes (per-element counts in LDS)

// Live work items of a ragged call of the pipelined kernel (one workgroup of 1024 threads). Batch
// element n has lq(n) = ceil(live rows / 256) live query blocks, so nsplit * lq(n) live work items per
// head. With H a multiple of 8 the list is 8 sections of equal length C, one per XCD: section x holds
// the heads h = x (mod 8) of every element, in work-item order, so every XCD gets the same work and
// each (n, h)'s work items stay together (its K / V shared in that XCD's L2); list[0] = C. Otherwise
// one section in work-item order; list[0] = its length. Entries are work-item indices
// ((n * H + h) * nsplit + split) * nqb + qb. lq is scanned in LDS (each thread a run of up to 8
// elements, then a scan of the 1024 run totals); every entry finds its element by binary search.
__global__ __launch_bounds__(1024) void icl_live_list_kernel(IclParams p, int32_t* list) {
  __shared__ int pre[ICL_LIST_MAXN + 1];
  __shared__ int tot[1024];
  const int tid = threadIdx.x;
  const int qbr = IP_QW * IP_NW;
  constexpr int RUN = ICL_LIST_MAXN / 1024;
  int acc = 0;
  int c[RUN];
#pragma unroll
  for (int i = 0; i < RUN; ++i) {
    const int n = tid * RUN + i;
    c[i] = n < p.N ? (icl_live_rows(p, n) + qbr - 1) / qbr : 0;
    acc += c[i];
  }
  tot[tid] = acc;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // inclusive scan of the run totals
    const int x = tid >= d ? tot[tid - d] : 0;
    __syncthreads();
    tot[tid] += x;
    __syncthreads();
  }
  int run0 = tid == 0 ? 0 : tot[tid - 1];
#pragma unroll
  for (int i = 0; i < RUN; ++i) {
    const int n = tid * RUN + i;
    if (n <= p.N) pre[n] = run0;
    run0 += c[i];
  }
  __syncthreads();
  const bool by_xcd = p.H % 8 == 0;
  const int hx = by_xcd ? p.H / 8 : p.H;     // heads per section
  const int per = hx * p.nsplit;              // section entries per live query block
  const int C = per * pre[p.N];               // section length
  const int nsec = by_xcd ? 8 : 1;
  for (int t = tid; t < nsec * C; t += 1024) {
    const int x = t / C, r = t % C;
    const int key = r / per;  // the element n holds pre[n] <= key < pre[n + 1]
    int lo = 0, hi = p.N;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid] <= key) lo = mid; else hi = mid;
    }
    const int n = lo, lq = pre[n + 1] - pre[n];
    const int rr = r - per * pre[n];
    const int hh = rr / (p.nsplit * lq), rem = rr % (p.nsplit * lq);
    const int h = by_xcd ? hh * 8 + x : hh;
    list[1 + t] = ((n * p.H + h) * p.nsplit + rem / lq) * p.nqb + rem % lq;
  }
  if (tid == 0) list[0] = C;
}

// Workspace layout: [per-work-item flags, bf16 d = 64 only, 256-byte aligned][prefix view of a key
// mask, bf16 d = 64 only: valid [N], ok [N], 256-byte aligned][live work-item list of ragged calls,
// bf16 d = 64 only: count, items, 256-byte aligned][split partials: O fp32 [nsplit][rows][D], (m, l)
// [nsplit][rows][2]].
int64_t flag_bytes(int64_t nblk) { return (nblk * 4 + 255) / 256 * 256; }
int64_t list_bytes(int64_t nblk) { return ((nblk + 1) * 4 + 255) / 256 * 256; }
int64_t pref_bytes(int64_t N) { return (N * 8 + 255) / 256 * 256; }
int64_t part_bytes(int nsplit, int64_t rows, int D) { return nsplit > 1 ? (int64_t)nsplit * rows * (D + 2) * 4 : 0; }

template <typename T, int NW, int QC, int D>
int64_t workspace_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv) {
  const int64_t nqb = (Tq + 32 * QC * NW - 1) / (32 * QC * NW);
  const int s = pick_splits<T, NW, QC, D>(N * H * nqb, Tkv);
  return (sizeof(T) == 2 && D == ICL_D ? flag_bytes(N * H * nqb * s) + pref_bytes(N) + list_bytes(N * H * nqb * s) : 0) +
         part_bytes(s, N * H * Tq, D);
}

// bf16 d = 64 with a large enough workspace: pipelined kernel, then icl_fwd_kernel on the work
// items it flagged, then the split merge. Otherwise icl_fwd_kernel alone (splitting only if the
// workspace holds the partials).
// List modes of ragged calls: ICL_LIST_BUILD computes the live work-item list into the workspace and
// runs the call; ICL_LIST_READY takes the list an earlier ICL_LIST_ONLY launch (same sizes, q_len
// contents and workspace) left there; ICL_LIST_ONLY computes the list and launches nothing else.
enum { ICL_LIST_BUILD = 0, ICL_LIST_READY = 1, ICL_LIST_ONLY = 2 };

template <typename T, int NW, int QC, int D>
void launch(const IclParams& p0, void* ws, int64_t ws_bytes, hipStream_t stream, int list_mode = ICL_LIST_BUILD) {
  IclParams p = p0;
  p.nqb = (p.Tq + 32 * QC * NW - 1) / (32 * QC * NW);
  const int64_t rows = (int64_t)p.N * p.H * p.Tq;
  const int64_t items = (int64_t)p.N * p.H * p.nqb;
  p.nsplit = pick_splits<T, NW, QC, D>(items, p.Tkv);
  const int64_t have = ws ? ws_bytes : 0;
  bool fast = false;
  int64_t fb = 0;
  // the pipelined kernel's tile copies take 32-bit byte offsets within a tile (64 rows)
  const bool strides_fit = p.k_st >= 0 && p.v_st >= 0 && p.k_st < (1 << 24) && p.v_st < (1 << 24);
  if (sizeof(T) == 2 && D == ICL_D && strides_fit) {
    const int64_t pb = pref_bytes(p.N);
    auto head = [&](int s) { return flag_bytes(items * s) + pb + list_bytes(items * s); };
    if (have < head(p.nsplit) + part_bytes(p.nsplit, rows, D)) p.nsplit = 1;
    fb = head(p.nsplit);
    fast = have >= fb + part_bytes(p.nsplit, rows, D);
  }
  if (!fast) {
    fb = 0;
    if (have < part_bytes(p.nsplit, rows, D)) p.nsplit = 1;
  }
  p.flags = fast ? (int*)ws : nullptr;
  p.ws_o = (float*)((char*)ws + fb);
  p.ws_ml = p.ws_o + (p.nsplit > 1 ? (int64_t)p.nsplit * rows * D : 0);
  const int64_t nblk = items * p.nsplit;
  if (fast && p.bias) {
    // prefix view of the key mask, per n (or one row when neither the mask nor the valid length
    // varies over n), for the pipelined kernel
    p.pn = (p.bias_n == 1 && p.valid_n <= 1) ? 1 : p.N;
    int32_t* pv = (int32_t*)((char*)ws + flag_bytes(nblk));
    p.pvalid = pv;
    p.pok = pv + p.pn;
    tabicl_launch_key_prefix(p.bias, p.bias_sn, p.bias_n, p.Tkv, p.valid, p.valid_n, p.pn, pv, pv + p.pn, stream);
  }
  if (fast && p.qlen && p.N < ICL_LIST_MAXN) {
    int32_t* list = (int32_t*)((char*)ws + flag_bytes(nblk) + pref_bytes(p.N));
    if (list_mode != ICL_LIST_READY)
      hipLaunchKernelGGL(icl_live_list_kernel, dim3(1), dim3(1024), 0, stream, p, list);
    p.live = list;
  }
  if (list_mode == ICL_LIST_ONLY) return;
  if (fast) {
    hipLaunchKernelGGL(icl_pipe_kernel<false>, dim3((unsigned)nblk), dim3(IP_NW * 64), 0, stream, p);
    // rows whose key mask is not a prefix mask: the pipelined kernel adds it when the scale is a
    // power of two (q times the scale is then exact in bf16)
    int e = 0;
    if (p.bias && std::frexp(p.scale, &e) == 0.5f)
      hipLaunchKernelGGL(icl_pipe_kernel<true>, dim3((unsigned)nblk), dim3(IP_NW * 64), 0, stream, p);
  }
  if (p.bias)
    hipLaunchKernelGGL((icl_fwd_kernel<T, NW, QC, D, true>), dim3((unsigned)nblk), dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((icl_fwd_kernel<T, NW, QC, D>), dim3((unsigned)nblk), dim3(NW * 64), 0, stream, p);
  if (p.nsplit > 1) {
    const int64_t threads = rows * (D / 4);
    hipLaunchKernelGGL((icl_merge_kernel<T, D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
  }
}

}  // namespace

// Host launchers (called from the C ABI in abi.hip). D: head dim, 64 (ICL) or 128 (folded ISAB-1).
int64_t tabicl_launch_icl_ws_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int dtype) {
  if (D == 128)
    return dtype == 0 ? workspace_bytes<bf16, 4, 1, 128>(N, H, Tq, Tkv) : workspace_bytes<float, 8, 1, 128>(N, H, Tq, Tkv);
  return dtype == 0 ? workspace_bytes<bf16, 4, 2, 64>(N, H, Tq, Tkv) : workspace_bytes<float, 4, 1, 64>(N, H, Tq, Tkv);
}

int tabicl_launch_icl_fwd(const void* q, const void* k, const void* v, const int32_t* valid,
                          int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq,
                          int64_t Tkv, int64_t D, int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn,
                          int64_t k_sh, int64_t k_st, int64_t v_sn, int64_t v_sh, int64_t v_st,
                          int64_t o_sn, int64_t o_sh, int64_t o_st, float scale, int dtype,
                          void* ws, int64_t ws_bytes, hipStream_t stream, const int32_t* qlen,
                          int64_t qlen_n, const float* bias, int64_t bias_n, int64_t bias_sn, int list_mode,
                          float* stat) {
  IclParams p;
  p.q = q; p.k = k; p.v = v; p.o = out;
  p.valid = valid; p.valid_n = (int)valid_n;
  p.qlen = qlen; p.qlen_n = (int)qlen_n;
  p.N = (int)N; p.H = (int)H; p.Tq = (int)Tq; p.Tkv = (int)Tkv;
  p.nqb = 0;
  p.q_sn = q_sn; p.q_sh = q_sh; p.q_st = q_st;
  p.k_sn = k_sn; p.k_sh = k_sh; p.k_st = k_st;
  p.v_sn = v_sn; p.v_sh = v_sh; p.v_st = v_st;
  p.o_sn = o_sn; p.o_sh = o_sh; p.o_st = o_st;
  p.sc = scale * TA_LOG2E;
  p.nsplit = 1; p.ws_o = nullptr; p.ws_ml = nullptr; p.flags = nullptr;
  p.bias = bias; p.bias_n = (int)bias_n; p.bias_sn = bias_sn;
  p.bias_inv_scale = 1.0f / scale;
  p.scale = scale;
  p.pvalid = nullptr; p.pok = nullptr; p.pn = 0; p.live = nullptr;
  p.stat = stat;
  if (D == 128) {
    if (dtype == 0)
      launch<bf16, 4, 1, 128>(p, ws, ws_bytes, stream);
    else
      launch<float, 8, 1, 128>(p, ws, ws_bytes, stream);
  } else if (dtype == 0) {
    launch<bf16, 4, 2, 64>(p, ws, ws_bytes, stream, list_mode);
  } else if (list_mode != ICL_LIST_ONLY) {
    launch<float, 4, 1, 64>(p, ws, ws_bytes, stream);
  }
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Allocation-free launch: the work-item flags, the prefix view of a key mask, the live work-item list
// of ragged calls and the key-split partials live in `scratch`, a file-scope device array (one per GPU, held until the process ends),
// instead of a workspace from the caller. Host code never passes the array's name to a kernel: its
// device address is taken once per device with hipGetSymbolAddress and kept in g_scratch_ptr.
// Every call on a GPU shares that GPU's array (no call clears it: each kernel writes every entry it
// later reads), so calls that overlap on one GPU race.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) char scratch[TABICL_ICL_SCRATCH_BYTES];

namespace {

constexpr int ICL_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[ICL_MAX_DEVICES] = {};

// Device address of the current device's scratch array (looked up on the first call per device).
hipError_t scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= ICL_MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

int64_t tabicl_launch_icl_noalloc_min_bytes(int64_t N, int64_t H, int64_t Tq, int64_t D, int dtype) {
  // unsplit: flags per work item, the prefix view and the live list (bf16, d = 64, the pipelined
  // kernel); nothing else
  if (dtype != 0 || D != ICL_D) return 0;
  const int64_t nqb = (Tq + IP_QW * IP_NW - 1) / (IP_QW * IP_NW);
  return flag_bytes(N * H * nqb) + pref_bytes(N) + list_bytes(N * H * nqb);
}

int tabicl_launch_icl_fwd_noalloc(const void* q, const void* k, const void* v, const int32_t* valid,
                                  int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                                  int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                                  int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                                  float scale, int dtype, hipStream_t stream, const int32_t* qlen, int64_t qlen_n,
                                  const float* bias, int64_t bias_n, int64_t bias_sn) {
  void* ws = nullptr;
  const hipError_t e = scratch_ptr(&ws);
  if (e != hipSuccess) return (int)e;
  return tabicl_launch_icl_fwd(q, k, v, valid, valid_n, out, N, H, Tq, Tkv, ICL_D, q_sn, q_sh, q_st, k_sn, k_sh, k_st,
                               v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale, dtype, ws, TABICL_ICL_SCRATCH_BYTES, stream,
                               qlen, qlen_n, bias, bias_n, bias_sn, 0);
}
