// Dataset-wise in-context attention over cached train-row K/V, head_dim 64 (gfx950).
//
// Math (the Splash hook of the reference, results/tpu_patch.diff:123-155, 95-102): per (n, h),
//   O = softmax(scale * Q K^T + mask) V,  mask[j] = -inf for key j >= valid,
// fp32 scores and softmax, probabilities cast to the value dtype before the PV product.
//
// Work decomposition: one workgroup = (n, h, block of QB = 32 * NW queries); each wave owns 32
// queries. Keys stream through LDS in tiles of KT = 64: K row-major [key][d], V transposed
// [d][key] (key order permuted inside each 16-key group so that an MFMA operand is one 16-byte
// read). Per tile and wave:
//   S^T (keys x queries) = K Q^T      v_mfma_f32_32x32x16_bf16, 2 key blocks x 4 d-slices
//   online softmax in registers       lane l owns query l%32 (keys split over lanes l, l^32)
//   O^T (d x queries)   += V^T P^T    2 d-blocks x 4 key-slices; P^T is the S^T accumulator
//                                     layout converted to bf16 in place (no shuffles)
// The running max is updated lazily: the accumulators are rescaled only when the tile max
// exceeds the running max by more than 2^8 (p <= 256 otherwise), which is exact because O and
// l always share the same reference max.
#include "common.h"

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
  int N, H, Tq, Tkv, nqb;
  int64_t q_sn, q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st;
  float sc;  // scale * log2(e)
};

template <typename T> struct IclLds {
  static constexpr int EPC = 16 / sizeof(T);      // elements per 16-byte chunk
  static constexpr int CPR = ICL_D / EPC;          // chunks per row
  static constexpr int KSTR = ICL_D + EPC;         // padded row strides (elements)
  static constexpr int VSTR = ICL_KT + EPC;
  static constexpr int K_ELEMS = ICL_KT * KSTR;
  static constexpr int V_ELEMS = ICL_D * VSTR;
};

// Position of key r (0..15) inside its 16-key group in the transposed V tile: bits 2 and 3
// swapped, so that lane half hh finds keys {4hh..4hh+3, 8+4hh..8+4hh+3} at 8hh..8hh+7.
__device__ __forceinline__ int vperm(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

template <typename T>
__device__ __forceinline__ void icl_fill(const IclParams& p, T* lds_k, T* lds_vt, const T* kbase,
                                         const T* vbase, int k0, int valid) {
  typedef IclLds<T> L;
  constexpr int EPC = L::EPC, CPR = L::CPR;
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int c = tid; c < ICL_KT * CPR; c += nt) {
    const int row = c / CPR, cc = c % CPR, key = k0 + row;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (key < valid) val = ldg16(kbase + (int64_t)key * p.k_st + cc * EPC);
    *(uint4*)(lds_k + row * L::KSTR + cc * EPC) = val;
  }
  for (int c = tid; c < (ICL_KT / 2) * CPR; c += nt) {
    const int pr = c / CPR, cc = c % CPR, key = k0 + 2 * pr;
    union { uint4 u; T e[EPC]; } a, b;
    a.u = make_uint4(0, 0, 0, 0);
    b.u = make_uint4(0, 0, 0, 0);
    if (key < valid) a.u = ldg16(vbase + (int64_t)key * p.v_st + cc * EPC);
    if (key + 1 < valid) b.u = ldg16(vbase + (int64_t)(key + 1) * p.v_st + cc * EPC);
    const int pos = (2 * pr & ~15) | vperm(2 * pr & 15);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      typedef T T2 __attribute__((ext_vector_type(2)));
      T2 pair;
      pair[0] = a.e[e];
      pair[1] = b.e[e];
      *(T2*)(lds_vt + (cc * EPC + e) * L::VSTR + pos) = pair;
    }
  }
}

template <typename T, int NW>
__global__ __launch_bounds__(NW * 64) void icl_fwd_kernel(IclParams p) {
  typedef IclLds<T> L;
  typedef typename OpVec<T, 8>::type Op8;
  __shared__ __attribute__((aligned(16))) T lds_k[L::K_ELEMS];
  __shared__ __attribute__((aligned(16))) T lds_vt[L::V_ELEMS];

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = work % p.nqb;
  const int nh = work / p.nqb;
  const int h = nh % p.H, n = nh / p.H;

  int valid = p.Tkv;
  if (p.valid) {
    valid = p.valid[p.valid_n == 1 ? 0 : n];
    valid = valid < 0 ? 0 : (valid > p.Tkv ? p.Tkv : valid);
  }

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 31, hh = lane >> 5;
  const int qi = qb * (32 * NW) + wave * 32 + lr;
  const bool qok = qi < p.Tq;
  const bool wave_active = qb * (32 * NW) + wave * 32 < p.Tq;

  const T* qbase = (const T*)p.q + n * p.q_sn + h * p.q_sh;
  const T* kbase = (const T*)p.k + n * p.k_sn + h * p.k_sh;
  const T* vbase = (const T*)p.v + n * p.v_sn + h * p.v_sh;

  Op8 qop[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    Op8 z = {};
    qop[s] = qok ? *(const Op8*)(qbase + (int64_t)qi * p.q_st + 16 * s + 8 * hh) : z;
  }

  f32x16 o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m_run = TA_NEG_INF, l_run = 0.f;
  const float sc = p.sc;

  const int ntiles = (valid + ICL_KT - 1) / ICL_KT;
  for (int t = 0; t < ntiles; ++t) {
    const int k0 = t * ICL_KT;
    if (t > 0) __syncthreads();
    icl_fill<T>(p, lds_k, lds_vt, kbase, vbase, k0, valid);
    __syncthreads();
    if (!wave_active) continue;

    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) {
        Op8 a = *(const Op8*)(lds_k + (kb * 32 + lr) * L::KSTR + 16 * sl + 8 * hh);
        s[kb] = mfma32x32x16(a, qop[sl], s[kb]);
      }
    }
    if (k0 + ICL_KT > valid) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= valid) s[kb][r] = TA_NEG_INF;
        }
    }
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = xor_max(mx, 32);
    const float m_new = fmaxf(m_run, mx);
    if (wave_any((m_new - m_run) * sc > ICL_LAZY)) {
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * sc);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      m_run = m_new;
    }
    const float nm = -m_run * sc;
    Op8 pop[2][2];
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = __builtin_amdgcn_exp2f(fmaf(s[kb][r], sc, nm));
        lsum += pr;
        pop[kb][r >> 3][r & 7] = from_f32<T>(pr);
      }
    l_run += lsum;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          Op8 a = *(const Op8*)(lds_vt + (db * 32 + lr) * L::VSTR + kb * 32 + 16 * m + 8 * hh);
          o[db] = mfma32x32x16(a, pop[kb][m], o[db]);
        }
  }

  if (!qok) return;
  const float lt = xor_sum(l_run, 32);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  T* orow = (T*)p.o + n * p.o_sn + h * p.o_sh + (int64_t)qi * p.o_st;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      typename OpVec<T, 4>::type ov;
#pragma unroll
      for (int r = 0; r < 4; ++r) ov[r] = from_f32<T>(o[db][4 * j + r] * inv);
      *(typename OpVec<T, 4>::type*)(orow + 32 * db + 8 * j + 4 * hh) = ov;
    }
}

}  // namespace

// Host launcher (called from the C ABI in abi.cpp).
int tabicl_launch_icl_fwd(const void* q, const void* k, const void* v, const int32_t* valid,
                          int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq,
                          int64_t Tkv, int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn,
                          int64_t k_sh, int64_t k_st, int64_t v_sn, int64_t v_sh, int64_t v_st,
                          int64_t o_sn, int64_t o_sh, int64_t o_st, float scale, int dtype,
                          hipStream_t stream) {
  constexpr int NW = 4;
  IclParams p;
  p.q = q; p.k = k; p.v = v; p.o = out;
  p.valid = valid; p.valid_n = (int)valid_n;
  p.N = (int)N; p.H = (int)H; p.Tq = (int)Tq; p.Tkv = (int)Tkv;
  p.nqb = (int)((Tq + 32 * NW - 1) / (32 * NW));
  p.q_sn = q_sn; p.q_sh = q_sh; p.q_st = q_st;
  p.k_sn = k_sn; p.k_sh = k_sh; p.k_st = k_st;
  p.v_sn = v_sn; p.v_sh = v_sh; p.v_st = v_st;
  p.o_sn = o_sn; p.o_sh = o_sh; p.o_st = o_st;
  p.sc = scale * TA_LOG2E;
  const int64_t nblk = N * H * (int64_t)p.nqb;
  if (dtype == 0)
    hipLaunchKernelGGL((icl_fwd_kernel<bf16, NW>), dim3((unsigned)nblk), dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((icl_fwd_kernel<float, NW>), dim3((unsigned)nblk), dim3(NW * 64), 0, stream, p);
  return (int)hipGetLastError();
}
