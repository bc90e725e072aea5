// Dataset-wise in-context attention over cached train-row K/V, head_dim 64 (gfx950).
//
// Math (the Splash hook of the reference, results/tpu_patch.diff:123-155, 95-102): per (n, h),
//   O = softmax(scale * Q K^T + mask) V,  mask[j] = -inf for key j >= valid,
// fp32 scores and softmax, probabilities cast to the value dtype before the PV product.
//
// Work decomposition: one workgroup = (n, h, block of NW * QW queries); each wave owns QW = 32 * QC
// queries (QC column blocks of 32). Keys stream through LDS in tiles of KT = 64, double buffered:
// the global loads of tile t+1 are issued into registers before tile t is computed and written to
// the other LDS buffer afterwards, so one barrier per tile suffices and the load latency hides
// behind the MFMA/softmax work. K is stored row-major [key][d], V transposed [d][key] with the key
// order permuted inside each 16-key group so that every MFMA operand is one 16-byte LDS read.
// Per tile and wave:
//   S^T (keys x queries) = K Q^T      v_mfma_f32_32x32x16_bf16, 2 key blocks x 4 d-slices x QC
//   online softmax in registers       lane l owns query l%32 of each column block; the two lanes
//                                     l, l^32 holding a query are combined with v_permlane32_swap
//   O^T (d x queries)   += V^T P^T    2 d-blocks x 4 key-slices x QC; P^T is the S^T accumulator
//                                     layout converted to bf16 in place (no shuffles)
// The running max is updated lazily: the accumulators are rescaled only when the tile max exceeds
// the running max by more than 2^8 (so p <= 256 otherwise); exact because O and l always share
// the same reference max.
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
  // key split: nsplit > 1 writes unnormalised partials (O, m, l) per split to the workspace
  int nsplit;
  float* ws_o;   // [nsplit][N*H][Tq][64]
  float* ws_ml;  // [nsplit][N*H][Tq][2]
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
template <typename T, int NT> struct Stage {
  static constexpr int EPC = IclLds<T>::EPC, CPR = IclLds<T>::CPR;
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
    typedef IclLds<T> L;
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

template <typename T, int QC> struct IclState {
  typedef typename OpVec<T, 8>::type Op8;
  Op8 qop[QC][4];
  f32x16 o[QC][2];
  float m_run[QC], l_run[QC];
};

// One key tile: S^T = K Q^T, online softmax, O^T += V^T P^T. MASK: the tile crosses `valid`.
template <typename T, int QC, bool MASK>
__device__ __forceinline__ void icl_tile(IclState<T, QC>& st, const T* lk, const T* lv, int k0,
                                         int valid, float sc, int lr, int hh) {
  typedef IclLds<T> L;
  typedef typename OpVec<T, 8>::type Op8;
  f32x16 s[QC][2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int qc = 0; qc < QC; ++qc)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[qc][kb][r] = 0.f;
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) {
      const Op8 a = *(const Op8*)(lk + (kb * 32 + lr) * L::KSTR + 16 * sl + 8 * hh);
#pragma unroll
      for (int qc = 0; qc < QC; ++qc) s[qc][kb] = mfma32x32x16(a, st.qop[qc][sl], s[qc][kb]);
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
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.o[qc][db][r] *= alpha;
      st.m_run[qc] = m_new;
    }
    const float nm = -st.m_run[qc] * sc;
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          pop[qc][kb][m][j] = from_f32<T>(__builtin_amdgcn_exp2f(fmaf(s[qc][kb][8 * m + j], sc, nm)));
        lsum = psum8(pop[qc][kb][m], lsum);
      }
    st.l_run[qc] += lsum;
  }

#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Op8 a = *(const Op8*)(lv + vt_off(db * 32 + lr, kb * 32 + 16 * m + 8 * hh, L::VSTR));
#pragma unroll
        for (int qc = 0; qc < QC; ++qc) st.o[qc][db] = mfma32x32x16(a, pop[qc][kb][m], st.o[qc][db]);
      }
}

template <typename T, int NW, int QC>
__global__ __launch_bounds__(NW * 64) void icl_fwd_kernel(IclParams p) {
  typedef IclLds<T> L;
  typedef typename OpVec<T, 8>::type Op8;
  constexpr int NT = NW * 64;
  constexpr int QW = 32 * QC;
  __shared__ __attribute__((aligned(16))) T lds_k[2][L::K_ELEMS];
  __shared__ __attribute__((aligned(16))) T lds_vt[2][L::V_ELEMS];

  // work item = (n, h, split, query block); consecutive items share (n, h) and stay on one XCD
  const int work = xcd_remap(blockIdx.x, gridDim.x);
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

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 31, hh = lane >> 5;
  const int qw0 = qb * (QW * NW) + wave * QW;

  const T* qbase = (const T*)p.q + n * p.q_sn + h * p.q_sh;
  const T* kbase = (const T*)p.k + n * p.k_sn + h * p.k_sh;
  const T* vbase = (const T*)p.v + n * p.v_sn + h * p.v_sh;

  IclState<T, QC> st;
#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    const int qi = qw0 + qc * 32 + lr;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      Op8 z = {};
      st.qop[qc][s] = qi < p.Tq ? *(const Op8*)(qbase + (int64_t)qi * p.q_st + 16 * s + 8 * hh) : z;
    }
    st.m_run[qc] = TA_NEG_INF;
    st.l_run[qc] = 0.f;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.o[qc][db][r] = 0.f;
  }
  const float sc = p.sc;

  // this split's tiles [t0, t1) of the ceil(valid / KT) key tiles
  const int ntiles = (valid + ICL_KT - 1) / ICL_KT;
  const int per = (ntiles + p.nsplit - 1) / p.nsplit;
  const int t0 = min(split * per, ntiles), t1 = min(t0 + per, ntiles);
  if (t1 > t0) {
    Stage<T, NT> stg;
    stg.load(kbase, vbase, p.k_st, p.v_st, t0 * ICL_KT, valid);
    stg.store(lds_k[0], lds_vt[0]);
    __syncthreads();
    // all tiles but the last one of the range: no key past `valid`
    for (int t = t0; t + 1 < t1; ++t) {
      const int k0 = t * ICL_KT, buf = (t - t0) & 1;
      stg.load(kbase, vbase, p.k_st, p.v_st, k0 + ICL_KT, valid);
      icl_tile<T, QC, false>(st, lds_k[buf], lds_vt[buf], k0, valid, sc, lr, hh);
      stg.store(lds_k[buf ^ 1], lds_vt[buf ^ 1]);
      __syncthreads();
    }
    const int tl = t1 - 1, bl = (tl - t0) & 1;
    if (t1 == ntiles)
      icl_tile<T, QC, true>(st, lds_k[bl], lds_vt[bl], tl * ICL_KT, valid, sc, lr, hh);
    else
      icl_tile<T, QC, false>(st, lds_k[bl], lds_vt[bl], tl * ICL_KT, valid, sc, lr, hh);
  }

  if (p.nsplit > 1) {
    // unnormalised partial result of this key range: O (fp32), running max m and sum l
#pragma unroll
    for (int qc = 0; qc < QC; ++qc) {
      const float lt = lane_pair_sum(st.l_run[qc]);
      const int qi = qw0 + qc * 32 + lr;
      if (qi < p.Tq) {
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
        if (hh == 0) *(float2*)(p.ws_ml + row * 2) = make_float2(st.m_run[qc], lt);
      }
    }
    return;
  }

#pragma unroll
  for (int qc = 0; qc < QC; ++qc) {
    const float lt = lane_pair_sum(st.l_run[qc]);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int qi = qw0 + qc * 32 + lr;
    if (qi < p.Tq) {
      T* orow = (T*)p.o + n * p.o_sn + h * p.o_sh + (int64_t)qi * p.o_st;
#pragma unroll
      for (int db = 0; db < 2; ++db)
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

// Combines the per-split partials: m* = max_s m_s, w_s = 2^((m_s - m*) sc),
// O = sum_s w_s O_s / sum_s w_s l_s (0 when no split saw a valid key). One thread per 4 outputs.
template <typename T>
__global__ __launch_bounds__(256) void icl_merge_kernel(IclParams p) {
  const int64_t rows = (int64_t)p.N * p.H * p.Tq;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * (ICL_D / 4)) return;
  const int64_t row = idx / (ICL_D / 4);
  const int c4 = (int)(idx % (ICL_D / 4)) * 4;
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
    const float w = __builtin_amdgcn_exp2f((ml.x - mstar) * p.sc);
    const float4 o = *(const float4*)(p.ws_o + ((int64_t)s * rows + row) * ICL_D + c4);
    acc.x += w * o.x; acc.y += w * o.y; acc.z += w * o.z; acc.w += w * o.w;
    l += w * ml.y;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int64_t nh = row / p.Tq;
  const int qi = (int)(row % p.Tq);
  const int n = (int)(nh / p.H), h = (int)(nh % p.H);
  T* dst = (T*)p.o + n * p.o_sn + h * p.o_sh + (int64_t)qi * p.o_st + c4;
  typename OpVec<T, 4>::type ov;
  ov[0] = from_f32<T>(acc.x * inv); ov[1] = from_f32<T>(acc.y * inv);
  ov[2] = from_f32<T>(acc.z * inv); ov[3] = from_f32<T>(acc.w * inv);
  *(typename OpVec<T, 4>::type*)dst = ov;
}

template <typename T, int NW, int QC>
int blocks_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_fwd_kernel<T, NW, QC>, NW * 64, 0) != hipSuccess)
    return 1;
  return n > 0 ? n : 1;
}

// Number of key splits that best fills whole rounds of resident workgroups:
// minimises ceil(items * S / slots) / S over S = 1..4, each split keeping >= 8 key tiles.
template <typename T, int NW, int QC>
int pick_splits(int64_t items, int64_t Tkv) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 1;
  const int64_t slots = (int64_t)cus * blocks_per_cu<T, NW, QC>();
  const int64_t tiles = (Tkv + ICL_KT - 1) / ICL_KT;
  int best = 1;
  double best_cost = (double)((items + slots - 1) / slots);
  for (int s = 2; s <= 4; ++s) {
    if (tiles / s < 8) break;
    const double cost = (double)((items * s + slots - 1) / slots) / s;
    if (cost < best_cost - 1e-9) { best = s; best_cost = cost; }
  }
  return best;
}

template <typename T, int NW, int QC>
int64_t workspace_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv) {
  const int64_t nqb = (Tq + 32 * QC * NW - 1) / (32 * QC * NW);
  const int s = pick_splits<T, NW, QC>(N * H * nqb, Tkv);
  return s > 1 ? (int64_t)s * N * H * Tq * (ICL_D + 2) * (int64_t)sizeof(float) : 0;
}

template <typename T, int NW, int QC>
void launch(const IclParams& p0, void* ws, int64_t ws_bytes, hipStream_t stream) {
  IclParams p = p0;
  p.nqb = (p.Tq + 32 * QC * NW - 1) / (32 * QC * NW);
  const int64_t rows = (int64_t)p.N * p.H * p.Tq;
  p.nsplit = pick_splits<T, NW, QC>((int64_t)p.N * p.H * p.nqb, p.Tkv);
  if (p.nsplit > 1 && (ws == nullptr || ws_bytes < (int64_t)p.nsplit * rows * (ICL_D + 2) * 4)) p.nsplit = 1;
  p.ws_o = (float*)ws;
  p.ws_ml = p.ws_o + (p.nsplit > 1 ? (int64_t)p.nsplit * rows * ICL_D : 0);
  const int64_t nblk = (int64_t)p.N * p.H * p.nsplit * p.nqb;
  hipLaunchKernelGGL((icl_fwd_kernel<T, NW, QC>), dim3((unsigned)nblk), dim3(NW * 64), 0, stream, p);
  if (p.nsplit > 1) {
    const int64_t threads = rows * (ICL_D / 4);
    hipLaunchKernelGGL((icl_merge_kernel<T>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
  }
}

}  // namespace

// Host launchers (called from the C ABI in abi.hip).
int64_t tabicl_launch_icl_ws_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int dtype) {
  return dtype == 0 ? workspace_bytes<bf16, 4, 2>(N, H, Tq, Tkv) : workspace_bytes<float, 4, 1>(N, H, Tq, Tkv);
}

int tabicl_launch_icl_fwd(const void* q, const void* k, const void* v, const int32_t* valid,
                          int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq,
                          int64_t Tkv, int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn,
                          int64_t k_sh, int64_t k_st, int64_t v_sn, int64_t v_sh, int64_t v_st,
                          int64_t o_sn, int64_t o_sh, int64_t o_st, float scale, int dtype,
                          void* ws, int64_t ws_bytes, hipStream_t stream) {
  IclParams p;
  p.q = q; p.k = k; p.v = v; p.o = out;
  p.valid = valid; p.valid_n = (int)valid_n;
  p.N = (int)N; p.H = (int)H; p.Tq = (int)Tq; p.Tkv = (int)Tkv;
  p.nqb = 0;
  p.q_sn = q_sn; p.q_sh = q_sh; p.q_st = q_st;
  p.k_sn = k_sn; p.k_sh = k_sh; p.k_st = k_st;
  p.v_sn = v_sn; p.v_sh = v_sh; p.v_st = v_st;
  p.o_sn = o_sn; p.o_sh = o_sh; p.o_st = o_st;
  p.sc = scale * TA_LOG2E;
  p.nsplit = 1; p.ws_o = nullptr; p.ws_ml = nullptr;
  if (dtype == 0)
    launch<bf16, 4, 2>(p, ws, ws_bytes, stream);
  else
    launch<float, 4, 1>(p, ws, ws_bytes, stream);
  return (int)hipGetLastError();
}
