// Backward of the d = 64 ICL attention (gfx950): per (n, h),
//   O = softmax(S) V,  S = scale q k^T + b,
// keys at or past valid[n] masked, b an optional additive fp32 key mask (one row for every n, or one
// per n) added to the scaled scores, as the reference's gradient path computes it (autograd through
// _tiled_online_sdpa, results/tpu_patch.diff:158-193, which upstream's attention takes for calls with
// a gradient, diff:263-270). With P recomputed in fp32:
//   dP = dO V^T,  D = sum over the 64 dims of dO * O,  dS = P (dP - D) (cast to the input dtype),
//   dq = scale dS k,  dk = scale dS^T q,  dv = cast(P)^T dO   (fp32 accumulation).
// Two kernels, no atomics, every gradient element written once:
//   ib_dq_kernel   workgroup = ((n, h), 64 queries), wave = 16 queries. Keys stream through LDS in
//                  64-key tiles: a first sweep takes each query's softmax statistics (row maximum m and
//                  log2 of the sum, log2 units) and D, written to the workspace; a second sweep forms
//                  e = exp2(x - m), dP - D (the dP product's accumulator input is -D) and dq' += e (dP - D) k,
//                  scaled by 1 / l at the end.
//   ib_dkdv_kernel workgroup = ((n, h), 64 keys), wave = 16 keys. Queries stream through LDS in 64-row
//                  tiles with their statistics and -D: P, dP - D, dS, dk' and dv.
// MFMA 16x16x16 (bf16) or 4 x 16x16x4 (fp32) in the lane layout of mfma16x16x16 (common.h); the head's
// 64 dims are four 16-dim chunks of every contraction over dims. Transposed operands come from
// ds_read_b64_tr_b16 on the row-major tiles (bf16) or from transposed copies (fp32). All tensors are
// contiguous [N, H, T, 64].
#include "common.h"
#include "launch.h"

namespace {

constexpr int IB_D = 64;
constexpr int IB_NW = 4;          // waves per workgroup
constexpr int IB_T = 16 * IB_NW;  // rows per workgroup and per tile
constexpr float IB_BIAS_FLOOR = -1e37f;

struct IbParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  const int32_t* valid;
  int valid_n;
  const float* bias;
  int64_t bias_sn;
  int bias_n;
  int N, H, Tq, Tkv;
  float scale;
  // per (n, h, query), [N * H][Tq] each: row maximum m of x = S log2e (log2 units; +inf for a row with
  // no visible key), log2 of the sum of exp2(x - m), and D
  float* mx;
  float* lg;
  float* dd;
};

template <typename T> struct IbTile {
  static constexpr int PAD = 16 / sizeof(T);
  static constexpr int RSTR = IB_D + PAD;  // row-major tile: 64 dims per row
  static constexpr int TSTR = IB_T + PAD;  // transposed copy (fp32 only): 64 rows of IB_T
  static constexpr int T_ELEMS = sizeof(T) == 2 ? 4 : IB_D * TSTR;
};

__device__ __forceinline__ int ib_valid(const IbParams& p, int n) {
  if (!p.valid) return p.Tkv;
  const int v = p.valid[p.valid_n == 1 ? 0 : n];
  return v < 0 ? 0 : (v > p.Tkv ? p.Tkv : v);
}

// Additive term of key `key` in log2 units: -inf at or past the valid length; the key mask times log2e,
// floored at -1e37 (a row masked everywhere stays uniform, as the reference's finite fill gives it).
__device__ __forceinline__ float ib_b2(const IbParams& p, int n, int key, int valid) {
  if (key >= valid) return TA_NEG_INF;
  if (!p.bias) return 0.f;
  return fmaxf(p.bias[(int64_t)(p.bias_n == 1 ? 0 : n) * p.bias_sn + key] * TA_LOG2E, IB_BIAS_FLOOR);
}

// Rows r0 .. r0 + 63 of a [rows, 64] slab into a row-major tile (and, for fp32 with a non-null tcopy,
// its transposed copy); rows at or past lim are zero.
template <typename T>
__device__ __forceinline__ void ib_fill(const T* base, int r0, int lim, T* tile, T* tcopy) {
  typedef IbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  for (int u = threadIdx.x; u < IB_T * (IB_D / 4); u += IB_NW * 64) {
    const int row = u >> 4, c = (u & 15) * 4;
    Op4 x;
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = from_f32<T>(0.f);
    if (r0 + row < lim) x = *(const Op4*)(base + (int64_t)(r0 + row) * IB_D + c);
    *(Op4*)(tile + row * L::RSTR + c) = x;
    if constexpr (sizeof(T) == 4) {
      if (tcopy != nullptr) {
#pragma unroll
        for (int j = 0; j < 4; ++j) tcopy[(c + j) * L::TSTR + row] = x[j];
      }
    }
  }
}

// Row operand: dims 16 jd + 4 kap .. + 3 of tile row `row`.
template <typename T>
__device__ __forceinline__ typename OpVec<T, 4>::type ib_row(const T* tile, int row, int jd, int kap) {
  return *(const typename OpVec<T, 4>::type*)(tile + row * IbTile<T>::RSTR + 16 * jd + 4 * kap);
}

// Transposed operand A[i][4 kap + j] = tile[row0 + 4 kap + j][16 jd + i] for lane (i = l16, kap).
template <typename T>
__device__ __forceinline__ typename OpVec<T, 4>::type ib_rowT(const T* tile, const T* tcopy, int row0, int jd,
                                                             int l16, int kap) {
  typedef IbTile<T> L;
  if constexpr (sizeof(T) == 2) {
    const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(tile + (row0 + 4 * kap + (l16 >> 2)) * L::RSTR + 16 * jd + 4 * (l16 & 3)));
    return __builtin_bit_cast(bf16x4, t);
  } else {
    return *(const f32x4*)(tcopy + (16 * jd + l16) * L::TSTR + row0 + 4 * kap);
  }
}

// x = S^T log2e + b2 of keys 16 kt + 4 kap + r (tile rows) against this lane's query: the score
// product over the four dim chunks.
template <typename T>
__device__ __forceinline__ f32x4 ib_scores_t(const T* lk, const float* lb2, const typename OpVec<T, 4>::type (&qop)[4],
                                             int kt, int l16, int kap, float c) {
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) s = mfma16x16x16(ib_row<T>(lk, 16 * kt + l16, jd, kap), qop[jd], s);
  const f32x4 b2 = *(const f32x4*)(lb2 + 16 * kt + 4 * kap);
  f32x4 x;
#pragma unroll
  for (int r = 0; r < 4; ++r) x[r] = fmaf(s[r], c, b2[r]);
  return x;
}

template <typename T>
__global__ __launch_bounds__(IB_NW * 64) void ib_dq_kernel(IbParams p) {
  typedef IbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  __shared__ __attribute__((aligned(16))) T lk[IB_T * L::RSTR];
  __shared__ __attribute__((aligned(16))) T lkt[L::T_ELEMS];
  __shared__ __attribute__((aligned(16))) T lv[IB_T * L::RSTR];
  __shared__ __attribute__((aligned(16))) float lb2[IB_T];

  const int nqb = (p.Tq + IB_T - 1) / IB_T;
  const int nh = blockIdx.x / nqb, qb = blockIdx.x % nqb, n = nh / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int valid = ib_valid(p, n);
  const int qi = qb * IB_T + wave * 16 + l16;
  const bool qok = qi < p.Tq;
  const T* qrow = (const T*)p.q + ((int64_t)nh * p.Tq + qi) * IB_D;
  const T* kbase = (const T*)p.k + (int64_t)nh * p.Tkv * IB_D;
  const T* vbase = (const T*)p.v + (int64_t)nh * p.Tkv * IB_D;
  const float c = p.scale * TA_LOG2E;

  // q and dO operands of query qi (B operands of S^T = K Q^T and dP^T = V dO^T), D
  Op4 qop[4], dop[4];
  float dsum = 0.f;
#pragma unroll
  for (int jd = 0; jd < 4; ++jd)
#pragma unroll
    for (int j = 0; j < 4; ++j) { qop[jd][j] = from_f32<T>(0.f); dop[jd][j] = from_f32<T>(0.f); }
  if (qok) {
    const int64_t orow = ((int64_t)nh * p.Tq + qi) * IB_D;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
      qop[jd] = *(const Op4*)(qrow + 16 * jd + 4 * kap);
      dop[jd] = *(const Op4*)((const T*)p.dout + orow + 16 * jd + 4 * kap);
      const Op4 ov = *(const Op4*)((const T*)p.o + orow + 16 * jd + 4 * kap);
#pragma unroll
      for (int j = 0; j < 4; ++j) dsum += to_f32<T>(dop[jd][j]) * to_f32<T>(ov[j]);
    }
  }
  dsum = xor_sum(dsum, 16);
  dsum = xor_sum(dsum, 32);

  const int ntiles = (valid + IB_T - 1) / IB_T;
  // sweep 1: the statistics over this lane's keys (4 per 16-key block), merged over the lane quad
  float m = TA_NEG_INF, l = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    ib_fill<T>(kbase, t * IB_T, valid, lk, (T*)nullptr);
    for (int j = threadIdx.x; j < IB_T; j += IB_NW * 64) lb2[j] = ib_b2(p, n, t * IB_T + j, valid);
    __syncthreads();
    f32x4 x[4];
    float tm = TA_NEG_INF;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      x[kt] = ib_scores_t<T>(lk, lb2, qop, kt, l16, kap, c);
#pragma unroll
      for (int r = 0; r < 4; ++r) tm = fmaxf(tm, x[kt][r]);
    }
    if (tm > TA_NEG_INF) {
      const float mn = fmaxf(m, tm);
      float s = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s += __builtin_amdgcn_exp2f(x[kt][r] - mn);
      l = l * __builtin_amdgcn_exp2f(m - mn) + s;
      m = mn;
    }
  }
  const float mq = quad_max(m);
  const float lt = quad_sum(m > TA_NEG_INF ? l * __builtin_amdgcn_exp2f(m - mq) : 0.f);  // >= 1, or 0: no key
  const float lgl = lt > 0.f ? __builtin_amdgcn_logf(lt) : 0.f;
  const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;

  // sweep 2: dq' l = sum e (dP - D) k with e = exp2(x - m)
  f32x4 acc[4];
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) acc[jd] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 cnd = {-dsum, -dsum, -dsum, -dsum};
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    ib_fill<T>(kbase, t * IB_T, valid, lk, lkt);
    ib_fill<T>(vbase, t * IB_T, valid, lv, (T*)nullptr);
    for (int j = threadIdx.x; j < IB_T; j += IB_NW * 64) lb2[j] = ib_b2(p, n, t * IB_T + j, valid);
    __syncthreads();
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const f32x4 x = ib_scores_t<T>(lk, lb2, qop, kt, l16, kap, c);
      f32x4 dp = cnd;
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) dp = mfma16x16x16(ib_row<T>(lv, 16 * kt + l16, jd, kap), dop[jd], dp);
      Op4 ds;
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[r] = from_f32<T>(__builtin_amdgcn_exp2f(x[r] - mq) * dp[r]);
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) acc[jd] = mfma16x16x16(ib_rowT<T>(lk, lkt, 16 * kt, jd, l16, kap), ds, acc[jd]);
      __builtin_amdgcn_sched_barrier(0);  // one key block at a time: hoisting them costs registers
    }
  }
  if (qok) {
    const float ysc = p.scale * inv;
    T* dqrow = (T*)p.dq + ((int64_t)nh * p.Tq + qi) * IB_D;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
      Op4 out;
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = from_f32<T>(acc[jd][r] * ysc);
      *(Op4*)(dqrow + 16 * jd + 4 * kap) = out;
    }
    if (kap == 0) {
      const int64_t s = (int64_t)nh * p.Tq + qi;
      p.mx[s] = lt > 0.f ? mq : __builtin_inff();  // no visible key: P = 0 in the dk / dv kernel
      p.lg[s] = lgl;
      p.dd[s] = dsum;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(IB_NW * 64) void ib_dkdv_kernel(IbParams p) {
  typedef IbTile<T> L;
  typedef typename OpVec<T, 4>::type Op4;
  __shared__ __attribute__((aligned(16))) T lq[IB_T * L::RSTR];
  __shared__ __attribute__((aligned(16))) T lqt[L::T_ELEMS];
  __shared__ __attribute__((aligned(16))) T ld[IB_T * L::RSTR];
  __shared__ __attribute__((aligned(16))) T ldt[L::T_ELEMS];
  __shared__ __attribute__((aligned(16))) float lmx[IB_T];
  __shared__ __attribute__((aligned(16))) float llg[IB_T];
  __shared__ __attribute__((aligned(16))) float lnd[IB_T];

  const int nkb = (p.Tkv + IB_T - 1) / IB_T;
  const int nh = blockIdx.x / nkb, kb = blockIdx.x % nkb, n = nh / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int valid = ib_valid(p, n);
  const int kj = kb * IB_T + wave * 16 + l16;
  const float c = p.scale * TA_LOG2E;
  f32x4 dk[4], dv[4];
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) dk[jd] = dv[jd] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (kb * IB_T < valid) {  // uniform over the workgroup; keys past valid get zero gradients
    // k and V operands of key kj (B operands of S = Q K^T and dP = dO V^T) and its b2
    Op4 kop[4], vop[4];
#pragma unroll
    for (int jd = 0; jd < 4; ++jd)
#pragma unroll
      for (int j = 0; j < 4; ++j) { kop[jd][j] = from_f32<T>(0.f); vop[jd][j] = from_f32<T>(0.f); }
    if (kj < valid) {
      const int64_t row = ((int64_t)nh * p.Tkv + kj) * IB_D;
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) {
        kop[jd] = *(const Op4*)((const T*)p.k + row + 16 * jd + 4 * kap);
        vop[jd] = *(const Op4*)((const T*)p.v + row + 16 * jd + 4 * kap);
      }
    }
    const float b2 = ib_b2(p, n, kj, valid);
    const T* qbase = (const T*)p.q + (int64_t)nh * p.Tq * IB_D;
    const T* dbase = (const T*)p.dout + (int64_t)nh * p.Tq * IB_D;
    const int ntiles = (p.Tq + IB_T - 1) / IB_T;
    for (int t = 0; t < ntiles; ++t) {
      __syncthreads();
      ib_fill<T>(qbase, t * IB_T, p.Tq, lq, lqt);
      ib_fill<T>(dbase, t * IB_T, p.Tq, ld, ldt);
      for (int j = threadIdx.x; j < IB_T; j += IB_NW * 64) {
        const int qi = t * IB_T + j;
        const int64_t s = (int64_t)nh * p.Tq + qi;
        // queries past Tq: m = +inf gives P = 0
        lmx[j] = qi < p.Tq ? p.mx[s] : __builtin_inff();
        llg[j] = qi < p.Tq ? p.lg[s] : 0.f;
        lnd[j] = qi < p.Tq ? -p.dd[s] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int qs = 0; qs < 4; ++qs) {
        // S[query 16 qs + 4 kap + r][key kj], dP - D likewise (the accumulator input is -D)
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
        f32x4 dp = *(const f32x4*)(lnd + 16 * qs + 4 * kap);
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) {
          s = mfma16x16x16(ib_row<T>(lq, 16 * qs + l16, jd, kap), kop[jd], s);
          dp = mfma16x16x16(ib_row<T>(ld, 16 * qs + l16, jd, kap), vop[jd], dp);
        }
        const f32x4 ms = *(const f32x4*)(lmx + 16 * qs + 4 * kap);
        const f32x4 ls = *(const f32x4*)(llg + 16 * qs + 4 * kap);
        Op4 pt, ds;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f((fmaf(s[r], c, b2) - ms[r]) - ls[r]);
          pt[r] = from_f32<T>(pr);
          ds[r] = from_f32<T>(pr * dp[r]);
        }
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) {
          dv[jd] = mfma16x16x16(ib_rowT<T>(ld, ldt, 16 * qs, jd, l16, kap), pt, dv[jd]);
          dk[jd] = mfma16x16x16(ib_rowT<T>(lq, lqt, 16 * qs, jd, l16, kap), ds, dk[jd]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if (kj < p.Tkv) {
    const int64_t row = ((int64_t)nh * p.Tkv + kj) * IB_D;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
      Op4 ok, ov;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ok[r] = from_f32<T>(dk[jd][r] * p.scale);
        ov[r] = from_f32<T>(dv[jd][r]);
      }
      *(Op4*)((T*)p.dk + row + 16 * jd + 4 * kap) = ok;
      *(Op4*)((T*)p.dv + row + 16 * jd + 4 * kap) = ov;
    }
  }
}

int64_t ib_part_bytes(int64_t N, int64_t H, int64_t Tq) { return (N * H * Tq * 4 + 255) / 256 * 256; }

}  // namespace

int64_t tabicl_launch_icl_bwd_ws_bytes(int64_t N, int64_t H, int64_t Tq) { return 3 * ib_part_bytes(N, H, Tq); }

int tabicl_launch_icl_bwd(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                          const float* bias, int64_t bias_n, int64_t bias_sn, const void* o, const void* dout,
                          void* dq, void* dk, void* dv, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, float scale,
                          int dtype, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (ws_bytes < tabicl_launch_icl_bwd_ws_bytes(N, H, Tq)) return (int)hipErrorInvalidValue;
  IbParams p;
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout;
  p.dq = dq; p.dk = dk; p.dv = dv;
  p.valid = valid; p.valid_n = (int)valid_n;
  p.bias = bias; p.bias_sn = bias_sn; p.bias_n = (int)bias_n;
  p.N = (int)N; p.H = (int)H; p.Tq = (int)Tq; p.Tkv = (int)Tkv;
  p.scale = scale;
  const int64_t part = ib_part_bytes(N, H, Tq);
  p.mx = (float*)ws;
  p.lg = (float*)((char*)ws + part);
  p.dd = (float*)((char*)ws + 2 * part);
  const int64_t nqb = (Tq + IB_T - 1) / IB_T, nkb = (Tkv + IB_T - 1) / IB_T;
  const dim3 block(IB_NW * 64);
  if (nqb > 0) {
    if (dtype == 0)
      hipLaunchKernelGGL(ib_dq_kernel<bf16>, dim3((unsigned)(N * H * nqb)), block, 0, stream, p);
    else
      hipLaunchKernelGGL(ib_dq_kernel<float>, dim3((unsigned)(N * H * nqb)), block, 0, stream, p);
  }
  if (nkb > 0) {
    if (dtype == 0)
      hipLaunchKernelGGL(ib_dkdv_kernel<bf16>, dim3((unsigned)(N * H * nkb)), block, 0, stream, p);
    else
      hipLaunchKernelGGL(ib_dkdv_kernel<float>, dim3((unsigned)(N * H * nkb)), block, 0, stream, p);
  }
  return (int)hipGetLastError();
}
