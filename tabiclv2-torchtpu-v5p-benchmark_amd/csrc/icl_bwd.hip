// Backward of the d = 64 ICL attention (gfx950): per (n, h),
//   O = softmax(S) V,  S = scale q k^T + b,
// keys at or past valid[n] masked, b an optional additive fp32 key mask (one row for every n, or one
// per n) added to the scaled scores, as the reference's gradient path computes it (autograd through
// _tiled_online_sdpa, results/tpu_patch.diff:158-193, which upstream's attention takes for calls with
// a gradient, diff:263-270). With P recomputed in fp32:
//   dP = dO V^T,  D = sum over the 64 dims of dO * O,  dS = P (dP - D) (cast to the input dtype),
//   dq = scale dS k,  dk = scale dS^T q,  dv = cast(P)^T dO   (fp32 accumulation).
// Two kernels per call, no atomics, every gradient element written once: a dq kernel (one workgroup per
// (n, h) and query block, keys streamed through LDS) that also leaves each query's softmax statistics
// and D in the workspace, then a dk / dv kernel (one workgroup per (n, h) and key block, queries and
// their statistics streamed through LDS).
//   bf16: ic_dq_kernel / ic_dkdv_kernel, 16x16x32 products with two 16-row blocks per wave; the
//         statistics come from the forward (tabicl_icl_fwd_stats) when the call has no key mask.
//   fp32: ib_dq_kernel / ib_dkdv_kernel, 4 x 16x16x4 products in the lane layout of mfma16x16x16
//         (common.h), one 16-row block per wave, transposed operands from transposed LDS copies.
// All tensors are contiguous [N, H, T, 64].
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
  // optional (bf16, no key mask): the forward's per-query (m, l) [N * H][Tq][2], m in log2 units, l
  // the sum of exp2(x - m); with it the dq kernel skips its statistics sweep
  const float* stat;
};

// fp32 tiles: row-major [64 rows][64 dims] and the transposed copy [64 dims][64 rows], each row padded
// by 16 bytes
constexpr int IB_RSTR = IB_D + 4;
constexpr int IB_TSTR = IB_T + 4;

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

// Rows r0 .. r0 + 63 of a [rows, 64] fp32 slab into a row-major tile (and, with a non-null tcopy, its
// transposed copy); rows at or past lim are zero.
__device__ __forceinline__ void ib_fill(const float* base, int r0, int lim, float* tile, float* tcopy) {
  for (int u = threadIdx.x; u < IB_T * (IB_D / 4); u += IB_NW * 64) {
    const int row = u >> 4, c = (u & 15) * 4;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if (r0 + row < lim) x = *(const f32x4*)(base + (int64_t)(r0 + row) * IB_D + c);
    *(f32x4*)(tile + row * IB_RSTR + c) = x;
    if (tcopy != nullptr) {
#pragma unroll
      for (int j = 0; j < 4; ++j) tcopy[(c + j) * IB_TSTR + row] = x[j];
    }
  }
}

// Row operand: dims 16 jd + 4 kap .. + 3 of tile row `row`.
__device__ __forceinline__ f32x4 ib_row(const float* tile, int row, int jd, int kap) {
  return *(const f32x4*)(tile + row * IB_RSTR + 16 * jd + 4 * kap);
}

// Transposed operand A[i][4 kap + j] = tile[row0 + 4 kap + j][16 jd + i] for lane (i = l16, kap), from
// the transposed copy.
__device__ __forceinline__ f32x4 ib_rowT(const float* tcopy, int row0, int jd, int l16, int kap) {
  return *(const f32x4*)(tcopy + (16 * jd + l16) * IB_TSTR + row0 + 4 * kap);
}

// x = S^T log2e + b2 of keys 16 kt + 4 kap + r (tile rows) against this lane's query: the score
// product over the four dim chunks.
__device__ __forceinline__ f32x4 ib_scores_t(const float* lk, const float* lb2, const f32x4 (&qop)[4], int kt,
                                             int l16, int kap, float c) {
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) s = mfma16x16x16(ib_row(lk, 16 * kt + l16, jd, kap), qop[jd], s);
  const f32x4 b2 = *(const f32x4*)(lb2 + 16 * kt + 4 * kap);
  f32x4 x;
#pragma unroll
  for (int r = 0; r < 4; ++r) x[r] = fmaf(s[r], c, b2[r]);
  return x;
}

// fp32 dq: workgroup = ((n, h), 64 queries), wave = 16 queries. Keys stream through LDS in 64-key tiles:
// a first sweep takes each query's softmax statistics (row maximum m and log2 of the sum, log2 units)
// and D, written to the workspace; a second sweep forms e = exp2(x - m), dP - D (the dP product's
// accumulator input is -D) and dq' += e (dP - D) k, scaled by 1 / l at the end.
__global__ __launch_bounds__(IB_NW * 64) void ib_dq_kernel(IbParams p) {
  typedef f32x4 Op4;
  __shared__ __attribute__((aligned(16))) float lk[IB_T * IB_RSTR];
  __shared__ __attribute__((aligned(16))) float lkt[IB_D * IB_TSTR];
  __shared__ __attribute__((aligned(16))) float lv[IB_T * IB_RSTR];
  __shared__ __attribute__((aligned(16))) float lb2[IB_T];

  const int nqb = (p.Tq + IB_T - 1) / IB_T;
  const int nh = blockIdx.x / nqb, qb = blockIdx.x % nqb, n = nh / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int valid = ib_valid(p, n);
  const int qi = qb * IB_T + wave * 16 + l16;
  const bool qok = qi < p.Tq;
  const float* qrow = (const float*)p.q + ((int64_t)nh * p.Tq + qi) * IB_D;
  const float* kbase = (const float*)p.k + (int64_t)nh * p.Tkv * IB_D;
  const float* vbase = (const float*)p.v + (int64_t)nh * p.Tkv * IB_D;
  const float c = p.scale * TA_LOG2E;

  // q and dO operands of query qi (B operands of S^T = K Q^T and dP^T = V dO^T), D
  Op4 qop[4], dop[4];
  float dsum = 0.f;
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) qop[jd] = dop[jd] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (qok) {
    const int64_t orow = ((int64_t)nh * p.Tq + qi) * IB_D;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
      qop[jd] = *(const Op4*)(qrow + 16 * jd + 4 * kap);
      dop[jd] = *(const Op4*)((const float*)p.dout + orow + 16 * jd + 4 * kap);
      const Op4 ov = *(const Op4*)((const float*)p.o + orow + 16 * jd + 4 * kap);
#pragma unroll
      for (int j = 0; j < 4; ++j) dsum += dop[jd][j] * ov[j];
    }
  }
  dsum = xor_sum(dsum, 16);
  dsum = xor_sum(dsum, 32);

  const int ntiles = (valid + IB_T - 1) / IB_T;
  // sweep 1: the statistics over this lane's keys (4 per 16-key block), merged over the lane quad
  float m = TA_NEG_INF, l = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    ib_fill(kbase, t * IB_T, valid, lk, nullptr);
    for (int j = threadIdx.x; j < IB_T; j += IB_NW * 64) lb2[j] = ib_b2(p, n, t * IB_T + j, valid);
    __syncthreads();
    f32x4 x[4];
    float tm = TA_NEG_INF;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      x[kt] = ib_scores_t(lk, lb2, qop, kt, l16, kap, c);
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
    ib_fill(kbase, t * IB_T, valid, lk, lkt);
    ib_fill(vbase, t * IB_T, valid, lv, nullptr);
    for (int j = threadIdx.x; j < IB_T; j += IB_NW * 64) lb2[j] = ib_b2(p, n, t * IB_T + j, valid);
    __syncthreads();
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const f32x4 x = ib_scores_t(lk, lb2, qop, kt, l16, kap, c);
      f32x4 dp = cnd;
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) dp = mfma16x16x16(ib_row(lv, 16 * kt + l16, jd, kap), dop[jd], dp);
      Op4 ds;
#pragma unroll
      for (int r = 0; r < 4; ++r) ds[r] = __builtin_amdgcn_exp2f(x[r] - mq) * dp[r];
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) acc[jd] = mfma16x16x16(ib_rowT(lkt, 16 * kt, jd, l16, kap), ds, acc[jd]);
      __builtin_amdgcn_sched_barrier(0);  // one key block at a time: hoisting them costs registers
    }
  }
  if (qok) {
    const float ysc = p.scale * inv;
    float* dqrow = (float*)p.dq + ((int64_t)nh * p.Tq + qi) * IB_D;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
      Op4 out;
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = acc[jd][r] * ysc;
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

// fp32 dk / dv: workgroup = ((n, h), 64 keys), wave = 16 keys. Queries stream through LDS in 64-row tiles
// with their statistics and -D: P, dP - D, dS, dk' and dv.
__global__ __launch_bounds__(IB_NW * 64) void ib_dkdv_kernel(IbParams p) {
  typedef f32x4 Op4;
  __shared__ __attribute__((aligned(16))) float lq[IB_T * IB_RSTR];
  __shared__ __attribute__((aligned(16))) float lqt[IB_D * IB_TSTR];
  __shared__ __attribute__((aligned(16))) float ld[IB_T * IB_RSTR];
  __shared__ __attribute__((aligned(16))) float ldt[IB_D * IB_TSTR];
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
    for (int jd = 0; jd < 4; ++jd) kop[jd] = vop[jd] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (kj < valid) {
      const int64_t row = ((int64_t)nh * p.Tkv + kj) * IB_D;
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) {
        kop[jd] = *(const Op4*)((const float*)p.k + row + 16 * jd + 4 * kap);
        vop[jd] = *(const Op4*)((const float*)p.v + row + 16 * jd + 4 * kap);
      }
    }
    const float b2 = ib_b2(p, n, kj, valid);
    const float* qbase = (const float*)p.q + (int64_t)nh * p.Tq * IB_D;
    const float* dbase = (const float*)p.dout + (int64_t)nh * p.Tq * IB_D;
    const int ntiles = (p.Tq + IB_T - 1) / IB_T;
    for (int t = 0; t < ntiles; ++t) {
      __syncthreads();
      ib_fill(qbase, t * IB_T, p.Tq, lq, lqt);
      ib_fill(dbase, t * IB_T, p.Tq, ld, ldt);
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
          s = mfma16x16x16(ib_row(lq, 16 * qs + l16, jd, kap), kop[jd], s);
          dp = mfma16x16x16(ib_row(ld, 16 * qs + l16, jd, kap), vop[jd], dp);
        }
        const f32x4 ms = *(const f32x4*)(lmx + 16 * qs + 4 * kap);
        const f32x4 ls = *(const f32x4*)(llg + 16 * qs + 4 * kap);
        Op4 pt, ds;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f((fmaf(s[r], c, b2) - ms[r]) - ls[r]);
          pt[r] = pr;
          ds[r] = pr * dp[r];
        }
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) {
          dv[jd] = mfma16x16x16(ib_rowT(ldt, 16 * qs, jd, l16, kap), pt, dv[jd]);
          dk[jd] = mfma16x16x16(ib_rowT(lqt, 16 * qs, jd, l16, kap), ds, dk[jd]);
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
        ok[r] = dk[jd][r] * p.scale;
        ov[r] = dv[jd][r];
      }
      *(Op4*)((float*)p.dk + row + 16 * jd + 4 * kap) = ok;
      *(Op4*)((float*)p.dv + row + 16 * jd + 4 * kap) = ov;
    }
  }
}

// ---------------------------------------------------------------------------------------------------
// bf16 kernels: 16x16x32 products (v_mfma_f32_16x16x32_bf16: lane (l16, kap) holds A[l16][8 kap + j]
// and B[8 kap + j][l16], j = 0..7; result reg r = C[4 kap + r][l16]), two 16-row blocks per wave so
// that every LDS operand read feeds two products, 64-row tiles staged through registers into two LDS
// buffers (one barrier per tile). Workgroup = 4 waves x 32 rows.
constexpr int IC_RS = IB_D + 8;       // bf16 row stride of the LDS tiles: 144 bytes, b128 reads conflict-free
constexpr int IC_WR = 32;             // queries (dq) or keys (dk / dv) per wave
constexpr int IC_ROWS = IC_WR * IB_NW;

typedef unsigned ic_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned ic_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 ic_mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ic_zero8() { return __builtin_bit_cast(bf16x8, ic_u32x4{0u, 0u, 0u, 0u}); }

// [a | b] as one 8-element operand, assembled from whole 32-bit words (element-wise assembly of
// transposed-read results is miscompiled by this compiler).
template <typename V> __device__ __forceinline__ bf16x8 ic_cat(V a, V b) {
  const ic_u32x2 x = __builtin_bit_cast(ic_u32x2, a), y = __builtin_bit_cast(ic_u32x2, b);
  return __builtin_bit_cast(bf16x8, ic_u32x4{x[0], x[1], y[0], y[1]});
}

// Row operand: A[l16][8 kap + j] = tile[row0 + l16][col0 + 8 kap + j].
__device__ __forceinline__ bf16x8 ic_row(const bf16* tile, int row0, int col0, int l16, int kap) {
  return *(const bf16x8*)(tile + (row0 + l16) * IC_RS + col0 + 8 * kap);
}

// Transposed operand over two 16-row blocks ra, rb: A[l16][8 kap + j] = tile[ra + 4 kap + j][col0 + l16]
// for j < 4 and tile[rb + 4 kap + j - 4][col0 + l16] for j >= 4, the k-slot order of a B operand made
// of two 16x16 product results (rows 4 kap + r of each).
__device__ __forceinline__ bf16x8 ic_rowT2(const bf16* tile, int ra, int rb, int col0, int l16, int kap) {
  const int off = (4 * kap + (l16 >> 2)) * IC_RS + col0 + 4 * (l16 & 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + ra * IC_RS + off));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + rb * IC_RS + off));
  return ic_cat(a, b);
}

// A 64-row slab [rows, 64] staged in registers: thread t holds the 16-byte chunks t and t + 256 (row
// u / 8, dims 8 (u % 8) ..); rows at or past lim are zero.
struct IcStage {
  bf16x8 c[2];
};
__device__ __forceinline__ void ic_load(IcStage& s, const bf16* base, int r0, int lim) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = threadIdx.x + 256 * i, row = u >> 3;
    s.c[i] = r0 + row < lim ? *(const bf16x8*)(base + (int64_t)(r0 + row) * IB_D + (u & 7) * 8) : ic_zero8();
  }
}
__device__ __forceinline__ void ic_store(const IcStage& s, bf16* tile) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = threadIdx.x + 256 * i;
    *(bf16x8*)(tile + (u >> 3) * IC_RS + (u & 7) * 8) = s.c[i];
  }
}

// dq: workgroup = ((n, h), 128 queries), wave = 32 queries (blocks b = 0, 1). Sweep 1 takes the
// statistics over 64-key tiles (S^T = K Q^T, K rows from LDS, q in registers); sweep 2 forms
// dS^T = e (dP^T - D) per key block and dq^T += K^T dS^T over key-block pairs. Stores dq and, per
// query, m (+inf for a row with no visible key), log2 l and -D for the dk / dv kernel (before sweep 2,
// so that they are not held across it: the launch bound of three workgroups per CU, i.e. three waves
// per SIMD, leaves 168 VGPRs).
// FS: the statistics come from the forward (p.stat; no key mask), there is no sweep 1, and the score
// product starts from -(m + log2 l) / c, so that exp2(S^T c) is P itself (one fma fewer per score).
template <bool FS>
__global__ __launch_bounds__(IB_NW * 64, 3) void ic_dq_kernel(IbParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lk[2][IB_T * IC_RS];
  __shared__ __attribute__((aligned(16))) bf16 lv[2][IB_T * IC_RS];
  __shared__ __attribute__((aligned(16))) float lb2[2][IB_T];

  const int nqb = (p.Tq + IC_ROWS - 1) / IC_ROWS;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  const int nh = item / nqb, qblk = item % nqb, n = nh / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int valid = ib_valid(p, n);
  const int q0 = qblk * IC_ROWS + wave * IC_WR;
  const int64_t rbase = (int64_t)nh * p.Tq;
  const bf16* kbase = (const bf16*)p.k + (int64_t)nh * p.Tkv * IB_D;
  const bf16* vbase = (const bf16*)p.v + (int64_t)nh * p.Tkv * IB_D;
  const float c = p.scale * TA_LOG2E;

  // q and dO of query q0 + 16 b + l16, dims 32 cc + 8 kap .. + 7 (B operands of S^T and dP^T), and -D
  bf16x8 qop[2][2], dop[2][2];
  float nd[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int qi = q0 + 16 * b + l16;
    float part = 0.f;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      qop[b][cc] = dop[b][cc] = ic_zero8();
      if (qi < p.Tq) {
        const int64_t off = (rbase + qi) * IB_D + 32 * cc + 8 * kap;
        qop[b][cc] = *(const bf16x8*)((const bf16*)p.q + off);
        dop[b][cc] = *(const bf16x8*)((const bf16*)p.dout + off);
        const bf16x8 ov = *(const bf16x8*)((const bf16*)p.o + off);
#pragma unroll
        for (int j = 0; j < 8; ++j) part += (float)dop[b][cc][j] * (float)ov[j];
      }
    }
    part = xor_sum(part, 16);
    nd[b] = -xor_sum(part, 32);
  }

  const int ntiles = (valid + IB_T - 1) / IB_T;
  const int tid = threadIdx.x;
  IcStage sk, sv;
  float b2r = 0.f;
  float mq[2], inv[2], lgv[2];
  if constexpr (FS) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int qi = q0 + 16 * b + l16;
      const float2 ml = qi < p.Tq ? *(const float2*)(p.stat + (rbase + qi) * 2) : make_float2(0.f, 1.f);
      const bool any = ml.y > 0.f;
      mq[b] = any ? ml.x : __builtin_inff();  // no visible key: P = 0 in the dk / dv kernel
      lgv[b] = any ? __builtin_amdgcn_logf(ml.y) : 0.f;
      inv[b] = 1.f;
    }
  } else {
  // sweep 1: per lane and query block, the running max and sum over the lane's keys (4 per key block)
  float m[2] = {TA_NEG_INF, TA_NEG_INF}, l[2] = {0.f, 0.f};
  if (ntiles > 0) {
    ic_load(sk, kbase, 0, valid);
    if (tid < IB_T) b2r = ib_b2(p, n, tid, valid);
  }
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    ic_store(sk, lk[buf]);
    if (tid < IB_T) lb2[buf][tid] = b2r;
    __syncthreads();
    if (t + 1 < ntiles) {
      ic_load(sk, kbase, (t + 1) * IB_T, valid);
      if (tid < IB_T) b2r = ib_b2(p, n, (t + 1) * IB_T + tid, valid);
    }
    f32x4 x[2][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const bf16x8 a0 = ic_row(lk[buf], 16 * kb, 0, l16, kap), a1 = ic_row(lk[buf], 16 * kb, 32, l16, kap);
      const f32x4 b2 = *(const f32x4*)(lb2[buf] + 16 * kb + 4 * kap);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const f32x4 s = ic_mfma(a1, qop[b][1], ic_mfma(a0, qop[b][0], f32x4{0.f, 0.f, 0.f, 0.f}));
#pragma unroll
        for (int r = 0; r < 4; ++r) x[b][kb][r] = fmaf(s[r], c, b2[r]);
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float tm = TA_NEG_INF;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) tm = fmaxf(tm, x[b][kb][r]);
      if (tm > TA_NEG_INF) {
        const float mn = fmaxf(m[b], tm);
        float s = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) s += __builtin_amdgcn_exp2f(x[b][kb][r] - mn);
        l[b] = l[b] * __builtin_amdgcn_exp2f(m[b] - mn) + s;
        m[b] = mn;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    mq[b] = quad_max(m[b]);
    const float lt = quad_sum(m[b] > TA_NEG_INF ? l[b] * __builtin_amdgcn_exp2f(m[b] - mq[b]) : 0.f);
    inv[b] = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;
    lgv[b] = lt > 0.f ? __builtin_amdgcn_logf(lt) : 0.f;
    if (!(lt > 0.f)) mq[b] = __builtin_inff();  // no visible key: P = 0 in the dk / dv kernel
  }
  __syncthreads();  // sweep 2 refills both buffers
  }
  // FS: the score product's start value -(m + log2 l) / c (rows past Tq hold m = 0, l = 1)
  float s0[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) s0[b] = FS ? -(mq[b] + lgv[b]) / c : 0.f;
  // the statistics for the dk / dv kernel, stored before the sweep (not kept live across it)
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int qi = q0 + 16 * b + l16;
    if (qi < p.Tq && kap == 0) {
      p.mx[rbase + qi] = mq[b];
      p.lg[rbase + qi] = lgv[b];
      p.dd[rbase + qi] = nd[b];
    }
  }

  // sweep 2: dq^T l = sum over keys of K^T e (dP^T - D), e = exp2(x - m)
  f32x4 acc[2][4];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) acc[b][jd] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (ntiles > 0) {
    ic_load(sk, kbase, 0, valid);
    ic_load(sv, vbase, 0, valid);
    if (tid < IB_T) b2r = ib_b2(p, n, tid, valid);
  }
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    ic_store(sk, lk[buf]);
    ic_store(sv, lv[buf]);
    if (tid < IB_T) lb2[buf][tid] = b2r;
    __syncthreads();
    if (t + 1 < ntiles) {
      ic_load(sk, kbase, (t + 1) * IB_T, valid);
      ic_load(sv, vbase, (t + 1) * IB_T, valid);
      if (tid < IB_T) b2r = ib_b2(p, n, (t + 1) * IB_T + tid, valid);
    }
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
      bf16x4 ds[2][2];  // [key block of the pair][query block]
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kb = 2 * kp + h;
        const bf16x8 a0 = ic_row(lk[buf], 16 * kb, 0, l16, kap), a1 = ic_row(lk[buf], 16 * kb, 32, l16, kap);
        const bf16x8 v0 = ic_row(lv[buf], 16 * kb, 0, l16, kap), v1 = ic_row(lv[buf], 16 * kb, 32, l16, kap);
        const f32x4 b2 = *(const f32x4*)(lb2[buf] + 16 * kb + 4 * kap);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const f32x4 s = ic_mfma(a1, qop[b][1], ic_mfma(a0, qop[b][0], f32x4{s0[b], s0[b], s0[b], s0[b]}));
          const f32x4 dp = ic_mfma(v1, dop[b][1], ic_mfma(v0, dop[b][0], f32x4{nd[b], nd[b], nd[b], nd[b]}));
          f32x4 e;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if constexpr (FS)
              e[r] = __builtin_amdgcn_exp2f(fmaf(s[r], c, b2[r])) * dp[r];
            else
              e[r] = __builtin_amdgcn_exp2f(fmaf(s[r], c, b2[r]) - mq[b]) * dp[r];
          }
          ds[h][b] = cvt_bf16x4(e);
        }
      }
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) {
        const bf16x8 at = ic_rowT2(lk[buf], 32 * kp, 32 * kp + 16, 16 * jd, l16, kap);
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[b][jd] = ic_mfma(at, ic_cat(ds[0][b], ds[1][b]), acc[b][jd]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int qi = q0 + 16 * b + l16;
    if (qi < p.Tq) {
      const float ysc = p.scale * inv[b];
      bf16* dqrow = (bf16*)p.dq + (rbase + qi) * IB_D;
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) *(bf16x4*)(dqrow + 16 * jd + 4 * kap) = cvt_bf16x4(acc[b][jd] * ysc);
    }
  }
}

// dk / dv: workgroup = ((n, h), 128 keys), wave = 32 keys (blocks h = 0, 1), k and V in registers.
// 64-query tiles of q, dO (rows) and their statistics stream through LDS: S = Q K^T and dP = dO V^T per
// query block, P = exp2(S c + b - m - log2 l), dS = P (dP - D), then over query-block pairs
// dv^T += dO^T P and dk^T += Q^T dS (transposed operands from ds_read_b64_tr_b16). Without a key mask
// the exponent takes -(m + log2 l) as one value; with one (HB) it subtracts m and log2 l in turn, as the
// statistics were taken: a row at the mask's floor (m ~ -1e37) would lose log2 l in the sum.
template <bool HB>
__global__ __launch_bounds__(IB_NW * 64) void ic_dkdv_kernel(IbParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lq[2][IB_T * IC_RS];
  __shared__ __attribute__((aligned(16))) bf16 ld[2][IB_T * IC_RS];
  __shared__ __attribute__((aligned(16))) float lms[2][IB_T];
  __shared__ __attribute__((aligned(16))) float lnd[2][IB_T];
  __shared__ __attribute__((aligned(16))) float llg[HB ? 2 : 1][HB ? IB_T : 4];

  const int nkb = (p.Tkv + IC_ROWS - 1) / IC_ROWS;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  const int nh = item / nkb, kblk = item % nkb, n = nh / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kap = lane >> 4;
  const int tid = threadIdx.x;
  const int valid = ib_valid(p, n);
  const int k0 = kblk * IC_ROWS + wave * IC_WR;
  const float c = p.scale * TA_LOG2E;
  f32x4 dkt[2][4], dvt[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) dkt[h][jd] = dvt[h][jd] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (kblk * IC_ROWS < valid) {  // uniform over the workgroup; keys past valid get zero gradients
    // k and V of key k0 + 16 h + l16, dims 32 cc + 8 kap .. + 7 (B operands of S and dP), and its b
    bf16x8 kop[2][2], vop[2][2];
    float b2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kj = k0 + 16 * h + l16;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        kop[h][cc] = vop[h][cc] = ic_zero8();
        if (kj < valid) {
          const int64_t off = ((int64_t)nh * p.Tkv + kj) * IB_D + 32 * cc + 8 * kap;
          kop[h][cc] = *(const bf16x8*)((const bf16*)p.k + off);
          vop[h][cc] = *(const bf16x8*)((const bf16*)p.v + off);
        }
      }
      b2[h] = ib_b2(p, n, kj, valid);
    }
    const int64_t rbase = (int64_t)nh * p.Tq;
    const bf16* qbase = (const bf16*)p.q + rbase * IB_D;
    const bf16* dbase = (const bf16*)p.dout + rbase * IB_D;
    const int ntiles = (p.Tq + IB_T - 1) / IB_T;
    // per-query values: threads 0-63 -(m + log2 l) / c, the score product's start value (m with HB;
    // past Tq -inf, +inf with HB: P = 0), threads 64-127 -D, threads 128-191 log2 l (HB)
    constexpr int NST = HB ? 3 * IB_T : 2 * IB_T;
    auto stat = [&](int q0) -> float {
      const int qi = q0 + (tid & 63);
      const bool in = qi < p.Tq;
      if (tid < IB_T) {
        if (HB) return in ? p.mx[rbase + qi] : __builtin_inff();
        return in ? -(p.mx[rbase + qi] + p.lg[rbase + qi]) / c : TA_NEG_INF;
      }
      if (tid < 2 * IB_T) return in ? p.dd[rbase + qi] : 0.f;
      return in ? p.lg[rbase + qi] : 0.f;
    };
    IcStage sq, sd;
    float st = 0.f;
    if (ntiles > 0) {
      ic_load(sq, qbase, 0, p.Tq);
      ic_load(sd, dbase, 0, p.Tq);
      if (tid < NST) st = stat(0);
    }
    for (int t = 0; t < ntiles; ++t) {
      const int buf = t & 1;
      ic_store(sq, lq[buf]);
      ic_store(sd, ld[buf]);
      if (tid < IB_T) lms[buf][tid] = st;
      else if (tid < 2 * IB_T) lnd[buf][tid - IB_T] = st;
      else if (HB && tid < NST) llg[HB ? buf : 0][tid - 2 * IB_T] = st;
      __syncthreads();
      if (t + 1 < ntiles) {
        ic_load(sq, qbase, (t + 1) * IB_T, p.Tq);
        ic_load(sd, dbase, (t + 1) * IB_T, p.Tq);
        if (tid < NST) st = stat((t + 1) * IB_T);
      }
#pragma unroll
      for (int qp = 0; qp < 2; ++qp) {
        bf16x4 pt[2][2], dst[2][2];  // [query block of the pair][key block]
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const int qb = 2 * qp + g;
          const bf16x8 aq0 = ic_row(lq[buf], 16 * qb, 0, l16, kap), aq1 = ic_row(lq[buf], 16 * qb, 32, l16, kap);
          const bf16x8 ad0 = ic_row(ld[buf], 16 * qb, 0, l16, kap), ad1 = ic_row(ld[buf], 16 * qb, 32, l16, kap);
          const f32x4 ms = *(const f32x4*)(lms[buf] + 16 * qb + 4 * kap);
          const f32x4 ndv = *(const f32x4*)(lnd[buf] + 16 * qb + 4 * kap);
          f32x4 lgq = {0.f, 0.f, 0.f, 0.f};
          if constexpr (HB) lgq = *(const f32x4*)(llg[buf] + 16 * qb + 4 * kap);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const f32x4 s = ic_mfma(aq1, kop[h][1], ic_mfma(aq0, kop[h][0], HB ? f32x4{0.f, 0.f, 0.f, 0.f} : ms));
            const f32x4 dp = ic_mfma(ad1, vop[h][1], ic_mfma(ad0, vop[h][0], ndv));
            f32x4 pr, dsv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if constexpr (HB)
                pr[r] = __builtin_amdgcn_exp2f((fmaf(s[r], c, b2[h]) - ms[r]) - lgq[r]);
              else
                pr[r] = __builtin_amdgcn_exp2f(fmaf(s[r], c, b2[h]));
              dsv[r] = pr[r] * dp[r];
            }
            pt[g][h] = cvt_bf16x4(pr);
            dst[g][h] = cvt_bf16x4(dsv);
          }
        }
#pragma unroll
        for (int jd = 0; jd < 4; ++jd) {
          const bf16x8 atd = ic_rowT2(ld[buf], 32 * qp, 32 * qp + 16, 16 * jd, l16, kap);
          const bf16x8 atq = ic_rowT2(lq[buf], 32 * qp, 32 * qp + 16, 16 * jd, l16, kap);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            dvt[h][jd] = ic_mfma(atd, ic_cat(pt[0][h], pt[1][h]), dvt[h][jd]);
            dkt[h][jd] = ic_mfma(atq, ic_cat(dst[0][h], dst[1][h]), dkt[h][jd]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kj = k0 + 16 * h + l16;
    if (kj < p.Tkv) {
      const int64_t row = ((int64_t)nh * p.Tkv + kj) * IB_D;
#pragma unroll
      for (int jd = 0; jd < 4; ++jd) {
        *(bf16x4*)((bf16*)p.dk + row + 16 * jd + 4 * kap) = cvt_bf16x4(dkt[h][jd] * p.scale);
        *(bf16x4*)((bf16*)p.dv + row + 16 * jd + 4 * kap) = cvt_bf16x4(dvt[h][jd]);
      }
    }
  }
}

int64_t ib_part_bytes(int64_t N, int64_t H, int64_t Tq) { return (N * H * Tq * 4 + 255) / 256 * 256; }

}  // namespace

int64_t tabicl_launch_icl_bwd_ws_bytes(int64_t N, int64_t H, int64_t Tq) { return 3 * ib_part_bytes(N, H, Tq); }

int tabicl_launch_icl_bwd(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                          const float* bias, int64_t bias_n, int64_t bias_sn, const void* o, const void* dout,
                          const float* stat,
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
  p.stat = stat;
  const int64_t part = ib_part_bytes(N, H, Tq);
  p.mx = (float*)ws;
  p.lg = (float*)((char*)ws + part);
  p.dd = (float*)((char*)ws + 2 * part);
  const dim3 block(IB_NW * 64);
  if (dtype == 0) {
    const int64_t nqb = (Tq + IC_ROWS - 1) / IC_ROWS, nkb = (Tkv + IC_ROWS - 1) / IC_ROWS;
    if (nqb > 0) {
      if (p.stat && !bias)
        hipLaunchKernelGGL(ic_dq_kernel<true>, dim3((unsigned)(N * H * nqb)), block, 0, stream, p);
      else
        hipLaunchKernelGGL(ic_dq_kernel<false>, dim3((unsigned)(N * H * nqb)), block, 0, stream, p);
    }
    if (nkb > 0) {
      if (bias)
        hipLaunchKernelGGL(ic_dkdv_kernel<true>, dim3((unsigned)(N * H * nkb)), block, 0, stream, p);
      else
        hipLaunchKernelGGL(ic_dkdv_kernel<false>, dim3((unsigned)(N * H * nkb)), block, 0, stream, p);
    }
  } else {
    const int64_t nqb = (Tq + IB_T - 1) / IB_T, nkb = (Tkv + IB_T - 1) / IB_T;
    if (nqb > 0) hipLaunchKernelGGL(ib_dq_kernel, dim3((unsigned)(N * H * nqb)), block, 0, stream, p);
    if (nkb > 0) hipLaunchKernelGGL(ib_dkdv_kernel, dim3((unsigned)(N * H * nkb)), block, 0, stream, p);
  }
  return (int)hipGetLastError();
}
