// Row LayerNorm of the layers around the attention (gfx950): the pre-norms of the column, row and ICL
// blocks and the out / final norms of the cached-KV query (upstream's SafeLayerNorm,
// results/tpu_patch.diff:1385-1397, which normalises in its weights' dtype: fp32 here).
//
//   y = (s - mean(s)) * rsqrt(var(s) + eps) * w + b,   s = x (+ r when a residual is given)
//
// per row of W = 128 or 512 values, x / r fp32 or bf16, w / b fp32, y fp32 or bf16; mean and the
// biased variance in fp32 from the row held in registers (two passes, no Welford). With a residual the
// sum s is rounded to the input dtype, written out, and that rounded value is normalised: the result of
// `s = x + r` followed by LayerNorm(s) in the input dtype.
//
// Layout: a lane holds 16-byte chunks of one row (4 fp32 or 8 bf16 values); G = min(64, W / chunk)
// lanes share a row, so a wave covers 64 / G rows per step (W = 128: 2 rows fp32, 4 rows bf16).
// Grid-stride over row groups, two steps in flight per wave. HBM-bound: read W (or 2W) values and
// write W (or 2W) values per row, once.
#include "common.h"
#include "launch.h"

namespace {

template <typename T> struct Chunk16;
template <> struct Chunk16<float> { typedef f32x4 type; static constexpr int N = 4; };
template <> struct Chunk16<bf16> { typedef bf16x8 type; static constexpr int N = 8; };

template <typename T>
__device__ __forceinline__ void chunk_to_f32(typename Chunk16<T>::type c, float* v) {
#pragma unroll
  for (int i = 0; i < Chunk16<T>::N; ++i) v[i] = (float)c[i];
}

// Store N fp32 values as TO at p (N = 4 or 8: 16 or 32 bytes for fp32 / 8 or 16 bytes for bf16).
template <typename TO, int N>
__device__ __forceinline__ void store_vals(TO* p, const float* v) {
  if constexpr (sizeof(TO) == 4) {
#pragma unroll
    for (int i = 0; i < N; i += 4) *(f32x4*)(p + i) = f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]};
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) *(bf16x4*)(p + i) = cvt_bf16x4(f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]});
  }
}

template <int G>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

constexpr int LN_NT = 256;
constexpr int LN_STEPS = 2;  // row groups per wave per iteration (loads in flight)

template <typename TI, typename TO, int W, bool RES>
__global__ __launch_bounds__(LN_NT) void ln_kernel(const TI* __restrict__ x, const TI* __restrict__ r, TI* xs,
                                                  const float* __restrict__ w, const float* __restrict__ b,
                                                  TO* __restrict__ y, int64_t rows, float eps) {
  typedef typename Chunk16<TI>::type CT;
  constexpr int C = Chunk16<TI>::N;
  constexpr int G = (W / C) < 64 ? (W / C) : 64;  // lanes per row
  constexpr int K = W / (C * G);                  // chunks per lane
  constexpr int RPW = 64 / G;                     // rows per wave and step
  static_assert(W % (C * G) == 0 && K >= 1, "row width must be a multiple of the chunk layout");
  const int lane = threadIdx.x & 63, li = lane % G, sub = lane / G;
  const int64_t wave = (int64_t)blockIdx.x * (LN_NT / 64) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (LN_NT / 64);

  // this lane's weight and bias values (columns (j G + li) C .. + C - 1)
  float wv[K][C], bv[K][C];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const int col = (j * G + li) * C;
#pragma unroll
    for (int i = 0; i < C; i += 4) {
      const f32x4 ww = w ? *(const f32x4*)(w + col + i) : f32x4{1.f, 1.f, 1.f, 1.f};
      const f32x4 bb = b ? *(const f32x4*)(b + col + i) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        wv[j][i + t] = ww[t];
        bv[j][i + t] = bb[t];
      }
    }
  }
  const float inv_w = 1.0f / (float)W;
  for (int64_t base = wave * LN_STEPS * RPW; base < rows; base += nwaves * LN_STEPS * RPW) {
    CT cx[LN_STEPS][K], cr[LN_STEPS][K];
#pragma unroll
    for (int s = 0; s < LN_STEPS; ++s) {
      const int64_t row = base + s * RPW + sub;
      if (row < rows) {
#pragma unroll
        for (int j = 0; j < K; ++j) {
          const int64_t off = row * W + (j * G + li) * C;
          cx[s][j] = *(const CT*)(x + off);
          if (RES) cr[s][j] = *(const CT*)(r + off);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < LN_STEPS; ++s) {
      const int64_t row = base + s * RPW + sub;
      const bool ok = row < rows;
      float v[K][C];
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        chunk_to_f32<TI>(cx[s][j], v[j]);
        if (RES) {
          float rv[C];
          chunk_to_f32<TI>(cr[s][j], rv);
          CT sc;
#pragma unroll
          for (int i = 0; i < C; ++i) {
            sc[i] = (TI)(v[j][i] + rv[i]);  // the sum in the input dtype, as `x + r` gives it
            v[j][i] = (float)sc[i];
          }
          if (ok) *(CT*)(xs + row * W + (j * G + li) * C) = sc;
        }
#pragma unroll
        for (int i = 0; i < C; ++i) sum += v[j][i];
      }
      const float mean = group_sum<G>(sum) * inv_w;
      float sq = 0.f;
#pragma unroll
      for (int j = 0; j < K; ++j)
#pragma unroll
        for (int i = 0; i < C; ++i) {
          const float d = v[j][i] - mean;
          sq = __builtin_fmaf(d, d, sq);
        }
      const float rstd = __builtin_amdgcn_rsqf(group_sum<G>(sq) * inv_w + eps);
      if (ok) {
#pragma unroll
        for (int j = 0; j < K; ++j) {
          float o[C];
#pragma unroll
          for (int i = 0; i < C; ++i) o[i] = __builtin_fmaf((v[j][i] - mean) * rstd, wv[j][i], bv[j][i]);
          store_vals<TO, C>(y + row * W + (j * G + li) * C, o);
        }
      }
    }
  }
}

template <typename TI, typename TO, int W>
void launch_ln(const void* x, const void* r, void* xs, const float* w, const float* b, void* y, int64_t rows, float eps,
               hipStream_t stream) {
  constexpr int C = Chunk16<TI>::N;
  constexpr int G = (W / C) < 64 ? (W / C) : 64;
  constexpr int64_t rows_per_block = (int64_t)(LN_NT / 64) * (64 / G) * LN_STEPS;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t need = (rows + rows_per_block - 1) / rows_per_block;
  const int64_t cap = (int64_t)(cus > 0 ? cus : 256) * 8;  // eight workgroups per CU, grid-stride beyond
  const unsigned grid = (unsigned)(need < cap ? need : cap);
  if (r)
    hipLaunchKernelGGL((ln_kernel<TI, TO, W, true>), dim3(grid), dim3(LN_NT), 0, stream, (const TI*)x,
                       (const TI*)r, (TI*)xs, w, b, (TO*)y, rows, eps);
  else
    hipLaunchKernelGGL((ln_kernel<TI, TO, W, false>), dim3(grid), dim3(LN_NT), 0, stream, (const TI*)x,
                       (const TI*)nullptr, (TI*)nullptr, w, b, (TO*)y, rows, eps);
}

template <int W>
void launch_ln_w(const void* x, const void* r, void* xs, const float* w, const float* b, void* y, int64_t rows,
                 float eps, int in_dtype, int out_dtype, hipStream_t stream) {
  if (in_dtype == 0 && out_dtype == 0) launch_ln<bf16, bf16, W>(x, r, xs, w, b, y, rows, eps, stream);
  else if (in_dtype == 0) launch_ln<bf16, float, W>(x, r, xs, w, b, y, rows, eps, stream);
  else if (out_dtype == 0) launch_ln<float, bf16, W>(x, r, xs, w, b, y, rows, eps, stream);
  else launch_ln<float, float, W>(x, r, xs, w, b, y, rows, eps, stream);
}

}  // namespace

int tabicl_launch_layer_norm(const void* x, const void* r, void* xs, const float* w, const float* b, void* y,
                             int64_t rows, int64_t width, float eps, int in_dtype, int out_dtype, hipStream_t stream) {
  if (rows <= 0) return 0;
  if (width == 128)
    launch_ln_w<128>(x, r, xs, w, b, y, rows, eps, in_dtype, out_dtype, stream);
  else
    launch_ln_w<512>(x, r, xs, w, b, y, rows, eps, in_dtype, out_dtype, stream);
  return (int)hipGetLastError();
}
