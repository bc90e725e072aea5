// Key-only additive masks read as key-validity lengths, on the device (no host synchronisation).
//
// Upstream tabicl turns a tensor train size into an additive mask over the keys whenever its
// device-specific fast path does not apply (results/tpu_patch.diff:1526-1542: 0 for key positions
// below the train size, finfo(dtype).min from there on), and row / column callers build key-padding
// masks of the same form (diff:1253-1271). Such a mask is a *prefix mask* of length v >= 1:
//   bias[j] == 0 for j < v,   bias[j] <= -1e30 for j >= v.
// Next to a key with bias 0, a key with bias <= -1e30 gets softmax weight exp(s - m - 1e30), which
// is exactly 0 in fp32 for every finite score, so attention under a prefix mask equals attention over
// the first v keys. The fast kernels (fixed-reference sweeps) take v as their valid length; a row
// whose mask is anything else (a finite non-zero term, or every key masked) is flagged, and a kernel
// that adds the bias term by term computes it instead.
#include "common.h"
#include "launch.h"

namespace {

constexpr float KM_MASKED = -1e30f;
constexpr int KM_THREADS = 1024;
constexpr int KM_UNROLL = 8;  // independent loads per thread in flight

// One workgroup of 1024 threads per output row r (bias row nb == 1 ? 0 : r, valid entry valid_n == 1 ?
// 0 : r), one pass over the row: v = first position whose bias is not 0 (NaN counts as not 0) and u =
// last position whose bias is not <= -1e30 (NaN counts); the row is a prefix mask of length v when
// v >= 1 and u < v (every entry from v on is <= -1e30; the zeros before v make u = v - 1).
// out_valid[r] = min(v, valid) when ok, else the plain valid length (or L). Each thread keeps 8 loads
// in flight per round (a row of 45,000 entries is 6 rounds), no early exit.
__global__ __launch_bounds__(KM_THREADS) void key_prefix_kernel(const float* bias, int64_t bias_sr, int nb, int L,
                                                                const int32_t* valid, int valid_n, int32_t* out_valid,
                                                                int32_t* out_ok) {
  __shared__ int s_first;
  __shared__ int s_last;
  const int r = blockIdx.x;
  const float* row = bias + (nb == 1 ? 0 : (int64_t)r * bias_sr);
  if (threadIdx.x == 0) {
    s_first = L;
    s_last = -1;
  }
  int first = L, last = -1;
  for (int j0 = 0; j0 < L; j0 += KM_THREADS * KM_UNROLL) {
    float x[KM_UNROLL];
#pragma unroll
    for (int u = 0; u < KM_UNROLL; ++u) {
      const int j = j0 + u * KM_THREADS + (int)threadIdx.x;
      x[u] = j < L ? row[j] : KM_MASKED;
    }
#pragma unroll
    for (int u = 0; u < KM_UNROLL; ++u) {
      const int j = j0 + u * KM_THREADS + (int)threadIdx.x;
      if (j < L) {
        if (!(x[u] == 0.f)) first = min(first, j);
        if (!(x[u] <= KM_MASKED)) last = max(last, j);
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    first = min(first, __shfl_xor(first, m, 64));
    last = max(last, __shfl_xor(last, m, 64));
  }
  __syncthreads();  // s_first / s_last initialised
  if ((threadIdx.x & 63) == 0) {
    atomicMin(&s_first, first);
    atomicMax(&s_last, last);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int v = s_first;
    int vl = L;
    if (valid) {
      vl = valid[valid_n == 1 ? 0 : r];
      vl = vl < 0 ? 0 : (vl > L ? L : vl);
    }
    const int ok = v >= 1 && s_last < v;
    out_ok[r] = ok;
    out_valid[r] = ok ? (v < vl ? v : vl) : vl;
  }
}

}  // namespace

int tabicl_launch_key_prefix(const float* bias, int64_t bias_sr, int64_t nb, int64_t L, const int32_t* valid,
                             int64_t valid_n, int64_t rows, int32_t* out_valid, int32_t* out_ok,
                             hipStream_t stream) {
  hipLaunchKernelGGL(key_prefix_kernel, dim3((unsigned)rows), dim3(KM_THREADS), 0, stream, bias, bias_sr, (int)nb, (int)L,
                     valid, (int)valid_n, out_valid, out_ok);
  return (int)hipGetLastError();
}
