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

// One workgroup per output row r (bias row nb == 1 ? 0 : r, valid entry valid_n == 1 ? 0 : r):
// v = first position whose bias is not 0 (NaN counts as not 0), ok = v >= 1 and every bias from v on
// is <= -1e30. out_valid[r] = min(v, valid) when ok, else the plain valid length (or L).
__global__ __launch_bounds__(256) void key_prefix_kernel(const float* bias, int64_t bias_sr, int nb, int L,
                                                         const int32_t* valid, int valid_n, int32_t* out_valid,
                                                         int32_t* out_ok) {
  __shared__ int s_first;
  __shared__ int s_bad;
  const int r = blockIdx.x;
  const float* row = bias + (nb == 1 ? 0 : (int64_t)r * bias_sr);
  if (threadIdx.x == 0) {
    s_first = L;
    s_bad = 0;
  }
  __syncthreads();
  int first = L;
  for (int j = threadIdx.x; j < L; j += blockDim.x)
    if (!(row[j] == 0.f)) {
      first = j;
      break;
    }
  atomicMin(&s_first, first);
  __syncthreads();
  const int v = s_first;
  int bad = 0;
  for (int j = v + threadIdx.x; j < L; j += blockDim.x) bad |= !(row[j] <= KM_MASKED);
  if (bad) atomicOr(&s_bad, 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int vl = L;
    if (valid) {
      vl = valid[valid_n == 1 ? 0 : r];
      vl = vl < 0 ? 0 : (vl > L ? L : vl);
    }
    const int ok = v >= 1 && s_bad == 0;
    out_ok[r] = ok;
    out_valid[r] = ok ? (v < vl ? v : vl) : vl;
  }
}

}  // namespace

int tabicl_launch_key_prefix(const float* bias, int64_t bias_sr, int64_t nb, int64_t L, const int32_t* valid,
                             int64_t valid_n, int64_t rows, int32_t* out_valid, int32_t* out_ok,
                             hipStream_t stream) {
  hipLaunchKernelGGL(key_prefix_kernel, dim3((unsigned)rows), dim3(256), 0, stream, bias, bias_sr, (int)nb, (int)L,
                     valid, (int)valid_n, out_valid, out_ok);
  return (int)hipGetLastError();
}
