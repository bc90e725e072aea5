// Issue-rate microbenchmarks for gfx950 (MI355X): the measurements behind the design limits of the
// ICL attention kernel (icl_pipe_kernel) and the small-head kernels. Not part of libtabicl_attn.so.
//
//   rates    cost per wave64 instruction per SIMD of v_fma_f32, v_exp_f32, v_exp_f16,
//            v_cvt_pk_bf16_f32, v_cvt_pkrtz_f16_f32, v_pk_fma_f16: 8 independent chains per lane,
//            4 waves per SIMD (1024 workgroups of 4 waves on 256 CUs).
//   coissue  a chain of two v_mfma_f32_32x32x16_bf16 per iteration with N independent VALU
//            instructions (fma or exp) placed between them, 1 and 2 waves per SIMD: how much of the
//            VALU time hides behind the matrix core.
//   step     the ICL kernel's step: per iteration two 32x32x16 MFMAs (the next scores, and the PV
//            product of the previous iteration's bf16 probabilities) and the VALU work of 4
//            probabilities (fma, v_exp_f32) plus 2 packed converts on the previous scores, with the
//            kernel's interleaving; also each VALU kind alone and the fma issued one iteration
//            ahead of its exp; 2 and 4 waves per SIMD.
// Every timing is HIP events around one launch (after a warm-up launch); the reported figure is
// wall time per iteration per SIMD (ns), and for coissue / step also the clock64 cycles per
// iteration and wave and the clock those imply.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <vector>

#define CHECK(x)                                                                              \
  do {                                                                                        \
    hipError_t e_ = (x);                                                                      \
    if (e_ != hipSuccess) {                                                                   \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                           \
    }                                                                                         \
  } while (0)

typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// ------------------------------------------------------------------------------------------------
// rates
template <int K>
__global__ __launch_bounds__(256) void rates_kernel(float* out, int iters) {
  float a0 = -0.001f * threadIdx.x, a1 = a0 - 0.1f, a2 = a0 - 0.2f, a3 = a0 - 0.3f;
  float a4 = a0 - 0.4f, a5 = a0 - 0.5f, a6 = a0 - 0.6f, a7 = a0 - 0.7f;
  const float c = 0.999f;
  for (int it = 0; it < iters; ++it) {
#define RATE_OP(x)                                                                 \
  if (K == 0) asm volatile("v_exp_f32 %0, %0" : "+v"(x));                         \
  if (K == 1) asm volatile("v_exp_f16 %0, %0" : "+v"(x));                         \
  if (K == 2) asm volatile("v_cvt_pk_bf16_f32 %0, %0, %0" : "+v"(x));             \
  if (K == 3) asm volatile("v_cvt_pkrtz_f16_f32 %0, %0, %0" : "+v"(x));           \
  if (K == 4) asm volatile("v_fma_f32 %0, %0, %1, %1" : "+v"(x) : "v"(c));         \
  if (K == 5) asm volatile("v_pk_fma_f16 %0, %0, %1, %1" : "+v"(x) : "v"(c));
    RATE_OP(a0) RATE_OP(a1) RATE_OP(a2) RATE_OP(a3) RATE_OP(a4) RATE_OP(a5) RATE_OP(a6) RATE_OP(a7)
#undef RATE_OP
  }
  out[blockIdx.x * 256 + threadIdx.x] = a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7;
}

template <int K>
void rates(const char* name) {
  const int nblk = 1024, iters = 20000;
  float* out;
  CHECK(hipMalloc(&out, nblk * 256 * 4));
  hipLaunchKernelGGL(rates_kernel<K>, dim3(nblk), dim3(256), 0, 0, out, 100);
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL(rates_kernel<K>, dim3(nblk), dim3(256), 0, 0, out, iters);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  std::printf("rates   %-22s ns per wave64 instruction per SIMD = %6.3f\n", name, ms * 1e6 / (4.0 * iters * 8));
  CHECK(hipFree(out));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

// ------------------------------------------------------------------------------------------------
// coissue: KIND 0 fma, 1 exp (with MFMAs); 2 fma, 3 exp (VALU only, no MFMA)
template <int NF, int KIND>
__global__ __launch_bounds__(256) void coissue_kernel(float* out, long long* cyc, int iters) {
  f32x16 acc0 = {}, acc1 = {};
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (threadIdx.x + i));
    b[i] = (__bf16)(0.002f * i);
  }
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = 0.01f * (threadIdx.x + i);
  const long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
    if (KIND < 2) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, acc1, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      if (KIND == 1 || KIND == 3) x[j & 7] = __builtin_amdgcn_exp2f(x[j & 7]) * -0.5f;
      else x[j & 7] = __builtin_fmaf(x[j & 7], 0.9999f, 0.5f);
    }
    if (KIND < 2) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NF / 2 * (KIND == 1 ? 2 : 1), 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NF / 2 * (KIND == 1 ? 2 : 1), 0);
    }
  }
  const long long t1 = clock64();
  float s = 0;
  for (int i = 0; i < 16; ++i) s += acc0[i] + acc1[i];
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if (threadIdx.x % 64 == 0) cyc[blockIdx.x * 4 + threadIdx.x / 64] = t1 - t0;
}

// ------------------------------------------------------------------------------------------------
// step: MODE 0 MFMA only, 1 VALU only, 2 both interleaved; K: 0 the fma -> exp -> convert mix,
// 1 fma only (8 fma + 2 converts), 2 exp only (4 exp + 2 converts), 3 the mix with each fma one
// iteration ahead of its exp
template <int MODE, int K>
__global__ __launch_bounds__(256) void step_kernel(float* out, long long* cyc, int iters) {
  f32x16 acc0 = {}, sp = {};
  bf16x8 a, b, pprev;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (threadIdx.x + i));
    b[i] = (__bf16)(0.002f * i);
    pprev[i] = (__bf16)0.f;
  }
  for (int i = 0; i < 16; ++i) sp[i] = -0.01f * (threadIdx.x + i);
  const f32x16 zero = {};
  float yy[4] = {0.f, 0.f, 0.f, 0.f};
  const long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
    f32x16 sn = sp;
    if (MODE != 1) sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, zero, 0, 0, 0);  // next scores
    bf16x8 p = pprev;
    if (MODE != 0) {
      float e[4];
      if (K == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[j], 0.18f, -0.5f));
      } else if (K == 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = __builtin_fmaf(__builtin_fmaf(sp[j], 0.18f, -0.5f), sp[j + 4], 0.25f);
      } else if (K == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = __builtin_amdgcn_exp2f(sp[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          e[j] = __builtin_amdgcn_exp2f(yy[j]);
          yy[j] = __builtin_fmaf(sp[j], 0.18f, -0.5f);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x2 q;
        q[0] = (__bf16)e[2 * j];
        q[1] = (__bf16)e[2 * j + 1];
        p[2 * j] = q[0];
        p[2 * j + 1] = q[1];
      }
    }
    if (MODE != 1) acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pprev, acc0, 0, 0, 0);  // PV of the last P
    if (MODE == 2) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
    }
    if (MODE == 1) {
      asm volatile("" : "+v"(sp));  // opaque each iteration: the VALU work stays in the loop
      asm volatile("" ::"v"(p));
    } else {
      sp = sn;
    }
    pprev = p;
  }
  const long long t1 = clock64();
  float s = 0;
  for (int i = 0; i < 16; ++i) s += acc0[i] + sp[i];
  for (int i = 0; i < 8; ++i) s += (float)pprev[i];
  for (int i = 0; i < 4; ++i) s += yy[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if (threadIdx.x % 64 == 0) cyc[blockIdx.x * 4 + threadIdx.x / 64] = t1 - t0;
}

// one timed launch of a (out, cyc, iters) kernel over 256 x wps workgroups of 4 waves: wps waves per SIMD
template <typename F>
void timed(const char* group, const char* name, int wps, F kernel) {
  const int nblk = 256 * wps, iters = 20000;
  float* out;
  long long* cyc;
  CHECK(hipMalloc(&out, nblk * 256 * 4));
  CHECK(hipMalloc(&cyc, nblk * 4 * 8));
  hipLaunchKernelGGL(kernel, dim3(nblk), dim3(256), 0, 0, out, cyc, 100);
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL(kernel, dim3(nblk), dim3(256), 0, 0, out, cyc, iters);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<long long> c(nblk * 4);
  CHECK(hipMemcpy(c.data(), cyc, c.size() * 8, hipMemcpyDeviceToHost));
  double avg = 0;
  for (long long v : c) avg += (double)v;
  avg /= (double)c.size();
  std::printf("%-7s %-26s wps=%d  wall ns/iter/SIMD=%6.2f  cyc/iter/wave=%7.1f  clock~%.2f GHz\n", group, name, wps,
              ms * 1e6 / iters / wps, avg / iters, avg / (ms * 1e6));
  CHECK(hipFree(out));
  CHECK(hipFree(cyc));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main(int argc, char** argv) {
  const char* only = argc > 1 ? argv[1] : "";
  if (!*only || !std::strcmp(only, "rates")) {
    rates<4>("v_fma_f32");
    rates<0>("v_exp_f32");
    rates<1>("v_exp_f16");
    rates<2>("v_cvt_pk_bf16_f32");
    rates<3>("v_cvt_pkrtz_f16_f32");
    rates<5>("v_pk_fma_f16");
  }
  if (!*only || !std::strcmp(only, "coissue")) {
    for (int wps = 1; wps <= 2; ++wps) {
      timed("coissue", "mfma x2 only", wps, coissue_kernel<0, 0>);
      timed("coissue", "valu 8 fma only", wps, coissue_kernel<8, 2>);
      timed("coissue", "valu 16 fma only", wps, coissue_kernel<16, 2>);
      timed("coissue", "valu 8 exp only", wps, coissue_kernel<8, 3>);
      timed("coissue", "mfma x2 + 8 fma", wps, coissue_kernel<8, 0>);
      timed("coissue", "mfma x2 + 16 fma", wps, coissue_kernel<16, 0>);
      timed("coissue", "mfma x2 + 32 fma", wps, coissue_kernel<32, 0>);
      timed("coissue", "mfma x2 + 8 exp", wps, coissue_kernel<8, 1>);
      timed("coissue", "mfma x2 + 16 exp", wps, coissue_kernel<16, 1>);
    }
  }
  if (!*only || !std::strcmp(only, "step")) {
    for (int wps = 2; wps <= 4; wps += 2) {
      timed("step", "mfma x2 only", wps, step_kernel<0, 0>);
      timed("step", "valu mix only", wps, step_kernel<1, 0>);
      timed("step", "mfma + valu mix", wps, step_kernel<2, 0>);
      timed("step", "mfma + 8 fma + 2 cvt", wps, step_kernel<2, 1>);
      timed("step", "mfma + 4 exp + 2 cvt", wps, step_kernel<2, 2>);
      timed("step", "valu mix fma-ahead only", wps, step_kernel<1, 3>);
      timed("step", "mfma + mix fma-ahead", wps, step_kernel<2, 3>);
    }
  }
  return 0;
}
