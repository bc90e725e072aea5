// Shared device helpers for the gfx950 attention kernels: vector types, MFMA wrappers with a
// uniform lane layout for bf16 and fp32 operands, cross-lane reductions, XCD-aware block mapping.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define TA_LOG2E 1.4426950408889634f
#define TA_LN2 0.6931471805599453f
#define TA_NEG_INF (-__builtin_inff())
// word 3 of a raw (stride 0) buffer resource on gfx9-family parts: 32-bit data format, no swizzle;
// accesses at byte offsets >= num_records are dropped (stores) or return 0 (loads)
#define TA_BUF_WORD3 0x00020000
// flag on a RoPE form: the cos / sin tables hold one head's 16 columns ([L, 16]) shared by every head
#define TA_ROPE_SHARED 0x10

// Operand vectors: N consecutive k-values of one row held by one lane.
template <typename T, int N> struct OpVec;
template <> struct OpVec<bf16, 4> { typedef bf16x4 type; };
template <> struct OpVec<bf16, 8> { typedef bf16x8 type; };
template <> struct OpVec<float, 4> { typedef f32x4 type; };
template <> struct OpVec<float, 8> { typedef f32x8 type; };

// 16x16 tile, 16-deep contraction. Lane l holds A[l%16][4*(l/16)+j] and B[4*(l/16)+j][l%16]
// (j = 0..3); result lane l, reg r = C[4*(l/16)+r][l%16].
// bf16: one v_mfma_f32_16x16x16_bf16. fp32: four v_mfma_f32_16x16x4_f32, the j-th one contracting
// k = 4*kappa + j over kappa = l/16 (so the lane data is the same four values in both cases).
__device__ __forceinline__ f32x4 mfma16x16x16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(f32x4 a, f32x4 b, f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  return c;
}

// 32x32 tile, 16-deep contraction. Lane l holds A[l%32][8*(l/32)+j] and B[8*(l/32)+j][l%32]
// (j = 0..7); result lane l, reg r = C[8*(r/4) + 4*(l/32) + r%4][l%32].
// bf16: one v_mfma_f32_32x32x16_bf16. fp32: eight v_mfma_f32_32x32x2_f32 (k = 8*kappa + j).
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(f32x8 a, f32x8 b, f32x16 c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }
// Four fp32 values to bf16 (round to nearest even), converted in pairs (v_cvt_pk_bf16_f32); built
// from two packed halves so that the compiler does not convert element by element and repack.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x4 cvt_bf16x4(f32x4 x) {
  const bf16x2 lo = __builtin_convertvector(f32x2{x[0], x[1]}, bf16x2);
  const bf16x2 hi = __builtin_convertvector(f32x2{x[2], x[3]}, bf16x2);
  const uint2 u = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
  return __builtin_bit_cast(bf16x4, u);
}
template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

// Max / sum across the lane pairs (l, l^32) and quads (l, l^16, l^32, l^48).
__device__ __forceinline__ float xor_max(float x, int mask) {
  return fmaxf(x, __shfl_xor(x, mask, 64));
}
__device__ __forceinline__ float xor_sum(float x, int mask) { return x + __shfl_xor(x, mask, 64); }

__device__ __forceinline__ bool wave_any(bool p) { return __ballot(p) != 0ull; }

// Max / sum over the lane quad (l, l^16, l^32, l^48) with the gfx950 permlane swaps (no LDS).
__device__ __forceinline__ float quad_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ds_read_b64_tr_b16 operands (LDS address space).
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

// Hardware dispatch places workgroup b on XCD b % 8. Map it to a work index so that each XCD
// receives a contiguous range of work items (neighbouring items share K/V in that XCD's L2).
__device__ __forceinline__ int xcd_remap(int bid, int nblk) {
  const int q8 = nblk >> 3, r8 = nblk & 7;
  const int xcd = bid & 7, idx = bid >> 3;
  return xcd * q8 + (xcd < r8 ? xcd : r8) + idx;
}

struct u32x4 { uint32_t x, y, z, w; };

// RoPE partner of dim jd (0..15) of a head: R(x)_jd = sign * x[partner]
// (reference: x*cos + R(x)*sin, R = signed rotate-half per head, pairs or halves, zero past rot;
// scripts/tabicl_tpu_pallas_attn.py:465-473).
__device__ __forceinline__ void rope_partner(int jd, int rope, int half, int rot, int* partner,
                                             float* sign) {
  if (rope == 1) {
    *partner = jd ^ 1;
    *sign = (jd & 1) ? 1.f : -1.f;
  } else if (jd < half) {
    *partner = jd + half;
    *sign = -1.f;
  } else {
    *partner = jd - half;
    *sign = 1.f;
  }
  if (jd >= rot) {
    *partner = jd;
    *sign = 0.f;
  }
}

// Four consecutive dims d0..d0+3 (d0 % 4 == 0) of one row after RoPE, in fp32.
template <typename T>
__device__ __forceinline__ f32x4 rope4(const T* row, const float* cs, const float* sn, int d0,
                                       int rope, int half, int rot, int tcol) {
  const int hb = d0 & ~15;
  const float4 c = *(const float4*)(cs + tcol);  // table columns of dims d0..d0+3
  const float4 s = *(const float4*)(sn + tcol);
  const float cv[4] = {c.x, c.y, c.z, c.w};
  const float sv[4] = {s.x, s.y, s.z, s.w};
  f32x4 y;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    int pt;
    float sg;
    rope_partner((d0 & 15) + r, rope, half, rot, &pt, &sg);
    const float x = to_f32<T>(row[d0 + r]);
    const float xp = to_f32<T>(row[hb + pt]);
    y[r] = x * cv[r] + sg * xp * sv[r];
  }
  return y;
}

// rope4 with fast paths for the full-width rotations (rot = 16): halves (partner chunk d0 ^ 8) and
// pairs (partner inside the chunk); other forms through rope4.
template <typename T>
__device__ __forceinline__ f32x4 rope4_fast(const T* row, const float* cs, const float* sn, int d0, int rope,
                                            int half, int rot) {
  typedef typename OpVec<T, 4>::type Op4;
  if (rope == 2 && half == 8 && rot == 16) {
    const Op4 own = *(const Op4*)(row + d0);
    const Op4 pt = *(const Op4*)(row + (d0 ^ 8));
    const float4 c = *(const float4*)(cs + d0);
    const float4 s = *(const float4*)(sn + d0);
    const float cv[4] = {c.x, c.y, c.z, c.w};
    const float sv[4] = {s.x, s.y, s.z, s.w};
    const float sg = (d0 & 8) ? 1.f : -1.f;
    f32x4 y;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = to_f32<T>(own[r]) * cv[r] + sg * to_f32<T>(pt[r]) * sv[r];
    return y;
  }
  if (rope == 1 && rot == 16) {
    const Op4 own = *(const Op4*)(row + d0);
    const float4 c = *(const float4*)(cs + d0);
    const float4 s = *(const float4*)(sn + d0);
    const float cv[4] = {c.x, c.y, c.z, c.w};
    const float sv[4] = {s.x, s.y, s.z, s.w};
    f32x4 y;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float xp = to_f32<T>(own[r ^ 1]);
      y[r] = to_f32<T>(own[r]) * cv[r] + ((r & 1) ? xp : -xp) * sv[r];
    }
    return y;
  }
  return rope4<T>(row, cs, sn, d0, rope, half, rot, d0);
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *(const uint4*)p; }

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): LDS[lds_addr + 16 * lane] =
// *src, lds_addr wave-uniform. Issued as inline assembly so that the compiler does not wait for it
// before unrelated LDS reads (it would put s_waitcnt vmcnt(0) in front of the next ds_read); the
// kernels wait with explicit vmcnt counts. M0 holds nothing else in these kernels.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
// The same copy from a wave-uniform base address plus this lane's 32-bit byte offset (the scalar-base
// form of the instruction: no 64-bit address arithmetic per lane).
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void* sbase, uint32_t lds_addr) {
  // readfirstlane returns int: take each half back as uint32_t so the low half is not sign-extended
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | lo;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"((const void*)(uintptr_t)bu), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
// The 4-byte form (global_load_lds_dword): LDS[lds_addr + 4 * lane] = *(sbase + voff).
__device__ __forceinline__ void lds_dma4_s(uint32_t voff, const void* sbase, uint32_t lds_addr) {
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | lo;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(voff), "s"((const void*)(uintptr_t)bu), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Byte address of a __shared__ object in the LDS aperture.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Wait until at most N of this wave's vector-memory operations are outstanding (LDS operations:
// none), then join the workgroup.
#define TA_WAIT_JOIN(N) asm volatile("s_waitcnt vmcnt(" #N ") lgkmcnt(0)\n\ts_barrier" ::: "memory")
// Join the workgroup after this wave's LDS operations have completed, leaving its vector-memory
// operations (copies into LDS, loads, stores) in flight: a barrier whose fence does not wait for them.
#define TA_JOIN_LDS() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
