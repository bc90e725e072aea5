// C ABI of libtabicl_attn.so: argument checks, stride/layout translation from the reference's op
// signatures to the two kernel families, and the fit-time cache append kernel.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/tabicl_attn.h"
#include "common.h"
#include "launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(int err, const char* what) {
  if (err == 0) return 0;
  return fail(-err, "%s: HIP launch failed: %s", what, hipGetErrorString((hipError_t)err));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
size_t esize(int32_t dtype) { return dtype == TABICL_DTYPE_BF16 ? 2 : 4; }
bool stride_ok(int64_t s, int32_t dtype) { return (s * (int64_t)esize(dtype)) % 16 == 0; }

// Shape rules of the small-head kernel: d = 16, h = 8, E = 128.
int smallhead_shape(const char* op, int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h,
                    int32_t dtype) {
  if (dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32)
    return fail(1, "%s: dtype code %d not supported", op, dtype);
  if (E != 128 || h != 8)
    return fail(1, "%s: needs E == 128 and h == 8 (head dim 16), got E=%lld h=%d", op,
                (long long)E, h);
  // no keys only where there is nothing to compute (no batch element or no query row: an empty
  // self-attention); the entry points return before any launch then
  const int64_t lk_min = B > 0 && Lq > 0 ? 1 : 0;
  if (B < 0 || Lq < 0 || Lk < lk_min || B > (1LL << 30) || Lq > (1LL << 30) || Lk > (1LL << 30))
    return fail(1, "%s: bad sizes B=%lld Lq=%lld Lk=%lld", op, (long long)B, (long long)Lq,
                (long long)Lk);
  return 0;
}

static_assert(TABICL_ROPE_SHARED_TABLES == TA_ROPE_SHARED, "shared-table RoPE flag");

// The rope code: none, or pairs / halves, optionally with TABICL_ROPE_SHARED_TABLES.
int rope_args(const char* op, int32_t rope, int32_t half, int32_t rot) {
  if (rope == TABICL_ROPE_NONE) return 0;
  rope &= ~TABICL_ROPE_SHARED_TABLES;
  if (rope != TABICL_ROPE_PAIRS && rope != TABICL_ROPE_HALVES)
    return fail(1, "%s: rope code %d not supported", op, rope);
  if (rot < 2 || rot > 16 || (rot & 1) || half * 2 != rot)
    return fail(1, "%s: rope needs even rot in [2, 16] and half == rot/2 (rot=%d half=%d)", op,
                rot, half);
  return 0;
}

template <typename T>
__global__ void cache_append_kernel(T* kc, T* vc, int64_t dst_sn, int64_t dst_sh, int64_t row0,
                                    const T* ks, const T* vs, int64_t src_sn, int64_t src_sh,
                                    int64_t src_st, int H, int T_rows, int D) {
  constexpr int EPC = 16 / sizeof(T);
  const int cpr = D / EPC;
  const int64_t total = (int64_t)gridDim.y * H * T_rows * cpr;  // gridDim.y = N
  const int n = blockIdx.y;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < total / gridDim.y;
       c += (int64_t)gridDim.x * blockDim.x) {
    const int cc = (int)(c % cpr);
    const int64_t rowg = c / cpr;
    const int t = (int)(rowg % T_rows);
    const int h = (int)(rowg / T_rows);
    const int64_t so = n * src_sn + h * src_sh + t * src_st + cc * EPC;
    const int64_t dofs = n * dst_sn + h * dst_sh + (row0 + t) * D + cc * EPC;
    *(uint4*)(kc + dofs) = ldg16(ks + so);
    *(uint4*)(vc + dofs) = ldg16(vs + so);
  }
}

// Checks shared by the three backward entry points.
int bwd_common(const char* op, int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h, int32_t dtype,
               const float* bias, int64_t bias_b, const void* o, const void* dout, void* ws, int64_t ws_bytes) {
  int st = smallhead_shape(op, B, Lq, Lk, E, h, dtype);
  if (st) return st;
  if (bias && bias_b != 1 && bias_b != B)
    return fail(1, "%s: bias batch %lld must be 1 or B=%lld", op, (long long)bias_b, (long long)B);
  if (B > 0 && Lq > 0 && (!o || !dout || !aligned16(o) || !aligned16(dout)))
    return fail(1, "%s: o and dout must be 16-byte aligned device pointers", op);
  if (B > 0 && Lq > 0 && (!ws || !aligned16(ws) || ws_bytes < tabicl_launch_smallhead_bwd_ws_bytes(B, Lq)))
    return fail(1, "%s: workspace of %lld bytes (16-byte aligned) required", op,
                (long long)tabicl_launch_smallhead_bwd_ws_bytes(B, Lq));
  if (B * ((Lq + 127) / 128 + (Lk + 127) / 128) * 8 > (1LL << 31) - 1) return fail(1, "%s: grid too large", op);
  return 0;
}

// Argument checks shared by the ICL entry points (status 0 or 1 with the message set).
int icl_args(const char* op, const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
             const float* key_bias, int64_t bias_n, int64_t bias_sn, const int32_t* q_len, int64_t q_len_n,
             const void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D, const int64_t* strides,
             float scale, int32_t dtype) {
  if (dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32) return fail(1, "%s: dtype code %d not supported", op, dtype);
  if (key_bias) {
    if (bias_n != 1 && bias_n != N) return fail(1, "%s: key_bias must hold 1 or N rows", op);
    if (bias_n > 1 && bias_sn < Tkv) return fail(1, "%s: key_bias row stride %lld < Tkv", op, (long long)bias_sn);
    if (!aligned16(key_bias)) return fail(1, "%s: key_bias must be 16-byte aligned", op);
    if (!(scale > 0.f) || !(scale < 1e30f)) return fail(1, "%s: a key mask needs a positive finite scale", op);
  }
  if (D != 64) return fail(1, "%s: head dim must be 64, got %lld", op, (long long)D);
  if (N < 0 || H < 0 || Tq < 0 || Tkv < 1 || Tq > (1LL << 30) || Tkv > (1LL << 30)) return fail(1, "%s: bad sizes", op);
  if (valid && valid_n != 1 && valid_n != N) return fail(1, "%s: valid must hold 1 or N entries", op);
  if (q_len && q_len_n != 1 && q_len_n != N) return fail(1, "%s: q_len must hold 1 or N entries", op);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(1, "%s: pointers must be 16-byte aligned", op);
  for (int i = 0; i < 12; ++i)
    if (strides[i] < 0 || !stride_ok(strides[i], dtype))
      return fail(1, "%s: strides must be non-negative multiples of 16 bytes", op);
  if (N * H * ((Tq + 127) / 128) > (1LL << 31) - 1) return fail(1, "%s: grid too large", op);
  return 0;
}

}  // namespace

extern "C" {

const char* tabicl_attn_last_error(void) { return g_err; }

const char* tabicl_attn_version(void) { return "tabicl_attn 0.1 gfx950"; }

int tabicl_attn_supported(int32_t op, int64_t Lq, int64_t Lk, int64_t E, int32_t h,
                          int32_t dtype) {
  if (dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32) return 0;
  if (Lq < 0 || Lk < 1 || Lq > (1LL << 30) || Lk > (1LL << 30)) return 0;
  switch (op) {
    case TABICL_OP_HX:
    case TABICL_OP_HXQ:
    case TABICL_OP_PK_SELF:
    case TABICL_OP_PK_CROSS:
      return E == 128 && h == 8;
    case TABICL_OP_ICL:
      return E == 64;
    default:
      return 0;
  }
}

int tabicl_hx_fwd(const void* q, const void* k, const void* v, const float* bias, int64_t bias_b,
                  void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h, int32_t dtype,
                  void* stream) {
  int st = smallhead_shape("hx_fwd", B, Lq, Lk, E, h, dtype);
  if (st) return st;
  if (bias && bias_b != 1 && bias_b != B)
    return fail(1, "hx_fwd: bias batch %lld must be 1 or B=%lld", (long long)bias_b, (long long)B);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (bias && !aligned16(bias)))
    return fail(1, "hx_fwd: pointers must be 16-byte aligned");
  if (B == 0 || Lq == 0) return 0;
  return launch_status(
      tabicl_launch_smallhead(q, Lq * E, E, k, Lk * E, E, v, Lk * E, E, out, bias,
                              bias && bias_b == B ? Lk : 0, nullptr, 0, nullptr, nullptr, nullptr,
                              nullptr, 0, 0, 0, 1.0f, B, Lq, Lk, dtype, nullptr, 0,
                              (hipStream_t)stream),
      "hx_fwd");
}

int tabicl_hxq_fwd(const int32_t* valid, int64_t valid_n, const void* q, const void* kv, void* out,
                   int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h, int32_t dtype,
                   void* workspace, int64_t workspace_bytes, void* stream) {
  int st = smallhead_shape("hxq_fwd", B, Lq, Lk, E, h, dtype);
  if (st) return st;
  if (!valid || (valid_n != 1 && valid_n != B))
    return fail(1, "hxq_fwd: valid must hold 1 or B=%lld entries (got %lld)", (long long)B,
                (long long)valid_n);
  if (!aligned16(q) || !aligned16(kv) || !aligned16(out))
    return fail(1, "hxq_fwd: pointers must be 16-byte aligned");
  if (B == 0 || Lq == 0) return 0;
  const char* kvb = (const char*)kv;
  void* ws = workspace && aligned16(workspace) ? workspace : nullptr;
  return launch_status(
      tabicl_launch_smallhead(q, Lq * E, E, kvb, Lk * 2 * E, 2 * E, kvb + E * esize(dtype),
                              Lk * 2 * E, 2 * E, out, nullptr, 0, valid, valid_n, nullptr, nullptr,
                              nullptr, nullptr, 0, 0, 0, 1.0f, B, Lq, Lk, dtype, ws,
                              ws ? workspace_bytes : 0, (hipStream_t)stream),
      "hxq_fwd");
}

int tabicl_hxq_fwd_masked(const int32_t* valid, int64_t valid_n, const float* key_bias, int64_t bias_b,
                          const void* q, const void* kv, void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                          int32_t h, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!key_bias) return tabicl_hxq_fwd(valid, valid_n, q, kv, out, B, Lq, Lk, E, h, dtype, workspace,
                                       workspace_bytes, stream);
  int st = smallhead_shape("hxq_fwd_masked", B, Lq, Lk, E, h, dtype);
  if (st) return st;
  if (valid && valid_n != 1 && valid_n != B)
    return fail(1, "hxq_fwd_masked: valid must hold 1 or B=%lld entries (got %lld)", (long long)B,
                (long long)valid_n);
  if (bias_b != 1 && bias_b != B)
    return fail(1, "hxq_fwd_masked: key_bias batch %lld must be 1 or B=%lld", (long long)bias_b, (long long)B);
  if (!aligned16(q) || !aligned16(kv) || !aligned16(out) || !aligned16(key_bias))
    return fail(1, "hxq_fwd_masked: pointers must be 16-byte aligned");
  if (B == 0 || Lq == 0) return 0;
  const char* kvb = (const char*)kv;
  void* ws = workspace && aligned16(workspace) ? workspace : nullptr;
  return launch_status(
      tabicl_launch_smallhead(q, Lq * E, E, kvb, Lk * 2 * E, 2 * E, kvb + E * esize(dtype), Lk * 2 * E, 2 * E, out,
                              key_bias, bias_b == B ? Lk : 0, valid, valid ? valid_n : 0, nullptr, nullptr,
                              nullptr, nullptr, 0, 0, 0, 1.0f, B, Lq, Lk, dtype, ws, ws ? workspace_bytes : 0,
                              (hipStream_t)stream),
      "hxq_fwd_masked");
}

int64_t tabicl_hxq_workspace_bytes(int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h,
                                   int32_t dtype) {
  if (E != 128 || h != 8 || B <= 0 || Lq <= 0 || Lk <= 0) return 0;
  if (dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32) return 0;
  // sized for tabicl_hxq_fwd_masked too (the prefix view of a key mask: 8 bytes per batch element)
  return tabicl_launch_smallhead_ws_bytes(B, Lq, Lk, dtype, true, 0);
}

int tabicl_pk_self_fwd(const void* qkv, const float* bias, int64_t bias_b, const float* cos_t,
                       const float* sin_t, void* out, int64_t B, int64_t L, int64_t E, int32_t h,
                       int32_t rope, int32_t half, int32_t rot, float scale, int32_t dtype,
                       void* stream) {
  int st = smallhead_shape("pk_self_fwd", B, L, L, E, h, dtype);
  if (st) return st;
  if ((st = rope_args("pk_self_fwd", rope, half, rot))) return st;
  if (rope && (!cos_t || !sin_t)) return fail(1, "pk_self_fwd: rope tables missing");
  if (bias && bias_b != 1 && bias_b != B)
    return fail(1, "pk_self_fwd: bias batch %lld must be 1 or B", (long long)bias_b);
  if (!aligned16(qkv) || !aligned16(out) || (rope && (!aligned16(cos_t) || !aligned16(sin_t))))
    return fail(1, "pk_self_fwd: pointers must be 16-byte aligned");
  if (B == 0 || L == 0) return 0;
  const char* base = (const char*)qkv;
  const size_t es = esize(dtype);
  return launch_status(
      tabicl_launch_smallhead(base, L * 3 * E, 3 * E, base + E * es, L * 3 * E, 3 * E,
                              base + 2 * E * es, L * 3 * E, 3 * E, out, bias,
                              bias && bias_b == B ? L : 0, nullptr, 0, cos_t, sin_t, cos_t, sin_t,
                              rope, half, rot, scale, B, L, L, dtype, nullptr, 0,
                              (hipStream_t)stream),
      "pk_self_fwd");
}

int tabicl_pk_cross_fwd(const void* q, int64_t q_b, const void* kv, const float* bias,
                        int64_t bias_b, const float* cq, const float* sq, const float* ck,
                        const float* sk, void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                        int32_t h, int32_t rope, int32_t half, int32_t rot, float scale,
                        int32_t dtype, void* stream) {
  return tabicl_pk_cross_fwd_ragged(q, q_b, kv, bias, bias_b, cq, sq, ck, sk, out, B, Lq, Lk, E, h, rope, half,
                                    rot, scale, dtype, nullptr, 0, stream);
}

int tabicl_pk_cross_fwd_ragged(const void* q, int64_t q_b, const void* kv, const float* bias,
                               int64_t bias_b, const float* cq, const float* sq, const float* ck,
                               const float* sk, void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                               int32_t h, int32_t rope, int32_t half, int32_t rot, float scale,
                               int32_t dtype, const int32_t* q_len, int64_t q_len_n, void* stream) {
  int st = smallhead_shape("pk_cross_fwd", B, Lq, Lk, E, h, dtype);
  if (st) return st;
  if ((st = rope_args("pk_cross_fwd", rope, half, rot))) return st;
  if (rope && (!cq || !sq || !ck || !sk)) return fail(1, "pk_cross_fwd: rope tables missing");
  if (q_b != 1 && q_b != B) return fail(1, "pk_cross_fwd: q batch must be 1 or B");
  if (q_len && q_len_n != 1 && q_len_n != B) return fail(1, "pk_cross_fwd: q_len must hold 1 or B entries");
  if (bias && bias_b != 1 && bias_b != B)
    return fail(1, "pk_cross_fwd: bias batch %lld must be 1 or B", (long long)bias_b);
  if (!aligned16(q) || !aligned16(kv) || !aligned16(out) ||
      (rope && (!aligned16(cq) || !aligned16(sq) || !aligned16(ck) || !aligned16(sk))))
    return fail(1, "pk_cross_fwd: pointers must be 16-byte aligned");
  if (B == 0 || Lq == 0) return 0;
  const char* kvb = (const char*)kv;
  return launch_status(
      tabicl_launch_smallhead(q, q_b == 1 && B > 1 ? 0 : Lq * E, E, kvb, Lk * 2 * E, 2 * E,
                              kvb + E * esize(dtype), Lk * 2 * E, 2 * E, out, bias,
                              bias && bias_b == B ? Lk : 0, nullptr, 0, cq, sq, ck, sk, rope, half,
                              rot, scale, B, Lq, Lk, dtype, nullptr, 0, (hipStream_t)stream, q_len,
                              q_len ? q_len_n : 0),
      "pk_cross_fwd");
}

int64_t tabicl_smallhead_bwd_workspace_bytes(int64_t B, int64_t Lq, int64_t E, int32_t h) {
  if (E != 128 || h != 8 || B < 0 || Lq < 0) return fail(-1, "smallhead_bwd_workspace_bytes: bad arguments");
  return tabicl_launch_smallhead_bwd_ws_bytes(B, Lq);
}

int tabicl_hx_bwd(const void* q, const void* k, const void* v, const float* bias, int64_t bias_b,
                  const void* o, const void* dout, void* dq, void* dk, void* dv, int64_t B, int64_t Lq,
                  int64_t Lk, int64_t E, int32_t h, int32_t dtype, void* workspace, int64_t workspace_bytes,
                  void* stream) {
  int st = bwd_common("hx_bwd", B, Lq, Lk, E, h, dtype, bias, bias_b, o, dout, workspace, workspace_bytes);
  if (st) return st;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return fail(1, "hx_bwd: pointers must be 16-byte aligned");
  if (B == 0 || Lk == 0) return 0;
  return launch_status(
      tabicl_launch_smallhead_bwd(q, Lq * E, E, k, Lk * E, E, v, Lk * E, E, o, dout, dq, Lq * E, E, dk, Lk * E, E,
                                  dv, Lk * E, E, bias, bias && bias_b == B ? Lk : 0, nullptr, nullptr, nullptr,
                                  nullptr, 0, 0, 0, 1.0f, B, Lq, Lk, dtype, workspace, workspace_bytes,
                                  (hipStream_t)stream),
      "hx_bwd");
}

int tabicl_pk_self_bwd(const void* qkv, const float* bias, int64_t bias_b, const float* cos_t,
                       const float* sin_t, const void* o, const void* dout, void* dqkv, int64_t B, int64_t L,
                       int64_t E, int32_t h, int32_t rope, int32_t half, int32_t rot, float scale, int32_t dtype,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  int st = bwd_common("pk_self_bwd", B, L, L, E, h, dtype, bias, bias_b, o, dout, workspace, workspace_bytes);
  if (st) return st;
  if ((st = rope_args("pk_self_bwd", rope, half, rot))) return st;
  if (rope && (!cos_t || !sin_t)) return fail(1, "pk_self_bwd: rope tables missing");
  if (!aligned16(qkv) || !aligned16(dqkv) || (rope && (!aligned16(cos_t) || !aligned16(sin_t))))
    return fail(1, "pk_self_bwd: pointers must be 16-byte aligned");
  if (B == 0 || L == 0) return 0;
  const char* base = (const char*)qkv;
  char* dbase = (char*)dqkv;
  const size_t es = esize(dtype);
  return launch_status(
      tabicl_launch_smallhead_bwd(base, L * 3 * E, 3 * E, base + E * es, L * 3 * E, 3 * E, base + 2 * E * es,
                                  L * 3 * E, 3 * E, o, dout, dbase, L * 3 * E, 3 * E, dbase + E * es, L * 3 * E,
                                  3 * E, dbase + 2 * E * es, L * 3 * E, 3 * E, bias, bias && bias_b == B ? L : 0,
                                  cos_t, sin_t, cos_t, sin_t, rope, half, rot, scale, B, L, L, dtype, workspace,
                                  workspace_bytes, (hipStream_t)stream),
      "pk_self_bwd");
}

int tabicl_pk_cross_bwd(const void* q, int64_t q_b, const void* kv, const float* bias, int64_t bias_b,
                        const float* cq, const float* sq, const float* ck, const float* sk, const void* o,
                        const void* dout, void* dq, void* dkv, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                        int32_t h, int32_t rope, int32_t half, int32_t rot, float scale, int32_t dtype,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  int st = bwd_common("pk_cross_bwd", B, Lq, Lk, E, h, dtype, bias, bias_b, o, dout, workspace, workspace_bytes);
  if (st) return st;
  if ((st = rope_args("pk_cross_bwd", rope, half, rot))) return st;
  if (rope && (!cq || !sq || !ck || !sk)) return fail(1, "pk_cross_bwd: rope tables missing");
  if (q_b != 1 && q_b != B) return fail(1, "pk_cross_bwd: q batch must be 1 or B");
  if (rope && (!aligned16(cq) || !aligned16(sq) || !aligned16(ck) || !aligned16(sk)))
    return fail(1, "pk_cross_bwd: rope tables must be 16-byte aligned");
  if (!aligned16(q) || !aligned16(kv) || !aligned16(dq) || !aligned16(dkv))
    return fail(1, "pk_cross_bwd: pointers must be 16-byte aligned");
  if (B == 0 || Lk == 0) return 0;
  const char* kvb = (const char*)kv;
  char* dkvb = (char*)dkv;
  const size_t es = esize(dtype);
  return launch_status(
      tabicl_launch_smallhead_bwd(q, q_b == 1 && B > 1 ? 0 : Lq * E, E, kvb, Lk * 2 * E, 2 * E, kvb + E * es,
                                  Lk * 2 * E, 2 * E, o, dout, dq, Lq * E, E, dkvb, Lk * 2 * E, 2 * E,
                                  dkvb + E * es, Lk * 2 * E, 2 * E, bias, bias && bias_b == B ? Lk : 0, cq, sq,
                                  ck, sk, rope, half, rot, scale, B, Lq, Lk, dtype, workspace, workspace_bytes,
                                  (hipStream_t)stream),
      "pk_cross_bwd");
}

int tabicl_icl_fwd(const void* q, const void* k, const void* v, const int32_t* valid,
                   int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                   int64_t D, int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh,
                   int64_t k_st, int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn,
                   int64_t o_sh, int64_t o_st, float scale, int32_t dtype, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  return tabicl_icl_fwd_ragged(q, k, v, valid, valid_n, nullptr, 0, out, N, H, Tq, Tkv, D, q_sn, q_sh, q_st, k_sn,
                               k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale, dtype, workspace,
                               workspace_bytes, stream);
}

int tabicl_icl_fwd_ragged(const void* q, const void* k, const void* v, const int32_t* valid,
                          int64_t valid_n, const int32_t* q_len, int64_t q_len_n, void* out, int64_t N,
                          int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int64_t q_sn, int64_t q_sh,
                          int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st, int64_t v_sn,
                          int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                          float scale, int32_t dtype, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  return tabicl_icl_fwd_masked(q, k, v, valid, valid_n, nullptr, 0, 0, q_len, q_len_n, out, N, H, Tq, Tkv, D, q_sn,
                               q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale, dtype,
                               workspace, workspace_bytes, stream);
}

int tabicl_icl_fwd_ragged_listed(const void* q, const void* k, const void* v, const int32_t* valid,
                                 int64_t valid_n, const int32_t* q_len, int64_t q_len_n, void* out, int64_t N,
                                 int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int64_t q_sn, int64_t q_sh,
                                 int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st, int64_t v_sn,
                                 int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                                 float scale, int32_t dtype, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  const int64_t strides[12] = {q_sn, q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st};
  int st = icl_args("icl_fwd_ragged_listed", q, k, v, valid, valid_n, nullptr, 0, 0, q_len, q_len_n, out, N, H, Tq,
                    Tkv, D, strides, scale, dtype);
  if (st || N == 0 || H == 0 || Tq == 0) return st;
  if (!q_len) return fail(1, "icl_fwd_ragged_listed: q_len is required");
  return launch_status(
      tabicl_launch_icl_fwd(q, k, v, valid, valid ? valid_n : 0, out, N, H, Tq, Tkv, 64, q_sn, q_sh, q_st, k_sn,
                            k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale, dtype,
                            workspace && aligned16(workspace) ? workspace : nullptr, workspace_bytes,
                            (hipStream_t)stream, q_len, q_len_n, nullptr, 0, 0, 1),
      "icl_fwd_ragged_listed");
}

int tabicl_icl_ragged_plan(const int32_t* q_len, int64_t q_len_n, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                           int64_t D, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  if (N < 0 || H < 0 || Tq < 0 || Tkv < 0) return fail(1, "icl_ragged_plan: negative size");
  if (D != 64) return fail(1, "icl_ragged_plan: D must be 64");
  if (dtype != 0 && dtype != 1) return fail(1, "icl_ragged_plan: dtype must be 0 (bf16) or 1 (fp32)");
  if (!q_len || (q_len_n != 1 && q_len_n != N)) return fail(1, "icl_ragged_plan: q_len [1 or N] is required");
  if (N == 0 || H == 0 || Tq == 0 || Tkv == 0) return 0;
  if (workspace && !aligned16(workspace)) return fail(1, "icl_ragged_plan: workspace must be 16-byte aligned");
  // the list goes where the call puts it: the kernels need no q / k / v / out here, only their sizes
  return launch_status(
      tabicl_launch_icl_fwd(nullptr, nullptr, nullptr, nullptr, 0, nullptr, N, H, Tq, Tkv, 64, 0, 0, 0, 0, 0, 0, 0,
                            0, 0, 0, 0, 0, 1.0f, dtype, workspace, workspace ? workspace_bytes : 0,
                            (hipStream_t)stream, q_len, q_len_n, nullptr, 0, 0, 2),
      "icl_ragged_plan");
}

int tabicl_icl_fwd_masked(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                          const float* key_bias, int64_t bias_n, int64_t bias_sn, const int32_t* q_len,
                          int64_t q_len_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                          int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                          int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                          float scale, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t strides[12] = {q_sn, q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st};
  int st = icl_args("icl_fwd", q, k, v, valid, valid_n, key_bias, bias_n, bias_sn, q_len, q_len_n, out, N, H, Tq,
                    Tkv, D, strides, scale, dtype);
  if (st || N == 0 || H == 0 || Tq == 0) return st;
  return launch_status(
      tabicl_launch_icl_fwd(q, k, v, valid, valid ? valid_n : 0, out, N, H, Tq, Tkv, 64, q_sn, q_sh,
                            q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale,
                            dtype, workspace && aligned16(workspace) ? workspace : nullptr,
                            workspace_bytes, (hipStream_t)stream, q_len, q_len ? q_len_n : 0, key_bias,
                            key_bias ? bias_n : 0, key_bias ? bias_sn : 0),
      "icl_fwd");
}

int64_t tabicl_icl_bwd_workspace_bytes(int64_t N, int64_t H, int64_t Tq) {
  if (N < 0 || H < 0 || Tq < 0) return fail(-1, "icl_bwd_workspace_bytes: bad sizes");
  return tabicl_launch_icl_bwd_ws_bytes(N, H, Tq);
}

int tabicl_icl_bwd(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                   const float* key_bias, int64_t bias_n, int64_t bias_sn, const void* o, const void* dout,
                   const float* stat, void* dq, void* dk, void* dv, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                   int64_t D, float scale, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  // contiguous [N, H, T, 64] tensors: the strides the shared checks take
  const int64_t sq[3] = {H * Tq * D, Tq * D, D}, sk[3] = {H * Tkv * D, Tkv * D, D};
  const int64_t strides[12] = {sq[0], sq[1], sq[2], sk[0], sk[1], sk[2], sk[0], sk[1], sk[2], sq[0], sq[1], sq[2]};
  int st = icl_args("icl_bwd", q, k, v, valid, valid_n, key_bias, bias_n, bias_sn, nullptr, 0, o, N, H, Tq, Tkv, D,
                    strides, scale, dtype);
  if (st) return st;
  if (!(scale > 0.f) || !(scale < 1e30f)) return fail(1, "icl_bwd: scale must be positive and finite");
  if (!aligned16(dout) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(stat))
    return fail(1, "icl_bwd: pointers must be 16-byte aligned");
  if (stat && key_bias) return fail(1, "icl_bwd: forward statistics are taken for calls without a key mask only");
  if (N * H * ((Tkv + 63) / 64) > (1LL << 31) - 1 || N * H * ((Tq + 63) / 64) > (1LL << 31) - 1)
    return fail(1, "icl_bwd: grid too large");
  if (N == 0 || H == 0) return 0;
  if (!workspace || !aligned16(workspace) || workspace_bytes < tabicl_launch_icl_bwd_ws_bytes(N, H, Tq))
    return fail(1, "icl_bwd: workspace of %lld bytes (16-byte aligned) required",
                (long long)tabicl_launch_icl_bwd_ws_bytes(N, H, Tq));
  return launch_status(tabicl_launch_icl_bwd(q, k, v, valid, valid ? valid_n : 0, key_bias, key_bias ? bias_n : 0,
                                             key_bias ? bias_sn : 0, o, dout, stat, dq, dk, dv, N, H, Tq, Tkv, scale,
                                             dtype, workspace, workspace_bytes, (hipStream_t)stream),
                       "icl_bwd");
}

int tabicl_icl_fwd_stats(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                         void* out, float* stat, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                         int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                         int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                         float scale, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t strides[12] = {q_sn, q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st};
  int st = icl_args("icl_fwd_stats", q, k, v, valid, valid_n, nullptr, 0, 0, nullptr, 0, out, N, H, Tq, Tkv, D,
                    strides, scale, dtype);
  if (st || N == 0 || H == 0 || Tq == 0) return st;
  if (!stat || !aligned16(stat)) return fail(1, "icl_fwd_stats: stat ([N, H, Tq, 2] fp32, 16-byte aligned) is required");
  return launch_status(
      tabicl_launch_icl_fwd(q, k, v, valid, valid ? valid_n : 0, out, N, H, Tq, Tkv, 64, q_sn, q_sh, q_st, k_sn,
                            k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale, dtype,
                            workspace && aligned16(workspace) ? workspace : nullptr, workspace_bytes,
                            (hipStream_t)stream, nullptr, 0, nullptr, 0, 0, 0, stat),
      "icl_fwd_stats");
}

int tabicl_icl_fwd_noalloc(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                           const float* key_bias, int64_t bias_n, int64_t bias_sn, const int32_t* q_len,
                           int64_t q_len_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                           int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                           int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                           float scale, int32_t dtype, void* stream) {
  const int64_t strides[12] = {q_sn, q_sh, q_st, k_sn, k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st};
  int st = icl_args("icl_fwd_noalloc", q, k, v, valid, valid_n, key_bias, bias_n, bias_sn, q_len, q_len_n, out, N, H,
                    Tq, Tkv, D, strides, scale, dtype);
  if (st || N == 0 || H == 0 || Tq == 0) return st;
  const int64_t need = tabicl_launch_icl_noalloc_min_bytes(N, H, Tq, D, dtype);
  if (need > TABICL_ICL_SCRATCH_BYTES)
    return fail(1, "icl_fwd_noalloc: the call needs %lld bytes of scratch, more than the library's %lld (use "
                "tabicl_icl_fwd with a workspace)", (long long)need, (long long)TABICL_ICL_SCRATCH_BYTES);
  return launch_status(
      tabicl_launch_icl_fwd_noalloc(q, k, v, valid, valid ? valid_n : 0, out, N, H, Tq, Tkv, q_sn, q_sh, q_st, k_sn,
                                    k_sh, k_st, v_sn, v_sh, v_st, o_sn, o_sh, o_st, scale, dtype, (hipStream_t)stream,
                                    q_len, q_len ? q_len_n : 0, key_bias, key_bias ? bias_n : 0,
                                    key_bias ? bias_sn : 0),
      "icl_fwd_noalloc");
}

int64_t tabicl_icl_noalloc_scratch_bytes(void) { return TABICL_ICL_SCRATCH_BYTES; }

int64_t tabicl_icl_workspace_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                                   int32_t dtype) {
  if ((dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32) || D != 64 || N < 0 || H < 0 ||
      Tq < 0 || Tkv < 1)
    return fail(-1, "icl_workspace_bytes: bad arguments");
  if (N == 0 || H == 0 || Tq == 0) return 0;
  return tabicl_launch_icl_ws_bytes(N, H, Tq, Tkv, 64, dtype);
}

int tabicl_hxf_fwd(const int32_t* valid, int64_t valid_n, const void* qf, int64_t q_b, const void* x, void* out,
                   int64_t B, int64_t hq, int64_t Lk, int64_t E, int32_t dtype, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  if (!valid) return fail(1, "hxf_fwd: valid is required");
  return tabicl_hxf_fwd_masked(valid, valid_n, nullptr, 0, qf, q_b, x, out, B, hq, Lk, E, dtype, workspace,
                               workspace_bytes, stream);
}

int tabicl_hxf_fwd_masked(const int32_t* valid, int64_t valid_n, const float* key_bias, int64_t bias_b,
                          const void* qf, int64_t q_b, const void* x, void* out, int64_t B, int64_t hq, int64_t Lk,
                          int64_t E, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  if (dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32)
    return fail(1, "hxf_fwd: dtype code %d not supported", dtype);
  if (key_bias && bias_b != 1 && bias_b != B) return fail(1, "hxf_fwd: key_bias must hold 1 or B rows");
  if (key_bias && !aligned16(key_bias)) return fail(1, "hxf_fwd: key_bias must be 16-byte aligned");
  if (E != 128) return fail(1, "hxf_fwd: needs E == 128, got %lld", (long long)E);
  if (B < 0 || hq < 0 || Lk < 1 || B > (1LL << 30) || hq > (1LL << 30) || Lk > (1LL << 30))
    return fail(1, "hxf_fwd: bad sizes B=%lld hq=%lld Lk=%lld", (long long)B, (long long)hq, (long long)Lk);
  if (q_b != 1 && q_b != B) return fail(1, "hxf_fwd: qf batch must be 1 or B");
  if (valid && valid_n != 1 && valid_n != B)
    return fail(1, "hxf_fwd: valid must hold 1 or B=%lld entries", (long long)B);
  if (!aligned16(qf) || !aligned16(x) || !aligned16(out)) return fail(1, "hxf_fwd: pointers must be 16-byte aligned");
  if (B == 0 || hq == 0) return 0;
  if (B * ((hq + 127) / 128) * 4 > (1LL << 31) - 1) return fail(1, "hxf_fwd: grid too large");
  return launch_status(
      tabicl_launch_icl_fwd(qf, x, x, valid, valid ? valid_n : 0, out, B, 1, hq, Lk, 128,
                            q_b == 1 && B > 1 ? 0 : hq * E, 0, E, Lk * E, 0, E, Lk * E, 0, E, hq * E, 0, E, 1.0f,
                            dtype, workspace && aligned16(workspace) ? workspace : nullptr, workspace_bytes,
                            (hipStream_t)stream, nullptr, 0, key_bias, key_bias ? bias_b : 0,
                            key_bias && bias_b > 1 ? Lk : 0),
      "hxf_fwd");
}

int64_t tabicl_hxf_workspace_bytes(int64_t B, int64_t hq, int64_t Lk, int64_t E, int32_t dtype) {
  if ((dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32) || E != 128 || B < 0 || hq < 0 || Lk < 1)
    return fail(-1, "hxf_workspace_bytes: bad arguments");
  if (B == 0 || hq == 0) return 0;
  return tabicl_launch_icl_ws_bytes(B, 1, hq, Lk, 128, dtype);
}

int tabicl_icl_cache_append(void* k_cache, void* v_cache, int64_t dst_sn, int64_t dst_sh,
                            int64_t row0, int64_t cap, const void* k_src, const void* v_src,
                            int64_t src_sn, int64_t src_sh, int64_t src_st, int64_t N, int64_t H,
                            int64_t T, int64_t D, int32_t dtype, void* stream) {
  if (dtype != TABICL_DTYPE_BF16 && dtype != TABICL_DTYPE_F32)
    return fail(1, "icl_cache_append: dtype code %d not supported", dtype);
  if (D < 1 || (D * (int64_t)esize(dtype)) % 16) return fail(1, "icl_cache_append: bad head dim");
  if (row0 < 0 || T < 0 || row0 + T > cap)
    return fail(1, "icl_cache_append: rows [%lld, %lld) exceed capacity %lld", (long long)row0,
                (long long)(row0 + T), (long long)cap);
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(k_src) || !aligned16(v_src))
    return fail(1, "icl_cache_append: pointers must be 16-byte aligned");
  const int64_t s[5] = {dst_sn, dst_sh, src_sn, src_sh, src_st};
  for (int i = 0; i < 5; ++i)
    if (s[i] < 0 || !stride_ok(s[i], dtype))
      return fail(1, "icl_cache_append: strides must be non-negative multiples of 16 bytes");
  if (N == 0 || H == 0 || T == 0) return 0;
  if (N > 65535) return fail(1, "icl_cache_append: N too large");
  const int64_t per_n = H * T * (D * (int64_t)esize(dtype) / 16);
  int64_t gx = (per_n + 255) / 256;
  if (gx > 65536) gx = 65536;
  hipStream_t s0 = (hipStream_t)stream;
  if (dtype == TABICL_DTYPE_BF16)
    hipLaunchKernelGGL(cache_append_kernel<bf16>, dim3((unsigned)gx, (unsigned)N), dim3(256), 0, s0,
                       (bf16*)k_cache, (bf16*)v_cache, dst_sn, dst_sh, row0, (const bf16*)k_src,
                       (const bf16*)v_src, src_sn, src_sh, src_st, (int)H, (int)T, (int)D);
  else
    hipLaunchKernelGGL(cache_append_kernel<float>, dim3((unsigned)gx, (unsigned)N), dim3(256), 0, s0,
                       (float*)k_cache, (float*)v_cache, dst_sn, dst_sh, row0, (const float*)k_src,
                       (const float*)v_src, src_sn, src_sh, src_st, (int)H, (int)T, (int)D);
  return launch_status((int)hipGetLastError(), "icl_cache_append");
}

}  // extern "C"

int tabicl_layer_norm(const void* x, const void* residual, void* x_out, const float* weight, const float* bias,
                      void* out, int64_t rows, int64_t width, float eps, int32_t in_dtype, int32_t out_dtype,
                      void* stream) {
  if (rows < 0) return fail(1, "layer_norm: negative row count");
  if (width != 128 && width != 512) return fail(1, "layer_norm: width %lld not supported (128 or 512)", (long long)width);
  if ((in_dtype != 0 && in_dtype != 1) || (out_dtype != 0 && out_dtype != 1))
    return fail(1, "layer_norm: dtypes must be 0 (bf16) or 1 (fp32)");
  if (!(eps > 0.f)) return fail(1, "layer_norm: eps must be positive");
  if (rows == 0) return 0;
  if (!x || !out || !aligned16(x) || !aligned16(out) || (weight && !aligned16(weight)) || (bias && !aligned16(bias)))
    return fail(1, "layer_norm: x, out, weight and bias must be 16-byte aligned device pointers");
  if (residual && (!x_out || !aligned16(residual) || !aligned16(x_out)))
    return fail(1, "layer_norm: with a residual, x_out (16-byte aligned) receives x + residual");
  return launch_status(tabicl_launch_layer_norm(x, residual, residual ? x_out : nullptr, weight, bias, out, rows, width,
                                                eps, in_dtype, out_dtype, (hipStream_t)stream),
                       "layer_norm");
}
