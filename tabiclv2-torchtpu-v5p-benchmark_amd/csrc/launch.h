// Host launchers of the kernel families (device pointers, element strides, HIP stream); the C ABI
// in abi.hip checks arguments and translates the reference's op signatures to these calls.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Prefix view of key-only additive masks (keymask.hip): for each of `rows` rows r, out_ok[r] = 1 if
// bias row (nb == 1 ? 0 : r) is 0 on its first v >= 1 keys and <= -1e30 on the rest, and
// out_valid[r] = min(v, valid[valid_n == 1 ? 0 : r]) then (else the plain valid length, or L).
int tabicl_launch_key_prefix(const float* bias, int64_t bias_sr, int64_t nb, int64_t L, const int32_t* valid,
                             int64_t valid_n, int64_t rows, int32_t* out_valid, int32_t* out_ok,
                             hipStream_t stream);

// Flash attention over [N, H, T, D] views (icl_fwd.hip): D = 64 is the cached-KV ICL attention,
// D = 128 the folded ISAB-1 attention (one head, K = V = the raw rows). qlen (device int32,
// qlen_n in {1, N}): query rows computed per n; rows at or past it are not written (null: all).
// bias: additive fp32 key mask [bias_n, Tkv] (row stride bias_sn, bias_n in {1, N}), added to the
// scaled scores.
int tabicl_launch_icl_fwd(const void* q, const void* k, const void* v, const int32_t* valid,
                          int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq,
                          int64_t Tkv, int64_t D, int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn,
                          int64_t k_sh, int64_t k_st, int64_t v_sn, int64_t v_sh, int64_t v_st,
                          int64_t o_sn, int64_t o_sh, int64_t o_st, float scale, int dtype,
                          void* ws, int64_t ws_bytes, hipStream_t stream,
                          const int32_t* qlen = nullptr, int64_t qlen_n = 0,
                          const float* bias = nullptr, int64_t bias_n = 0, int64_t bias_sn = 0,
                          int list_mode = 0, float* stat = nullptr);
int64_t tabicl_launch_icl_ws_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int dtype);

// Backward of the D = 64 ICL attention (icl_bwd.hip) over contiguous [N, H, T, 64] tensors: dq, dk, dv
// from q, k, v, the forward output o and its gradient dout; valid / bias as in the forward; stat (optional,
// no bias): the forward's per-query (m, l) from tabicl_launch_icl_fwd(..., stat). ws: at least
// tabicl_launch_icl_bwd_ws_bytes(N, H, Tq) bytes (per-query statistics passed between the two kernels).
int64_t tabicl_launch_icl_bwd_ws_bytes(int64_t N, int64_t H, int64_t Tq);
int tabicl_launch_icl_bwd(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                          const float* bias, int64_t bias_n, int64_t bias_sn, const void* o, const void* dout,
                          const float* stat,
                          void* dq, void* dk, void* dv, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, float scale,
                          int dtype, void* ws, int64_t ws_bytes, hipStream_t stream);

// The same launch (D = 64) with the library's per-GPU scratch array of TABICL_ICL_SCRATCH_BYTES in
// place of a workspace: no allocation. Key splits whose partials do not fit run unsplit; a call whose
// unsplit need (tabicl_launch_icl_noalloc_min_bytes) exceeds the array must be refused by the caller.
#define TABICL_ICL_SCRATCH_BYTES (32ll << 20)
int64_t tabicl_launch_icl_noalloc_min_bytes(int64_t N, int64_t H, int64_t Tq, int64_t D, int dtype);
int tabicl_launch_icl_fwd_noalloc(const void* q, const void* k, const void* v, const int32_t* valid,
                                  int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                                  int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                                  int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                                  float scale, int dtype, hipStream_t stream, const int32_t* qlen, int64_t qlen_n,
                                  const float* bias, int64_t bias_n, int64_t bias_sn);

// Small-head (8 x 16) attention (smallhead_fwd.hip): picks the resident, streaming or general
// kernel for the shape. ws may be null (no key split). qlen (device int32, qlen_n in {1, B}): query
// rows needed per batch element; the resident kernel neither computes nor writes the rows at or past
// it, the others compute every row (null: all Lq rows).
int tabicl_launch_smallhead(const void* q, int64_t q_sb, int64_t q_sr, const void* k, int64_t k_sb,
                            int64_t k_sr, const void* v, int64_t v_sb, int64_t v_sr, void* o,
                            const float* bias, int64_t bias_sb, const int32_t* valid,
                            int64_t valid_n, const float* cq, const float* sq, const float* ck,
                            const float* sk, int rope, int half, int rot, float scale, int64_t B,
                            int64_t Lq, int64_t Lk, int dtype, void* ws, int64_t ws_bytes,
                            hipStream_t stream, const int32_t* qlen = nullptr, int64_t qlen_n = 0);
int64_t tabicl_launch_smallhead_ws_bytes(int64_t B, int64_t Lq, int64_t Lk, int dtype, bool bias,
                                         int rope);

// Streaming bf16 small-head kernel without RoPE / key bias (smallhead_stream.hip). gate (device
// int32 [gate_n], gate_n in {1, B}, or null): batch elements whose entry is 0 are skipped (neither
// computed nor written).
int tabicl_launch_ss(const void* q, int64_t q_sb, int64_t q_sr, const void* k, int64_t k_sb,
                     int64_t k_sr, const void* v, int64_t v_sb, int64_t v_sr, void* o,
                     const int32_t* valid, int64_t valid_n, float scale, int64_t B, int64_t Lq,
                     int64_t Lk, void* ws, int64_t ws_bytes, hipStream_t stream,
                     const int32_t* gate = nullptr, int64_t gate_n = 0);
int64_t tabicl_launch_ss_ws_bytes(int64_t B, int64_t Lq, int64_t Lk);

// Backward of the small-head attention (smallhead_bwd.hip): dq, dk, dv (element strides as the
// inputs) from q, k, v, the forward output o and its gradient dout ([B, Lq, E] contiguous both).
// ws: tabicl_launch_smallhead_bwd_ws_bytes(B, Lq) bytes (per-query softmax statistics and D).
int tabicl_launch_smallhead_bwd(const void* q, int64_t q_sb, int64_t q_sr, const void* k, int64_t k_sb,
                                int64_t k_sr, const void* v, int64_t v_sb, int64_t v_sr, const void* o,
                                const void* dout, void* dq, int64_t dq_sb, int64_t dq_sr, void* dk,
                                int64_t dk_sb, int64_t dk_sr, void* dv, int64_t dv_sb, int64_t dv_sr,
                                const float* bias, int64_t bias_sb, const float* cq, const float* sq,
                                const float* ck, const float* sk, int rope, int half, int rot, float scale,
                                int64_t B, int64_t Lq, int64_t Lk, int dtype, void* ws, int64_t ws_bytes,
                                hipStream_t stream);
int64_t tabicl_launch_smallhead_bwd_ws_bytes(int64_t B, int64_t Lq);

// Row LayerNorm (layernorm.hip): rows x width (128 or 512) contiguous, fp32 / bf16 in (dtype codes 0 bf16,
// 1 fp32) and out, fp32 weight / bias (null: 1 / 0); with r, xs = x + r (input dtype) is written and
// normalised.
int tabicl_launch_layer_norm(const void* x, const void* r, void* xs, const float* w, const float* b, void* y,
                             int64_t rows, int64_t width, float eps, int in_dtype, int out_dtype, hipStream_t stream);
