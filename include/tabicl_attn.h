/*
 * tabicl_attn.h - C ABI of the MI355X (gfx950) small-head and cached-KV attention library
 * (libtabicl_attn.so).
 *
 * Every entry point takes raw device pointers, element strides and sizes, a dtype code and a
 * hipStream_t (passed as void* so that this header needs no HIP include). Outputs are allocated by
 * the caller. Return value: 0 = ok, >0 = unsupported shape or argument (the caller falls back),
 * <0 = HIP launch error. tabicl_attn_last_error() gives the message of the last non-zero status
 * on the calling host thread. No entry point synchronizes the stream, allocates device memory or
 * keeps mutable global state; all are safe to call from any host thread.
 *
 * Layout conventions (the reference's merged-head layout): E = h * d with d = 16 for the small-head
 * ops, rows are E (q/k/v), 2E (packed K|V) or 3E (packed Q|K|V) wide, heads are contiguous d-wide
 * column blocks. Softmax is fp32; scores accumulate in fp32; probabilities are cast to the value
 * dtype before the PV product; outputs are written in the query dtype.
 *
 * Empty calls: a batch of 0 elements or 0 query rows returns 0 without any launch (the key count may
 * then be 0 too, e.g. an empty self-attention); otherwise at least one key is required.
 */
#ifndef TABICL_ATTN_H
#define TABICL_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define TABICL_DTYPE_BF16 0
#define TABICL_DTYPE_F32 1

/* RoPE codes, as returned by rope_tables (reference scripts/tabicl_tpu_pallas_attn.py:681-698) */
#define TABICL_ROPE_NONE 0
#define TABICL_ROPE_PAIRS 1
#define TABICL_ROPE_HALVES 2
/* Flag ORed into TABICL_ROPE_PAIRS / _HALVES (forward and backward entry points): cos/sin are [L, E/h]
 * (one head's columns, used for every head) instead of [L, E]. rope_tables tiles the same columns over
 * the heads, so its [:, :E/h] slice is such a table; reading it instead of the tiled [L, E] one cuts
 * the table traffic by h. No counterpart in the reference (its Pallas kernel reads [L, E] tiles). */
#define TABICL_ROPE_SHARED_TABLES 0x10

/* op codes for tabicl_attn_supported */
#define TABICL_OP_HX 0
#define TABICL_OP_HXQ 1
#define TABICL_OP_PK_SELF 2
#define TABICL_OP_PK_CROSS 3
#define TABICL_OP_ICL 4

/*
 * Merged-head small-head attention, q pre-scaled.
 * Replaces tabicl_pk::hx_fwd (reference scripts/tabicl_tpu_pallas_attn.py:179-182, 194, 767-790).
 * q [B, Lq, E], k/v [B, Lk, E] contiguous; bias fp32 [bias_b, Lk] with bias_b in {1, B} or NULL;
 * out [B, Lq, E]. Any Lk >= 1 (the reference caps Lk at 1024; this kernel streams key tiles).
 */
int tabicl_hx_fwd(const void* q, const void* k, const void* v, const float* bias, int64_t bias_b,
                  void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h, int32_t dtype,
                  void* stream);

/*
 * Few queries over many keys with a key-validity length, q pre-scaled, K/V read from the packed
 * [B, Lk, 2E] projection (K = columns [0, E), V = columns [E, 2E)).
 * Replaces tabicl_pk::hxq_fwd (reference scripts/tabicl_tpu_pallas_attn.py:299-306, 323-336).
 * valid: device int32 [valid_n] with valid_n in {1, B} (valid_n = B extends the reference to ragged
 * batches); keys at positions >= valid are ignored; a row with no valid key is written as 0.
 * workspace: optional device buffer of tabicl_hxq_workspace_bytes(...) bytes (16-byte aligned).
 * With it the key range of long inputs may be split over more workgroups and merged by a second
 * kernel on the same stream; NULL (or too small) runs unsplit. Calls that overlap on the GPU must
 * not share a workspace.
 */
int tabicl_hxq_fwd(const int32_t* valid, int64_t valid_n, const void* q, const void* kv, void* out,
                   int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h, int32_t dtype,
                   void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes tabicl_hxq_fwd and tabicl_hxq_fwd_masked can use for these sizes on the current
 * device (0: they never need any). No counterpart in the reference (its Pallas grid needs no scratch
 * in HBM).
 */
int64_t tabicl_hxq_workspace_bytes(int64_t B, int64_t Lq, int64_t Lk, int64_t E, int32_t h,
                                   int32_t dtype);

/*
 * tabicl_hxq_fwd with an additive fp32 key mask key_bias [bias_b, Lk] (bias_b in {1, B}, rows
 * contiguous) in place of, or next to, the valid length (valid may be NULL). The mask is what upstream
 * tabicl builds from a tensor train size on every device but the reference's
 * (results/tpu_patch.diff:1526-1542: 0 below the train size, finfo(dtype).min from there on), so
 * this entry point serves the first ISAB attention when the caller hands over that mask: the
 * reference's routing sends such calls to its fallback paths (scripts/tabicl_tpu_mha.py:328-347).
 * Batch elements whose mask row is a prefix mask (0 on its first v >= 1 keys, <= -1e30 after) run on
 * the valid-length kernel with valid = min(v, valid[b]), decided on the device; any other row adds
 * the mask term by term (slower). With a bf16 input and keys past 128, the prefix path needs a
 * workspace of tabicl_hxq_workspace_bytes(...) bytes; without one every row takes the term-by-term
 * kernel. key_bias == NULL is tabicl_hxq_fwd.
 */
int tabicl_hxq_fwd_masked(const int32_t* valid, int64_t valid_n, const float* key_bias, int64_t bias_b,
                          const void* q, const void* kv, void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                          int32_t h, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Self attention over the packed in-projection qkv [B, L, 3E] with in-kernel RoPE on q and k, then
 * q * scale (fp32, cast to the input dtype), additive fp32 key bias.
 * Replaces tabicl_pk::pk_self_fwd (reference scripts/tabicl_tpu_pallas_attn.py:611-615, 722-732).
 * cos/sin: fp32 [L, E] tables (ignored when rope == TABICL_ROPE_NONE); out [B, L, E].
 */
int tabicl_pk_self_fwd(const void* qkv, const float* bias, int64_t bias_b, const float* cos_t,
                       const float* sin_t, void* out, int64_t B, int64_t L, int64_t E, int32_t h,
                       int32_t rope, int32_t half, int32_t rot, float scale, int32_t dtype,
                       void* stream);

/*
 * Cross attention: q [B, Lq, E] (q_b = 1 broadcasts one query set over the batch), packed kv
 * [B, Lk, 2E]; RoPE with positions 0..Lq-1 on q (cq/sq [Lq, E]) and 0..Lk-1 on k (ck/sk [Lk, E]).
 * Replaces tabicl_pk::pk_cross_fwd (reference scripts/tabicl_tpu_pallas_attn.py:625-630, 735-752).
 */
int tabicl_pk_cross_fwd(const void* q, int64_t q_b, const void* kv, const float* bias,
                        int64_t bias_b, const float* cq, const float* sq, const float* ck,
                        const float* sk, void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                        int32_t h, int32_t rope, int32_t half, int32_t rot, float scale,
                        int32_t dtype, void* stream);

/*
 * tabicl_pk_cross_fwd over a ragged batch: q_len (device int32 [q_len_n], q_len_n in {1, B}) gives
 * the query rows each batch element needs. Rows below q_len[b] equal tabicl_pk_cross_fwd's bit for
 * bit; the contents of rows at or past it are unspecified: the bf16 kernel for Lk <= 128 (the column
 * ISAB-2 shape) neither computes nor writes them, the other kernels compute them. No counterpart in the reference: its shape-bucketed runner
 * (scripts/tabicl_tpu_bucketed.py:36-103, 1287-1397) pads each table's rows to the bucket and
 * computes the padding; callers that know each table's row count pass it here instead.
 */
int tabicl_pk_cross_fwd_ragged(const void* q, int64_t q_b, const void* kv, const float* bias,
                               int64_t bias_b, const float* cq, const float* sq, const float* ck,
                               const float* sk, void* out, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                               int32_t h, int32_t rope, int32_t half, int32_t rot, float scale,
                               int32_t dtype, const int32_t* q_len, int64_t q_len_n, void* stream);

/*
 * Folded first ISAB attention (inference): U = softmax(qf x^T) x, one head of head dim E = 128 over
 * the raw rows x (K = V = x), qf pre-scaled (no scale applied).
 * Replaces tabicl_pk::hxf_fwd (reference scripts/tabicl_tpu_pallas_attn.py:345-404, 414-419, 429-442).
 * qf [q_b, hq, E] with q_b in {1, B} (1: one folded query set shared by every batch element),
 * x [B, Lk, E], out [B, hq, E], contiguous; valid: device int32 [valid_n], valid_n in {1, B} (keys
 * >= valid ignored; a row with no valid key is written as 0). workspace: optional, of
 * tabicl_hxf_workspace_bytes(...) bytes (key splits merged by a second kernel on the same stream).
 */
int tabicl_hxf_fwd(const int32_t* valid, int64_t valid_n, const void* qf, int64_t q_b, const void* x, void* out,
                   int64_t B, int64_t hq, int64_t Lk, int64_t E, int32_t dtype, void* workspace,
                   int64_t workspace_bytes, void* stream);

/*
 * tabicl_hxf_fwd with an additive fp32 key mask key_bias [bias_b, Lk] (bias_b in {1, B}, rows
 * contiguous; NULL: none) added to the scores, and valid optional (NULL: all Lk keys). This lets the
 * folded route serve the first ISAB attention when upstream hands over the train mask it builds from
 * a tensor train size (results/tpu_patch.diff:1526-1542) instead of the length. No counterpart in the
 * reference (its hxf kernel takes the length only, scripts/tabicl_tpu_pallas_attn.py:414-419).
 */
int tabicl_hxf_fwd_masked(const int32_t* valid, int64_t valid_n, const float* key_bias, int64_t bias_b,
                          const void* qf, int64_t q_b, const void* x, void* out, int64_t B, int64_t hq, int64_t Lk,
                          int64_t E, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes tabicl_hxf_fwd can use for these sizes on the current device (0: no key split).
 * No counterpart in the reference (its Pallas grid needs no scratch in HBM). <0 on bad arguments.
 */
int64_t tabicl_hxf_workspace_bytes(int64_t B, int64_t hq, int64_t Lk, int64_t E, int32_t dtype);

/*
 * Backward of the small-head ops (training). Inputs as the forward, plus the forward output o and
 * its gradient dout (both [B, Lq, E], contiguous). P is recomputed in fp32, dS = P (dP - D) with
 * D = sum over the head's dims of dout * o is cast to the input dtype, dq/dk/dv accumulate in fp32
 * and are written in the input dtype; the bias gets no gradient. Keys and queries of any length
 * (the reference stops at 1024 keys).
 * workspace: at least tabicl_smallhead_bwd_workspace_bytes(B, Lq, E, h) bytes of device memory
 * (per-query softmax statistics and D, written and read by the two kernels of one call on `stream`);
 * calls that overlap on the GPU must not share it.
 */
int64_t tabicl_smallhead_bwd_workspace_bytes(int64_t B, int64_t Lq, int64_t E, int32_t h);

/*
 * dq, dk, dv [B, L, E] of hx. Replaces tabicl_pk::hx_bwd (reference
 * scripts/tabicl_tpu_pallas_attn.py:87-122, 185-188, 202-205).
 */
int tabicl_hx_bwd(const void* q, const void* k, const void* v, const float* bias, int64_t bias_b,
                  const void* o, const void* dout, void* dq, void* dk, void* dv, int64_t B, int64_t Lq,
                  int64_t Lk, int64_t E, int32_t h, int32_t dtype, void* workspace,
                  int64_t workspace_bytes, void* stream);

/*
 * d(qkv) [B, L, 3E] packed like qkv: dq = rope_bwd(dq' scale), dk = rope_bwd(dk'), dv, with
 * rope_bwd(y) = y cos - R(y sin). Replaces tabicl_pk::pk_self_bwd (reference
 * scripts/tabicl_tpu_pallas_attn.py:512-531, 554-560, 618-621, 654-657).
 */
int tabicl_pk_self_bwd(const void* qkv, const float* bias, int64_t bias_b, const float* cos_t,
                       const float* sin_t, const void* o, const void* dout, void* dqkv, int64_t B, int64_t L,
                       int64_t E, int32_t h, int32_t rope, int32_t half, int32_t rot, float scale,
                       int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * dq [B, Lq, E] and d(kv) [B, Lk, 2E] packed like kv. With q_b = 1 (one query set broadcast over
 * the batch) dq still holds one gradient per batch element; the caller sums them. Replaces
 * tabicl_pk::pk_cross_bwd (reference scripts/tabicl_tpu_pallas_attn.py:512-553, 633-637, 664-667).
 */
int tabicl_pk_cross_bwd(const void* q, int64_t q_b, const void* kv, const float* bias, int64_t bias_b,
                        const float* cq, const float* sq, const float* ck, const float* sk, const void* o,
                        const void* dout, void* dq, void* dkv, int64_t B, int64_t Lq, int64_t Lk, int64_t E,
                        int32_t h, int32_t rope, int32_t half, int32_t rot, float scale, int32_t dtype,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Dataset-wise in-context attention over cached train-row K/V (head_dim 64).
 * Replaces the Splash hook _tpu_pallas_splash_sdpa / tabicl::tpu_splash_sdpa_{seg,full}
 * (reference results/tpu_patch.diff:95-155; scripts/tabicl_tpu_bucketed.py:221-246).
 * q [N, H, Tq, D], k/v [N, H, Tkv, D], out [N, H, Tq, D]; every tensor has a contiguous last dim and
 * arbitrary element strides for n, h and row (so a [est, block, head, row, d] cache is passed as
 * views). q is NOT pre-scaled: scores are multiplied by `scale` (D^-0.5 in the reference) in fp32.
 * valid: device int32 [valid_n] (valid_n in {1, N}) or NULL (= Tkv): keys >= valid are masked;
 * no padding of q or k is required. A query with no valid key gets output 0.
 * workspace: device memory of at least tabicl_icl_workspace_bytes(...) bytes, or NULL. With it the
 * key range may be split over more workgroups (to fill whole rounds of the GPU) and the partial
 * results merged by a second kernel on the same stream; without it the call runs unsplit. The
 * workspace is scratch: it must not be shared by calls that overlap on the GPU.
 */
int tabicl_icl_fwd(const void* q, const void* k, const void* v, const int32_t* valid,
                   int64_t valid_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                   int64_t D, int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh,
                   int64_t k_st, int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn,
                   int64_t o_sh, int64_t o_st, float scale, int32_t dtype, void* workspace,
                   int64_t workspace_bytes, void* stream);

/*
 * tabicl_icl_fwd over a ragged batch: q_len (device int32 [q_len_n], q_len_n in {1, N}) gives the
 * query rows of each n that are computed. Rows at or past q_len[n] are neither computed nor written
 * (out keeps what it held; no key-split partial is stored or merged for them), and work items
 * (256 query rows x one head) holding none of them exit at once. Rows below q_len[n] equal
 * tabicl_icl_fwd's bit for bit. No counterpart in the reference: its bucketed runner pads the
 * test rows of each table to a test bucket (scripts/tabicl_tpu_bucketed.py:36-103, 1329-1378) and
 * attends with the padding rows too; callers that know each table's test-row count pass it here.
 */
int tabicl_icl_fwd_ragged(const void* q, const void* k, const void* v, const int32_t* valid,
                          int64_t valid_n, const int32_t* q_len, int64_t q_len_n, void* out, int64_t N,
                          int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int64_t q_sn, int64_t q_sh,
                          int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st, int64_t v_sn,
                          int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                          float scale, int32_t dtype, void* workspace, int64_t workspace_bytes,
                          void* stream);

/*
 * Plan of a ragged ICL call: writes the list of live work items (those holding a row below q_len)
 * into `workspace` (at least tabicl_icl_workspace_bytes(N, H, Tq, Tkv, D, dtype) bytes) on `stream`,
 * and nothing else. tabicl_icl_fwd_ragged_listed then takes the list from that workspace instead of
 * computing it, so a caller that repeats one ragged call shape (the 12 ICL blocks of a bucket, one
 * call per block) computes the list once. No counterpart in the reference, whose bucketed runner has
 * no ragged calls. Only bf16 with D = 64 uses a list; for fp32 the call does nothing.
 */
int tabicl_icl_ragged_plan(const int32_t* q_len, int64_t q_len_n, int64_t N, int64_t H, int64_t Tq,
                           int64_t Tkv, int64_t D, int32_t dtype, void* workspace, int64_t workspace_bytes,
                           void* stream);

/*
 * tabicl_icl_fwd_ragged with the live work-item list taken from `workspace`, where an earlier
 * tabicl_icl_ragged_plan call on the same stream left it for the same N, H, Tq, Tkv, D, dtype, q_len
 * contents and workspace_bytes (the workspace is otherwise used as by tabicl_icl_fwd_ragged: each
 * call writes the parts it reads, so calls that follow each other on one stream may share it; calls
 * that overlap race). A stale list (q_len changed since the plan) leaves rows unwritten. Results equal
 * tabicl_icl_fwd_ragged's bit for bit. No counterpart in the reference.
 */
int tabicl_icl_fwd_ragged_listed(const void* q, const void* k, const void* v, const int32_t* valid,
                                 int64_t valid_n, const int32_t* q_len, int64_t q_len_n, void* out, int64_t N,
                                 int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int64_t q_sn, int64_t q_sh,
                                 int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st, int64_t v_sn,
                                 int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                                 float scale, int32_t dtype, void* workspace, int64_t workspace_bytes,
                                 void* stream);

/*
 * tabicl_icl_fwd_ragged with an additive fp32 key mask (NULL: none): key_bias [bias_n, Tkv] with
 * bias_n in {1, N}, row stride bias_sn elements, keys contiguous, added to the scaled scores
 * (softmax(scale q k^T + mask) v, the reference's attn_mask path, results/tpu_patch.diff:263-270,
 * 158-193, which sends every masked call to a torch fallback). Rows of N whose mask is a prefix mask
 * (0 on the first v >= 1 keys, <= -1e30 after: what upstream builds from a tensor train size,
 * diff:1526-1542) run on the pipelined kernel as the valid length min(v, valid[n]), decided on the
 * device; other rows run on the pipelined kernel's masked instance, which adds each key's mask term
 * to its scores (bf16 with a power-of-two scale and a workspace), or on the exact kernel, which also
 * takes the rows the masked instance cannot keep (every key carrying <= -1e30 gives equal weights,
 * like the reference's softmax over finfo.min terms). scale must be positive with a mask. q_len may
 * be NULL (all rows).
 */
int tabicl_icl_fwd_masked(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                          const float* key_bias, int64_t bias_n, int64_t bias_sn, const int32_t* q_len,
                          int64_t q_len_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                          int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                          int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                          float scale, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * tabicl_icl_fwd that also writes each query row's softmax statistics for tabicl_icl_bwd: stat
 * [N, H, Tq, 2] fp32 (contiguous, 16-byte aligned) receives (m, l), m in log2 units and l the sum over
 * the visible keys of exp2(scale log2(e) q.k - m) (l = 0: no visible key). The forward half of the
 * reference's gradient path (autograd through _tiled_online_sdpa, results/tpu_patch.diff:158-193,
 * routed at :263-270), whose saved tensors the backward uses; no key mask (masked calls with a gradient
 * use tabicl_icl_fwd_masked and take their statistics in the backward).
 */
int tabicl_icl_fwd_stats(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                         void* out, float* stat, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                         int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                         int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                         float scale, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Gradients of the ICL attention O = softmax(scale q k^T + mask) v (keys at or past valid[n] masked,
 * key_bias as in tabicl_icl_fwd_masked or NULL): dq, dk, dv [N, H, T, 64] from q, k, v, the forward
 * output o and its gradient dout, all contiguous [N, H, T, 64] (T = Tq for q, o, dout, dq; Tkv for k, v,
 * dk, dv) in one dtype. P is recomputed in fp32; dS = P (dP - D) with D = sum over the head's dims of
 * dout * o, rounded to the input dtype; dq = scale dS k, dk = scale dS^T q, dv = P^T dout (fp32
 * accumulation); keys at or past valid get zero gradients. Replaces the gradient of the reference's
 * autograd fallback for masked / grad-enabled long-key ICL attention, _tiled_online_sdpa
 * (results/tpu_patch.diff:158-193, routed at :263-270). stat: NULL, or (calls without key_bias) the
 * statistics tabicl_icl_fwd_stats wrote for this o; the bf16 path then skips its own statistics sweep
 * over the keys. workspace: at least tabicl_icl_bwd_workspace_bytes(N, H, Tq) bytes of device memory
 * (16-byte aligned); calls that overlap on the GPU must not share it.
 */
int64_t tabicl_icl_bwd_workspace_bytes(int64_t N, int64_t H, int64_t Tq);
int tabicl_icl_bwd(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                   const float* key_bias, int64_t bias_n, int64_t bias_sn, const void* o, const void* dout,
                   const float* stat, void* dq, void* dk, void* dv, int64_t N, int64_t H, int64_t Tq, int64_t Tkv,
                   int64_t D, float scale, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * tabicl_icl_fwd_masked without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart
 * in the reference. The key-split partials, work-item flags and the prefix view of a key mask live in
 * a file-scope device array of the library, one per GPU, of tabicl_icl_noalloc_scratch_bytes() bytes
 * (32 MiB), held until the process ends; the entry point itself calls no allocating routine. Calls
 * whose split partials do not fit run with the keys unsplit (the results then differ from
 * tabicl_icl_fwd's split result by rounding only); a call that needs more than the array even unsplit
 * (more than ~8M work items of 256 query rows x one head) returns 1 with a message. Every call on a GPU
 * shares that GPU's array and keeps no state in it between calls (each kernel writes every entry it
 * later reads): calls that overlap on one GPU (other streams, other host threads) race.
 */
int tabicl_icl_fwd_noalloc(const void* q, const void* k, const void* v, const int32_t* valid, int64_t valid_n,
                           const float* key_bias, int64_t bias_n, int64_t bias_sn, const int32_t* q_len,
                           int64_t q_len_n, void* out, int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                           int64_t q_sn, int64_t q_sh, int64_t q_st, int64_t k_sn, int64_t k_sh, int64_t k_st,
                           int64_t v_sn, int64_t v_sh, int64_t v_st, int64_t o_sn, int64_t o_sh, int64_t o_st,
                           float scale, int32_t dtype, void* stream);

/* Bytes of the per-GPU scratch array tabicl_icl_fwd_noalloc uses (no counterpart in the reference). */
int64_t tabicl_icl_noalloc_scratch_bytes(void);

/*
 * Workspace size (bytes) that tabicl_icl_fwd uses for these sizes on the current device: for bf16
 * with D = 64, the per-work-item trust flags, the prefix view of a key mask and the list of live
 * work items of ragged calls; plus the fp32 key-split partials when the launch splits the keys (0
 * for an fp32 call that does not split). Queries the device's CU count and occupancy; no device
 * memory is touched. Returns <0 on bad arguments.
 */
int64_t tabicl_icl_workspace_bytes(int64_t N, int64_t H, int64_t Tq, int64_t Tkv, int64_t D,
                                   int32_t dtype);

/*
 * Fit-time cache append: copies rows [0, T) of one block's K and V (src [N, H, T, D] with element
 * strides) into rows [row0, row0 + T) of that block's slice of the [N, NB, H, cap, D] caches
 * (dst pointers already offset to the block; element strides dst_sn, dst_sh, row stride D).
 * Replaces the per-block `k_l.to(cache_dtype)` stores of the prefill
 * (reference scripts/tabicl_tpu_bucketed.py:659-692, 736-764). src and dst share the dtype.
 */
int tabicl_icl_cache_append(void* k_cache, void* v_cache, int64_t dst_sn, int64_t dst_sh,
                            int64_t row0, int64_t cap, const void* k_src, const void* v_src,
                            int64_t src_sn, int64_t src_sh, int64_t src_st, int64_t N, int64_t H,
                            int64_t T, int64_t D, int32_t dtype, void* stream);

/*
 * Shape predicate, mirroring supported / hxq_supported / packed_supported
 * (reference scripts/tabicl_tpu_pallas_attn.py:319-320, 715-719, 762-764). Returns 1 if the op
 * accepts the shape, 0 otherwise. Lq/Lk are query/key lengths, E the merged width (ICL: head dim).
 */
int tabicl_attn_supported(int32_t op, int64_t Lq, int64_t Lk, int64_t E, int32_t h, int32_t dtype);

/* Message of the last non-zero status returned on this host thread ("" if none). */
const char* tabicl_attn_last_error(void);

/* Library version string. */
const char* tabicl_attn_version(void);

/*
 * Row LayerNorm of the layers around the attention in the cached-KV query (the column, row and ICL
 * blocks' pre-norms, the row stage's out-norm and the final norm): upstream's SafeLayerNorm
 * (results/tpu_patch.diff:1385-1397, normalising in its fp32 weights' dtype). out = (s - mean)
 * rsqrt(var + eps) weight + bias per row of `width` (128 or 512) values, rows contiguous, mean and biased
 * variance in fp32; s = x, or with `residual` non-NULL s = x + residual rounded to the input dtype and
 * also written to x_out (which may alias x). in_dtype / out_dtype: 0 bf16, 1 fp32; weight / bias fp32
 * [width] or NULL (1 / 0). All pointers 16-byte aligned. Returns 0, >0 unsupported, <0 HIP error.
 */
int tabicl_layer_norm(const void* x, const void* residual, void* x_out, const float* weight, const float* bias,
                      void* out, int64_t rows, int64_t width, float eps, int32_t in_dtype, int32_t out_dtype,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TABICL_ATTN_H */
