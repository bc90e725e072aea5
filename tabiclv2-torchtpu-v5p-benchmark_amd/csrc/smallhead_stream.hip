// Streaming small-head attention for long key sets (bf16, 8 heads x 16 dims, merged width 128).
//
// This is the column ISAB-1 shape of the reference's hxq op (scripts/tabicl_tpu_pallas_attn.py:
// 223-291, 323-336): 128 inducing queries over tens of thousands of rows read from a packed
// [B, L, 2E] K|V tensor, keys at or past valid_len[b] excluded. It also serves hx / pk_cross calls
// without RoPE or key bias once Lk exceeds what the resident kernel keeps in LDS.
//   O = softmax(q k^T, keys < valid) V   per (batch, head), fp32 scores and softmax, P cast to bf16.
//
// Work decomposition. A workgroup = (batch b, key split s, head group hg of 4 heads, 128 queries);
// 8 waves = 4 heads x 2 halves of 64 queries, each wave four 16-query blocks of one head (<= 128
// VGPRs, two workgroups per CU). Its key range streams through LDS in 64-key tiles (two 32-key
// sub-tiles, one workgroup join per tile) holding K and V of its 4 heads (two whole 128-byte lines
// per key), copied by the load unit itself (global_load_lds_dwordx4) three tiles ahead, with 16-byte
// chunks XOR-swizzled per key so that the LDS operand reads below do not conflict on banks.
//
// Per (16-query block, 32-key sub-tile) a wave runs four v_mfma_f32_16x16x32_bf16:
//   x  = K (q log2e) - m    two MFMAs; the 32-deep contraction holds q*log2e split in a bf16 high
//                           part (k-slots 0..15) and the bf16 rounding remainder (slots 16..31)
//                           against the same K, and the accumulator starts at -m: the MFMA output
//                           is already the exp2 argument, exact to ~2^-17 relative.
//   sum = 1 * p             p = bf16(exp2(x)); a ones operand gives the tile row sum.
//   O^T += V^T P^T          V^T operands come from ds_read_b64_tr_b16 on row-major V.
// so the VALU work per score is one v_exp_f32 and half a conversion.
//
// Softmax reference m (per query and head). The sweep over a split's keys does not track the
// running maximum: m is the (ceiled) maximum over the split's first 32 keys and stays fixed, so p =
// exp2(x) may exceed 1. The row sum l > 1/2 from the first sub-tile on; if at the end of the sweep l <=
// 2^96 and O is finite, every p stayed far inside the bf16/fp32 range and the result equals the
// max-subtracted softmax to rounding (fp32/bf16 relative precision does not depend on scale). A
// score more than ~66 nats above the first sub-tile's maximum (or a NaN / inf) breaks that test; the
// workgroup then sweeps the split again in exact mode, a classic online softmax that moves m by
// exact powers of two. No test or branch runs per tile in the fast sweep.
//
// Key splits write fp32 partial (O, m, l) into a caller workspace; a merge kernel combines them.
#include <atomic>

#include "common.h"

namespace {

constexpr int SS_E = 128;
constexpr int SS_H = 8;
constexpr int SS_HPW = 4;                // heads per workgroup
constexpr int SS_NHG = SS_H / SS_HPW;    // head groups
constexpr int SS_NW = 2 * SS_HPW;        // waves per workgroup: heads x 2 query halves
constexpr int SS_NB = 4;                 // 16-query blocks per wave
constexpr int SS_QG = 2 * 16 * SS_NB;    // queries per workgroup
constexpr int SS_KT = 64;                // keys per tile (one LDS buffer, one join of the sweep)
constexpr int SS_ST = 32;                // keys per sub-tile (one operand set of the products)
constexpr int SS_ROW = 32 * SS_HPW * 2;  // tile row bytes: K then V of the heads, bf16 (256)
constexpr int SS_CPR = SS_ROW / 16;      // 16-byte chunks per row (16)
constexpr int SS_STILE = SS_ST * SS_ROW;  // 8 KB
constexpr int SS_TILE = SS_KT * SS_ROW;   // 16 KB
constexpr int SS_NBUF = 4;
constexpr int SS_MAX_SPLIT = 8;
constexpr int SS_MIN_TILES = 8;          // per key split
constexpr float SS_L_HI = 0x1p96f;   // row-sum bound of the fast sweep

struct SsParams {
  const bf16* q;
  int64_t q_sb, q_sr;
  const bf16* k;
  int64_t k_sb, k_sr;
  const bf16* v;
  int64_t v_sb, v_sr;
  bf16* o;
  int64_t o_sb, o_sr;
  const int32_t* valid;
  int valid_n;
  float scale;
  int B, Lq, Lk;
  int nqg, nsplit, tps;
  float* ws_o;    // [nsplit][B*Lq][E] fp32 partial outputs
  float2* ws_ml;  // [nsplit][B*Lq][H] (m, l), m in log2 units
  // batch elements computed here (gate[b], or gate[0] for all; null: all): the others are neither
  // computed nor merged nor written
  const int32_t* gate;
  int gate_n;
};

// 16-byte chunk swizzle of a 256-byte tile row (key r): physical chunk = logical ^ ss_swz(r), a
// bijection on r mod 16. The 16 K-operand reads of one chunk column (rows r0..r0+15) land on 16
// distinct chunks, and so do the 32 transposed V reads of rows r0..r0+7 (chunk pairs {c, c^1}, c
// even): each covers all 64 banks once.
__device__ __forceinline__ int ss_swz(int r) { return ((2 * (r & 7)) | ((r >> 2) & 1)) ^ ((r >> 3) & 1); }
static_assert(SS_CPR == 16, "swizzle above is for 16 chunks per row");

// Every sweep iteration issues exactly one tile per wave, one copy per sub-tile (past the end of the
// range the last tile is copied again into a buffer nobody reads), so the wait for tile t is always
// "all but the newest SS_NBUF - 2 tiles' copies". The join also waits for this wave's LDS
// operations (the restart flag).
__device__ __forceinline__ void ss_wait_join() {
  static_assert((SS_NBUF - 2) * (SS_KT / SS_ST) == 4, "vmcnt below");
  TA_WAIT_JOIN(4);
}
__device__ __forceinline__ void ss_drain_join() {
  TA_WAIT_JOIN(0);
}

// Per-lane source of the tile copies: lane (row r = 4 * wave + lane / 16, physical chunk lane % 16)
// copies logical chunk (lane % 16) ^ ss_swz(r) of key row k0 + r: K of the head group for chunks
// 0..7, V for 8..15.
struct SsSrc {
  const char* base;  // chunk column of row 0
  uint32_t stride;   // bytes between key rows
  int row;
};

__device__ __forceinline__ SsSrc ss_src(const SsParams& p, int b, int hg, int wave, int lane) {
  constexpr int HALF = SS_CPR / 2;
  SsSrc s;
  s.row = (64 / SS_CPR) * wave + lane / SS_CPR;
  const int lc = (lane % SS_CPR) ^ ss_swz(s.row);
  const bf16* kb = p.k + b * p.k_sb + hg * (SS_HPW * 16);
  const bf16* vb = p.v + b * p.v_sb + hg * (SS_HPW * 16);
  s.base = lc < HALF ? (const char*)(kb + lc * 8) : (const char*)(vb + (lc - HALF) * 8);
  s.stride = (uint32_t)((lc < HALF ? p.k_sr : p.v_sr) * (int64_t)sizeof(bf16));
  return s;
}

// Copy the tile starting at key k0, sub-tile by sub-tile (rows clamped to lk - 1: no key past the
// valid length is read).
__device__ __forceinline__ void ss_issue(const SsSrc& s, uint32_t buf, int k0, int lk, int wave) {
#pragma unroll
  for (int h = 0; h < SS_KT / SS_ST; ++h) {
    const uint32_t key = (uint32_t)min(k0 + SS_ST * h + s.row, lk - 1);
    lds_dma16(s.base + (uint64_t)key * s.stride, buf + SS_STILE * h + 1024 * wave);
  }
}

// Scores x = K (q log2e) - m of one 16-query block over a 32-key sub-tile. Lane (l16, G) holds keys
// key0 + r (x0) and key0 + 16 + r (x1), key0 = tile start + 4G, r = 0..3, of query l16, which is the
// k-slot order 8G + j of the B operand of the 16x16x32 products.
template <bool MASK>
__device__ __forceinline__ void ss_scores(bf16x8 ka0, bf16x8 ka1, bf16x8 q, f32x4 negm, int key0, int lk,
                                          f32x4& x0, f32x4& x1) {
  x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka0, q, negm, 0, 0, 0);
  x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka1, q, negm, 0, 0, 0);
  if (MASK) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (key0 + r >= lk) x0[r] = TA_NEG_INF;
      if (key0 + 16 + r >= lk) x1[r] = TA_NEG_INF;
    }
  }
}

__device__ __forceinline__ bf16x8 ss_exp(f32x4 x0, f32x4 x1, float d) {
  bf16x8 pv;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    pv[r] = (bf16)__builtin_amdgcn_exp2f(x0[r] - d);
    pv[4 + r] = (bf16)__builtin_amdgcn_exp2f(x1[r] - d);
  }
  return pv;
}

__device__ __forceinline__ float ss_tile_sum(bf16x8 ones, bf16x8 pv) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pv, zero, 0, 0, 0)[0];
}

__device__ __forceinline__ float ss_tile_max(f32x4 x0, f32x4 x1) {
  float m = TA_NEG_INF;
#pragma unroll
  for (int r = 0; r < 4; ++r) m = fmaxf(m, fmaxf(x0[r], x1[r]));
  return quad_max(m);
}

// Integer shift ceil(x) clamped to [-1e4, 1e4] (NaN and -inf give 0).
__device__ __forceinline__ float ss_ceil_shift(float x) {
  return x > -1e4f ? fminf(ceilf(x), 1e4f) : 0.f;
}

struct SsState {
  bf16x8 ones;  // all-ones A operand of the row-sum products
  bf16x8 qop[SS_NB];
  f32x4 negm[SS_NB];
  f32x4 o[SS_NB];
  float l[SS_NB];
};

// One tile. Fast mode: p = exp2(x) against the fixed m. Exact mode: per tile, m moves up to the
// tile maximum (by a whole number, so that O and l rescale exactly).
template <bool EXACT, bool MASK>
__device__ __forceinline__ void ss_tile(SsState& st, bf16x8 ka0, bf16x8 ka1, bf16x8 va, int key0, int lk) {
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    f32x4 x0, x1;
    ss_scores<MASK>(ka0, ka1, st.qop[i], st.negm[i], key0, lk, x0, x1);
    bf16x8 pv;
    if (EXACT) {
      const float tmax = ss_tile_max(x0, x1);
      // with nothing accumulated yet m may also move down
      const float d = st.l[i] == 0.f ? ss_ceil_shift(tmax) : fmaxf(ss_ceil_shift(tmax), 0.f);
      if (st.l[i] != 0.f) {
        const float sc = __builtin_amdgcn_ldexpf(1.f, -(int)d);
#pragma unroll
        for (int r = 0; r < 4; ++r) st.o[i][r] *= sc;
        st.l[i] *= sc;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) st.negm[i][r] -= d;
      pv = ss_exp(x0, x1, d);
    } else {
      pv = ss_exp(x0, x1, 0.f);
    }
    st.l[i] += ss_tile_sum(st.ones, pv);
    st.o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pv, st.o[i], 0, 0, 0);
  }
}

// True when this lane's fast-sweep result may not be trusted (see the file comment).
__device__ __forceinline__ bool ss_suspect(const SsState& st) {
  bool bad = false;
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    bad |= !(st.l[i] <= SS_L_HI);
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= !(__builtin_fabsf(st.o[i][r]) <= 0x1p127f);
  }
  return bad;
}

// Operands of one tile from LDS: K for the two 16-key halves, V^T via transposed reads.
__device__ __forceinline__ void ss_operands(const char* buf, int koff, int voff, bf16x8& ka0, bf16x8& ka1,
                                            bf16x8& va) {
  ka0 = *(const bf16x8*)(buf + koff);
  ka1 = *(const bf16x8*)(buf + koff + 16 * SS_ROW);
  const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(buf + voff));
  const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(buf + voff + 16 * SS_ROW));
  const bf16x4 a0 = __builtin_bit_cast(bf16x4, v0), a1 = __builtin_bit_cast(bf16x4, v1);
  va = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
}

// One sweep over the split's tiles [t0, t0 + nt). Fast mode stops early (returns true) once any wave
// of the workgroup has flagged a row sum out of bound; all waves see the flag after the same join.
// Sweep step t: wait for tile t, queue the copy of tile t + SS_NBUF - 1 (clamped to the last tile
// of the range, whose repeated copies land in buffers nobody reads), process tile t.
template <bool EXACT, bool MASK>
__device__ __forceinline__ void ss_step(SsState& st, char* lds, uint32_t lds0, const SsSrc& src, int t0, int t,
                                        int tlast, int lk, int koff, int voff, int wave, int G) {
  ss_wait_join();
  ss_issue(src, lds0 + ((t + SS_NBUF - 1) % SS_NBUF) * SS_TILE, min(t0 + t + SS_NBUF - 1, tlast) * SS_KT, lk,
           wave);
#pragma unroll
  for (int h = 0; h < SS_KT / SS_ST; ++h) {
    const int k0 = (t0 + t) * SS_KT + SS_ST * h;
    if (MASK && k0 >= lk) break;  // a last tile's sub-tiles past the valid length (uniform)
    bf16x8 ka0, ka1, va;
    ss_operands(lds + (t % SS_NBUF) * SS_TILE + SS_STILE * h, koff, voff, ka0, ka1, va);
    ss_tile<EXACT, MASK>(st, ka0, ka1, va, k0 + 4 * G, lk);
  }
}

// One sweep over the split's tiles [t0, t0 + nt), nt >= 1; the last one masks keys past the valid
// length (a no-op unless it is the last tile of the key range).
template <bool EXACT>
__device__ __forceinline__ void ss_sweep(SsState& st, char* lds, const SsSrc& src, int t0, int nt, int lk,
                                         int koff, int voff, int wave, int G) {
  const uint32_t lds0 = lds_addr(lds);
  const int tlast = t0 + nt - 1;
#pragma unroll
  for (int i = 0; i < SS_NBUF - 1; ++i) ss_issue(src, lds0 + i * SS_TILE, min(t0 + i, tlast) * SS_KT, lk, wave);
  for (int t = 0; t < nt - 1; ++t) ss_step<EXACT, false>(st, lds, lds0, src, t0, t, tlast, lk, koff, voff, wave, G);
  ss_step<EXACT, true>(st, lds, lds0, src, t0, nt - 1, tlast, lk, koff, voff, wave, G);
  ss_drain_join();
}

__global__ __launch_bounds__(SS_NW * 64, 2) void ss_stream_kernel(SsParams p) {
  __shared__ __attribute__((aligned(1024))) char lds[SS_NBUF * SS_TILE];
  __shared__ int restart_flag;

  // Work items in the hardware's dispatch order (consecutive items go to different XCDs): items share
  // no K / V (other heads or other key ranges), and per-element valid lengths make elements' items
  // differ in work, which XCD-contiguous ranges of elements would concentrate on some XCDs (C5's
  // ragged ISAB-1 leg: 33.2 ms with XCD-contiguous ranges, 31.0 ms in dispatch order).
  const int work = blockIdx.x;
  const int qg = work % p.nqg;
  int rest = work / p.nqg;
  const int hg = rest % SS_NHG;
  rest /= SS_NHG;
  const int split = rest % p.nsplit;
  const int b = rest / p.nsplit;
  if (p.gate && !p.gate[p.gate_n == 1 ? 0 : b]) return;

  int lk = p.Lk;
  if (p.valid) {
    const int vl = p.valid[p.valid_n == 1 ? 0 : b];
    lk = vl < 0 ? 0 : (vl < lk ? vl : lk);
  }
  const int ntiles = (lk + SS_KT - 1) / SS_KT;
  const int t0 = split * p.tps;
  const int t1 = min(t0 + p.tps, ntiles);
  const int nt = t1 > t0 ? t1 - t0 : 0;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, G = lane >> 4;
  const int gl = wave % SS_HPW, g = hg * SS_HPW + gl;
  const int q0 = qg * SS_QG + (wave / SS_HPW) * (16 * SS_NB);

  // B operands: q*log2e of dims 8(G&1)..+7 of head g, bf16 high part (G < 2) or remainder (G >= 2)
  SsState st;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.ones[j] = (bf16)1.f;
  asm volatile("" : "+v"(st.ones));  // keep it in registers across the sweep, not rebuilt per use
  const bf16* qb = p.q + b * p.q_sb + g * 16 + 8 * (G & 1);
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    const int qi = q0 + 16 * i + l16;
    bf16x8 raw;
#pragma unroll
    for (int j = 0; j < 8; ++j) raw[j] = (bf16)0.f;
    if (qi < p.Lq) raw = *(const bf16x8*)(qb + (int64_t)qi * p.q_sr);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float f = (float)raw[j];
      if (p.scale != 1.f) f = (float)(bf16)(f * p.scale);
      f *= TA_LOG2E;
      const bf16 hi = (bf16)f;
      st.qop[i][j] = G < 2 ? hi : (bf16)(f - (float)hi);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) { st.negm[i][r] = 0.f; st.o[i][r] = 0.f; }
    st.l[i] = 0.f;
  }
  if (threadIdx.x == 0) restart_flag = 0;

  // per-lane operand offsets within a tile (keys 16..31: + 16 rows)
  const int koff = l16 * SS_ROW + (((2 * gl + (G & 1)) ^ ss_swz(l16)) << 4);
  const int vrow = 4 * G + (l16 >> 2), c4 = l16 & 3;
  const int voff =
      vrow * SS_ROW + (((SS_CPR / 2 + 2 * gl + (c4 >> 1)) ^ ss_swz(vrow)) << 4) + 8 * (c4 & 1);
  const SsSrc src = ss_src(p, b, hg, wave, lane);
  const uint32_t lds0 = lds_addr(lds);

  if (nt > 0) {
    // reference m: ceiled maximum over the split's first 32 keys
    ss_issue(src, lds0, t0 * SS_KT, lk, wave);
    ss_drain_join();
    bf16x8 ka0, ka1, va;
    ss_operands(lds, koff, voff, ka0, ka1, va);
#pragma unroll
    for (int i = 0; i < SS_NB; ++i) {
      f32x4 x0, x1;
      ss_scores<true>(ka0, ka1, st.qop[i], st.negm[i], t0 * SS_KT + 4 * G, lk, x0, x1);
      const float d = ss_ceil_shift(ss_tile_max(x0, x1));
#pragma unroll
      for (int r = 0; r < 4; ++r) st.negm[i][r] = -d;
    }
    ss_drain_join();  // everyone has read buffer 0 before the sweep refills it
    ss_sweep<false>(st, lds, src, t0, nt, lk, koff, voff, wave, G);
    if (wave_any(ss_suspect(st))) restart_flag = 1;
    __syncthreads();
    if (restart_flag) {
#pragma unroll
      for (int i = 0; i < SS_NB; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) { st.negm[i][r] = 0.f; st.o[i][r] = 0.f; }
        st.l[i] = 0.f;
      }
      ss_sweep<true>(st, lds, src, t0, nt, lk, koff, voff, wave, G);
    }
  }

  // O^T lane layout: dims 4G..4G+3 of query l16
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    const int qi = q0 + 16 * i + l16;
    if (qi >= p.Lq) continue;
    const int64_t row = (int64_t)b * p.Lq + qi;
    if (p.nsplit == 1) {
      const float inv = st.l[i] == 0.f ? 0.f : 1.f / st.l[i];
      bf16x4 ov;
#pragma unroll
      for (int r = 0; r < 4; ++r) ov[r] = (bf16)(st.o[i][r] * inv);
      *(bf16x4*)(p.o + b * p.o_sb + (int64_t)qi * p.o_sr + g * 16 + 4 * G) = ov;
    } else {
      const int64_t srow = (int64_t)split * p.B * p.Lq + row;
      *(f32x4*)(p.ws_o + srow * SS_E + g * 16 + 4 * G) = st.o[i];
      if (G == 0) p.ws_ml[srow * SS_H + g] = make_float2(-st.negm[i][0], st.l[i]);
    }
  }
}

// Combine the key splits: O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, M = max m_s over the
// splits that saw any key. One thread per (row, head, 4 dims).
__global__ __launch_bounds__(256) void ss_merge_kernel(SsParams p) {
  const int64_t rows = (int64_t)p.B * p.Lq;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * (SS_E / 4)) return;
  const int c = (int)(idx & 31);
  const int64_t row = idx >> 5;
  const int h = c >> 2, d0 = 4 * c;
  if (p.gate && !p.gate[p.gate_n == 1 ? 0 : (int)(row / p.Lq)]) return;
  float m_max = TA_NEG_INF;
  for (int s = 0; s < p.nsplit; ++s) {
    const float2 ml = p.ws_ml[((int64_t)s * rows + row) * SS_H + h];
    if (ml.y != 0.f) m_max = fmaxf(m_max, ml.x);
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const float2 ml = p.ws_ml[((int64_t)s * rows + row) * SS_H + h];
    if (ml.y == 0.f) continue;
    const float w = __builtin_amdgcn_exp2f(ml.x - m_max);
    lsum += w * ml.y;
    const f32x4 os = *(const f32x4*)(p.ws_o + ((int64_t)s * rows + row) * SS_E + d0);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += w * os[r];
  }
  const float inv = lsum == 0.f ? 0.f : 1.f / lsum;
  bf16x4 ov;
#pragma unroll
  for (int r = 0; r < 4; ++r) ov[r] = (bf16)(acc[r] * inv);
  const int b = (int)(row / p.Lq), qi = (int)(row % p.Lq);
  *(bf16x4*)(p.o + b * p.o_sb + (int64_t)qi * p.o_sr + d0) = ov;
}

// Resident streaming workgroups on the current device (CUs x workgroups per CU), queried once per
// device and cached.
int64_t ss_slots() {
  static std::atomic<int64_t> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int64_t hit = cache[dev].load(std::memory_order_relaxed);
    if (hit > 0) return hit;
  }
  int cus = 0, n = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, ss_stream_kernel, SS_NW * 64, 0) != hipSuccess || n < 1) n = 1;
  const int64_t slots = (int64_t)cus * n;
  if (dev >= 0 && dev < 64) cache[dev].store(slots, std::memory_order_relaxed);
  return slots;
}

// Key splits: the fewest that bring the grid within a few percent of whole waves of workgroups
// on the device, each split keeping at least SS_MIN_TILES tiles.
int ss_pick_splits(int64_t items, int64_t Lk) {
  const int64_t slots = ss_slots();
  if (slots <= 0) return 1;
  const int64_t tiles = (Lk + SS_KT - 1) / SS_KT;
  int best = 1;
  double best_cost = (double)((items + slots - 1) / slots);
  for (int s = 2; s <= SS_MAX_SPLIT; ++s) {
    if (tiles / s < SS_MIN_TILES) break;
    const double cost = (double)((items * s + slots - 1) / slots) / s;
    if (cost < best_cost * 0.97) { best = s; best_cost = cost; }
  }
  return best;
}

int64_t ss_items(int64_t B, int64_t Lq) { return B * SS_NHG * ((Lq + SS_QG - 1) / SS_QG); }

}  // namespace

// Workspace bytes the streaming kernel uses to split the keys of (B, Lq, Lk) (0: no split).
int64_t tabicl_launch_ss_ws_bytes(int64_t B, int64_t Lq, int64_t Lk) {
  const int s = ss_pick_splits(ss_items(B, Lq), Lk);
  return s > 1 ? (int64_t)s * B * Lq * (SS_E * 4 + SS_H * 8) : 0;
}

// Streaming kernel launch (bf16 only; q [B, Lq, 128] rows, k / v rows of 128 dims at the given
// batch and row strides, output [B, Lq, 128] contiguous). Without a large enough workspace the
// keys are not split.
int tabicl_launch_ss(const void* q, int64_t q_sb, int64_t q_sr, const void* k, int64_t k_sb,
                     int64_t k_sr, const void* v, int64_t v_sb, int64_t v_sr, void* o,
                     const int32_t* valid, int64_t valid_n, float scale, int64_t B, int64_t Lq,
                     int64_t Lk, void* ws, int64_t ws_bytes, hipStream_t stream, const int32_t* gate,
                     int64_t gate_n) {
  SsParams p;
  p.gate = gate; p.gate_n = (int)gate_n;
  p.q = (const bf16*)q; p.q_sb = q_sb; p.q_sr = q_sr;
  p.k = (const bf16*)k; p.k_sb = k_sb; p.k_sr = k_sr;
  p.v = (const bf16*)v; p.v_sb = v_sb; p.v_sr = v_sr;
  p.o = (bf16*)o; p.o_sb = Lq * SS_E; p.o_sr = SS_E;
  p.valid = valid; p.valid_n = (int)valid_n;
  p.scale = scale;
  p.B = (int)B; p.Lq = (int)Lq; p.Lk = (int)Lk;
  p.nqg = (int)((Lq + SS_QG - 1) / SS_QG);
  const int64_t items = ss_items(B, Lq);
  p.nsplit = ss_pick_splits(items, Lk);
  const int64_t rows = B * Lq;
  if (p.nsplit > 1 && (ws == nullptr || ws_bytes < (int64_t)p.nsplit * rows * (SS_E * 4 + SS_H * 8)))
    p.nsplit = 1;
  const int64_t tiles = (Lk + SS_KT - 1) / SS_KT;
  p.tps = (int)((tiles + p.nsplit - 1) / p.nsplit);
  p.ws_o = (float*)ws;
  p.ws_ml = (float2*)(p.ws_o + (p.nsplit > 1 ? (int64_t)p.nsplit * rows * SS_E : 0));
  const int64_t nblk = items * p.nsplit;
  hipLaunchKernelGGL(ss_stream_kernel, dim3((unsigned)nblk), dim3(SS_NW * 64), 0, stream, p);
  if (p.nsplit > 1) {
    const int64_t threads = rows * (SS_E / 4);
    hipLaunchKernelGGL(ss_merge_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
  }
  return (int)hipGetLastError();
}
