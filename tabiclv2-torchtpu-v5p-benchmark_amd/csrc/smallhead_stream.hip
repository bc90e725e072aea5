// Streaming small-head attention for long key sets (bf16, 8 heads x 16 dims, merged width 128).
//
// This is the column ISAB-1 shape of the reference's hxq op (scripts/tabicl_tpu_pallas_attn.py:
// 223-291, 323-336): 128 inducing queries over tens of thousands of rows read from a packed
// [B, L, 2E] K|V tensor, keys at or past valid_len[b] excluded. It also serves hx / pk_cross calls
// without RoPE or key bias once Lk exceeds what the resident kernel keeps in LDS.
//   O = softmax(q k^T, keys < valid) V   per (batch, head), fp32 scores and softmax, P cast to bf16.
//
// Work decomposition. A workgroup = (batch b, key split s, head pair hg, 128 queries); 4 waves =
// 2 heads x 2 halves of 64 queries, each wave four 16-query blocks of one head (145 VGPRs: three
// workgroups per CU). Its key range streams through LDS in 32-key tiles holding K and V of its 2
// heads (128 bytes per key, so every K/V byte is read from HBM once), copied by the load unit
// itself (global_load_lds_dwordx4) seven tiles ahead, with 16-byte chunks XOR-swizzled per key so
// that the LDS operand reads below do not conflict on banks.
//
// Per (16-query block, 32-key tile) a wave runs four v_mfma_f32_16x16x32_bf16:
//   x  = K (q log2e) - m    two MFMAs; the 32-deep contraction holds q*log2e split in a bf16 high
//                           part (k-slots 0..15) and the bf16 rounding remainder (slots 16..31)
//                           against the same K, and the accumulator starts at -m: the MFMA output
//                           is already the exp2 argument, exact to ~2^-17 relative.
//   sum = 1 * p             p = bf16(exp2(x)); a ones operand gives the tile row sum.
//   O^T += V^T P^T          V^T operands come from ds_read_b64_tr_b16 on row-major V.
// so the VALU work per score is one v_exp_f32 and half a conversion.
//
// Softmax reference m (per query and head). m is not the running maximum: it starts at 0 and is
// only moved when the running row sum l + sum would leave [2^-64, 2^64] (or is not finite). Then
// the tile is recomputed against m' = m + ceil(max(tile max, log2 l)) and O, l are scaled by the
// exact power of two 2^(m - m'). Between moves p <= 2^64, far inside the bf16/fp32 range, and the
// relative precision of every p is that of fp32/bf16 at any scale, so the result equals the
// max-subtracted softmax to rounding. The first tile of every split takes this path once.
//
// Key splits write fp32 partial (O, m, l) into a caller workspace; a merge kernel combines them.
#include "common.h"

namespace {

constexpr int SS_E = 128;
constexpr int SS_H = 8;
constexpr int SS_HPW = 2;                // heads per workgroup
constexpr int SS_NHG = SS_H / SS_HPW;    // head groups
constexpr int SS_NW = 2 * SS_HPW;        // waves per workgroup: heads x 2 query halves
constexpr int SS_NB = 4;                 // 16-query blocks per wave
constexpr int SS_QG = 2 * 16 * SS_NB;    // queries per workgroup
constexpr int SS_KT = 32;                // keys per tile
constexpr int SS_ROW = 32 * SS_HPW * 2;  // tile row bytes: K then V of the heads, bf16 (128)
constexpr int SS_CPR = SS_ROW / 16;      // 16-byte chunks per row (8)
constexpr int SS_TILE = SS_KT * SS_ROW;  // 4 KB
constexpr int SS_NBUF = 8;
constexpr int SS_MAX_SPLIT = 8;
constexpr int SS_MIN_TILES = 16;         // per key split
constexpr float SS_L_HI = 0x1p64f;
constexpr float SS_L_LO = 0x1p-64f;

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
};

// 16-byte chunk swizzle of a 128-byte tile row (key r): physical chunk = logical ^ ss_swz(r).
// The 16 K-operand reads of one chunk column (rows r0..r0+15) and the 32 transposed V reads of
// rows r0..r0+7 (chunk pairs {c, c^1}) each cover 16 distinct (row parity, chunk) bank slots of a
// 256-byte bank line.
__device__ __forceinline__ int ss_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// One 16-byte global -> LDS copy per lane: LDS[lds_addr + 16 * lane] = *src (lds_addr wave-uniform).
// Issued as inline assembly so that the compiler does not wait for it before unrelated LDS reads;
// the kernel waits with explicit vmcnt counts. M0 holds nothing else in this kernel.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void ss_dma(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's tile copies are outstanding, then join the workgroup: after
// it, every wave's copy of the tile N+1 copies back is in LDS and every wave has finished reading
// the buffer the next copy overwrites.
#define SS_WAIT_JOIN(N) asm volatile("s_waitcnt vmcnt(" #N ")\n\ts_barrier" ::: "memory")
__device__ __forceinline__ void ss_wait_join(int n) {
  static_assert(SS_NBUF - 2 == 6, "one case per possible count");
  switch (n) {
    case 0: SS_WAIT_JOIN(0); break;
    case 1: SS_WAIT_JOIN(1); break;
    case 2: SS_WAIT_JOIN(2); break;
    case 3: SS_WAIT_JOIN(3); break;
    case 4: SS_WAIT_JOIN(4); break;
    case 5: SS_WAIT_JOIN(5); break;
    default: SS_WAIT_JOIN(6); break;
  }
}
#undef SS_WAIT_JOIN

// Copy tile rows 8*wave .. 8*wave+7 (keys k0 + row, clamped to lk - 1 so that no key past the
// valid length is read) of the heads at kb / vb into the tile buffer at LDS byte address buf.
__device__ __forceinline__ void ss_issue(const bf16* kb, const bf16* vb, int64_t k_sr, int64_t v_sr,
                                         uint32_t buf, int k0, int lk, int wave, int lane) {
  constexpr int HALF = SS_CPR / 2;
  const int row = (64 / SS_CPR) * wave + lane / SS_CPR;
  const int lc = (lane % SS_CPR) ^ ss_swz(row);
  const int64_t key = min(k0 + row, lk - 1);
  const bf16* src = lc < HALF ? kb + key * k_sr + lc * 8 : vb + key * v_sr + (lc - HALF) * 8;
  ss_dma(src, buf + 1024 * wave);
}

// p = bf16(exp2(x)) of one 16-query block over a 32-key tile. Lane (l16, G) holds keys
// key0 + r and key0 + 16 + r (key0 = tile start + 4G, r = 0..3) of query l16, which is the
// k-slot order 8G + j of the B operand of the 16x16x32 products.
template <bool MASK>
__device__ __forceinline__ bf16x8 ss_probs(bf16x8 ka0, bf16x8 ka1, bf16x8 q, f32x4 negm, int key0,
                                           int lk) {
  const f32x4 x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka0, q, negm, 0, 0, 0);
  const f32x4 x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka1, q, negm, 0, 0, 0);
  bf16x8 pv;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float e0 = x0[r], e1 = x1[r];
    if (MASK) {
      if (key0 + r >= lk) e0 = TA_NEG_INF;
      if (key0 + 16 + r >= lk) e1 = TA_NEG_INF;
    }
    pv[r] = (bf16)__builtin_amdgcn_exp2f(e0);
    pv[4 + r] = (bf16)__builtin_amdgcn_exp2f(e1);
  }
  return pv;
}

__device__ __forceinline__ float ss_tile_sum(bf16x8 pv) {
  const bf16x8 ones = {(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f,
                       (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pv, zero, 0, 0, 0)[0];
}

__device__ __forceinline__ bool ss_out_of_range(float nl) { return !(nl >= SS_L_LO && nl <= SS_L_HI); }

// Move the reference m of the queries whose running sum left the range (see the file comment),
// rescale their O and l exactly, and recompute p and the new running sum for this tile.
template <bool MASK>
__device__ __forceinline__ void ss_rebase(bf16x8 ka0, bf16x8 ka1, bf16x8 q, f32x4& negm,
                                                    f32x4& o, float& l, bf16x8& pv, float& nl,
                                                    int key0, int lk) {
  const bool bad = ss_out_of_range(nl);
  const f32x4 x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka0, q, negm, 0, 0, 0);
  const f32x4 x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka1, q, negm, 0, 0, 0);
  float mx = TA_NEG_INF;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (!MASK || key0 + r < lk) mx = fmaxf(mx, x0[r]);
    if (!MASK || key0 + 16 + r < lk) mx = fmaxf(mx, x1[r]);
  }
  mx = quad_max(mx);
  // l < 2^el; l == 0 (nothing accumulated yet) puts no bound on the new reference
  const float el = (float)__builtin_amdgcn_frexp_expf(l);
  float ref = l != 0.f ? fmaxf(mx, el) : mx;
  ref = fminf(fmaxf(ref, -1e4f), 1e4f);
  const int d = bad ? (int)ceilf(ref) : 0;
  if (d != 0) {
    const float sc = __builtin_amdgcn_ldexpf(1.f, -d);
    if (l != 0.f) {
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] *= sc;
      l *= sc;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) negm[r] -= (float)d;
  }
  pv = ss_probs<MASK>(ka0, ka1, q, negm, key0, lk);
  nl = l + ss_tile_sum(pv);
}

template <bool MASK>
__device__ __forceinline__ void ss_tile(bf16x8 ka0, bf16x8 ka1, bf16x8 va, const bf16x8 (&qop)[SS_NB],
                                        f32x4 (&negm)[SS_NB], f32x4 (&o)[SS_NB], float (&l)[SS_NB],
                                        int key0, int lk) {
  bf16x8 pv[SS_NB];
  float nl[SS_NB];
  bool bad = false;
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    pv[i] = ss_probs<MASK>(ka0, ka1, qop[i], negm[i], key0, lk);
    nl[i] = l[i] + ss_tile_sum(pv[i]);
    bad |= ss_out_of_range(nl[i]);
  }
  if (wave_any(bad)) {
#pragma unroll
    for (int i = 0; i < SS_NB; ++i)
      if (wave_any(ss_out_of_range(nl[i])))
        ss_rebase<MASK>(ka0, ka1, qop[i], negm[i], o[i], l[i], pv[i], nl[i], key0, lk);
  }
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    l[i] = nl[i];
    o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pv[i], o[i], 0, 0, 0);
  }
}

__global__ __launch_bounds__(SS_NW * 64, 3) void ss_stream_kernel(SsParams p) {
  __shared__ __attribute__((aligned(1024))) char lds[SS_NBUF * SS_TILE];

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qg = work % p.nqg;
  int rest = work / p.nqg;
  const int hg = rest % SS_NHG;
  rest /= SS_NHG;
  const int split = rest % p.nsplit;
  const int b = rest / p.nsplit;

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
  bf16x8 qop[SS_NB];
  f32x4 negm[SS_NB], o[SS_NB];
  float l[SS_NB];
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
      qop[i][j] = G < 2 ? hi : (bf16)(f - (float)hi);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) { negm[i][r] = 0.f; o[i][r] = 0.f; }
    l[i] = 0.f;
  }

  const bf16* kb = p.k + b * p.k_sb + hg * (SS_HPW * 16);
  const bf16* vb = p.v + b * p.v_sb + hg * (SS_HPW * 16);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)lds;
#pragma unroll
  for (int i = 0; i < SS_NBUF - 1; ++i)
    if (i < nt) ss_issue(kb, vb, p.k_sr, p.v_sr, lds0 + i * SS_TILE, (t0 + i) * SS_KT, lk, wave, lane);

  // per-lane operand offsets within a tile (keys 16..31: + 16 rows)
  const int koff = l16 * SS_ROW + (((2 * gl + (G & 1)) ^ ss_swz(l16)) << 4);
  const int vrow = 4 * G + (l16 >> 2), c4 = l16 & 3;
  const int voff =
      vrow * SS_ROW + (((SS_CPR / 2 + 2 * gl + (c4 >> 1)) ^ ss_swz(vrow)) << 4) + 8 * (c4 & 1);

  for (int t = 0; t < nt; ++t) {
    // copies issued after tile t: min(nt - 1 - t, SS_NBUF - 2)
    ss_wait_join(min(nt - 1 - t, SS_NBUF - 2));
    if (t + SS_NBUF - 1 < nt)
      ss_issue(kb, vb, p.k_sr, p.v_sr, lds0 + ((t + SS_NBUF - 1) % SS_NBUF) * SS_TILE,
               (t0 + t + SS_NBUF - 1) * SS_KT, lk, wave, lane);
    const char* buf = lds + (t % SS_NBUF) * SS_TILE;
    const bf16x8 ka0 = *(const bf16x8*)(buf + koff);
    const bf16x8 ka1 = *(const bf16x8*)(buf + koff + 16 * SS_ROW);
    const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(buf + voff));
    const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(buf + voff + 16 * SS_ROW));
    const bf16x4 va0 = __builtin_bit_cast(bf16x4, v0), va1 = __builtin_bit_cast(bf16x4, v1);
    const bf16x8 va = {va0[0], va0[1], va0[2], va0[3], va1[0], va1[1], va1[2], va1[3]};
    const int key0 = (t0 + t) * SS_KT + 4 * G;
    if (t0 + t == ntiles - 1)
      ss_tile<true>(ka0, ka1, va, qop, negm, o, l, key0, lk);
    else
      ss_tile<false>(ka0, ka1, va, qop, negm, o, l, key0, lk);
  }

  // O^T lane layout: dims 4G..4G+3 of query l16
#pragma unroll
  for (int i = 0; i < SS_NB; ++i) {
    const int qi = q0 + 16 * i + l16;
    if (qi >= p.Lq) continue;
    const int64_t row = (int64_t)b * p.Lq + qi;
    if (p.nsplit == 1) {
      const float inv = l[i] == 0.f ? 0.f : 1.f / l[i];
      bf16x4 ov;
#pragma unroll
      for (int r = 0; r < 4; ++r) ov[r] = (bf16)(o[i][r] * inv);
      *(bf16x4*)(p.o + b * p.o_sb + (int64_t)qi * p.o_sr + g * 16 + 4 * G) = ov;
    } else {
      const int64_t srow = (int64_t)split * p.B * p.Lq + row;
      *(f32x4*)(p.ws_o + srow * SS_E + g * 16 + 4 * G) = o[i];
      if (G == 0) p.ws_ml[srow * SS_H + g] = make_float2(-negm[i][0], l[i]);
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

int ss_blocks_per_cu() {
  static int cached = 0;
  if (cached > 0) return cached;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, ss_stream_kernel, SS_NW * 64, 0) != hipSuccess || n < 1)
    n = 1;
  cached = n;
  return n;
}

// Key splits: the fewest that bring the grid within a few percent of whole waves of workgroups
// on the device, each split keeping at least SS_MIN_TILES tiles.
int ss_pick_splits(int64_t items, int64_t Lk) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 1;
  const int64_t slots = (int64_t)cus * ss_blocks_per_cu();
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
                     int64_t Lk, void* ws, int64_t ws_bytes, hipStream_t stream) {
  SsParams p;
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
