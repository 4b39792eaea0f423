// Split-K ("flash-decoding") attention for decode, speculative verify and every other
// small-T or fp32 call (include/forge_attn.h: forge_attn_decode).
//
// Work split. For one (batch row b, KV head) the G = H/K query heads times the T new
// queries form G*T "rows" (query-major: row = t*G + head-in-group); a block takes ROWS
// of them (the GQA fan-out: every K/V row is loaded once and used for all ROWS rows,
// in registers) and one chunk of `chunk` keys at absolute positions
// [c*chunk, (c+1)*chunk). Grid = (chunks, K * row-blocks, B).
//
// Inside a block, LPR = D / VEC lanes share one key row: each lane loads 16 bytes
// (VEC elements) of K and of V with one 128-bit load, so a group of LPR lanes reads a
// whole row. Per iteration, group g takes the NK keys kb0 + u*NG + g (u < NK), so each
// load instruction of a wave reads 64 / LPR consecutive rows (1 KB for D = 128). A
// rotating set of register buffers keeps the loads of the next iterations in flight while
// one is scored, and the q rows are requested before them, so HBM latency overlaps the
// math.
// Scores use v_dot2_f32_{bf16,f16} on packed q/k pairs and a DPP butterfly over the LPR
// lanes; the online softmax keeps a reference max that only moves when a score exceeds
// it by 2^8 (kRescaleLog2), so the rescale of (l, o) is rare. Groups are then merged
// (xor-shuffles in a wave, LDS across the 4 waves, fixed order) and the block writes the
// final output (the row sees only this chunk) or an fp32 partial (m, l, o).
//
// Determinism: the key -> (group, slot) assignment depends only on the key's absolute
// position, a key outside a row's visible range is an exact no-op on that row's state
// (score -inf -> weight 0, reference max unchanged), and merges run in a fixed order. So
// a row's output does not depend on T or on the other rows in the call: a verify row
// equals the decode of that token alone, bit for bit (same chunk).
#include <limits.h>
#include <stdio.h>

#include <mutex>

#include "common.h"
#include "forge_internal.h"

namespace forge {

#ifndef FORGE_SPLIT_NK
#define FORGE_SPLIT_NK 2
#endif
constexpr int kSplitThreads = 256;
constexpr int kSplitNK = FORGE_SPLIT_NK;  // keys per group per iteration
constexpr int kMaxChunk = 1024;
// ... but at least this many block iterations per unit: at head dim 32 (128 keys per
// iteration in bf16) 1024 keys are only 8, and 2048-key chunks stream C4's lengths at 16 q /
// 8 KV heads in 169 us against 189 us (at head dim 64, 16 iterations = 1024 keys, 2048 and
// 4096 were slower: 321 and 330 against 315 us).
constexpr int kMinMaxChunkIters = 16;
__host__ __device__ constexpr int max_chunk_keys(int kpi) {
  return kMaxChunk > kMinMaxChunkIters * kpi ? kMaxChunk : kMinMaxChunkIters * kpi;
}
constexpr float kRescaleLog2 = 8.0f;  // lazy rescale: weights stay <= 2^8
// Register buffers of the K/V pipeline (loads run PF - 1 iterations ahead): deeper where
// few query rows leave the registers for it. Measured on C4-shaped ragged decode: PF 4
// at 3 waves per SIMD streams faster than PF 3 at 4; at 3-4 rows per block PF 4 at 2 waves
// per SIMD (190 VGPRs) beats PF 3 at 3 (C4 lengths, 12 q / 4 KV heads: 339 against 355 us
// per step; 16 q / 8 KV heads at T = 2: 669 against 685 us; 8 q / 8 KV heads at T = 4: 668
// against 689 us; C2 19.6 against 19.8 us per graph-replayed call).
template <int ROWS> constexpr int split_pf() { return ROWS <= 4 ? 4 : 3; }
// New positions one lane group may hold in a call of forge_attn_decode_append (T up to
// kNewPerLane times the key groups of the block; the host checks it).
constexpr int kNewPerLane = 2;

struct SplitParams {
  const void* q;
  int64_t sqb, sqh, sqt;
  const float* qw;
  float eps;
  int flags;
  const float* cos;
  const float* sin;
  int64_t csb, cst;
  const void* kc;
  const void* vc;
  int64_t skb, skh, sks;
  int64_t max_len;
  const int32_t* row_pos;
  const int64_t* pos_dev;
  int64_t pos0;
  int B, T, H, K, G;
  int rows_total;  // G * T
  int window;
  float scale_log2;  // softmax scale * log2(e)
  int chunk;
  int max_chunks;
  void* out;
  int64_t sob, sot, soh;
  int persist;    // 1: persistent grid walking the unit list (splitk_kernel)
  int vec_tables; // 1: cos/sin rows and q gains are 16-byte aligned (vector loads)
  int small_dma;  // 1: q rows and tables may be fetched by 16-byte DMA with 32-bit offsets
  int span_chunks;  // dense grid of a windowed layer: blockIdx.x counts chunks from the unit's
                    // first visible one (the grid covers only the chunks a window can touch);
                    // 0: blockIdx.x is the absolute chunk
  float2* ws_ml;  // [B*H*T][max_chunks] (m, l)
  float* ws_o;    // [B*H*T][max_chunks][D]
  int* ws_ctr;    // work ticket of the persistent grid (zero when the split kernel starts), or null
  int ws_zeroed;  // 1: the caller's workspace already holds a zero ticket (no reset kernel)
  // The new tokens' raw keys and values (forge_attn_decode_append), or null: the unit whose
  // chunk holds a new position makes that key (norm + RoPE) and value (norm), writes them
  // into the cache and then streams its chunk (one row block per KV head: the only reader).
  const void* kn;
  const void* vn;
  int64_t sknb, sknh, sknt, svnb, svnh, svnt;
  const float* kw;  // gain of the key norm, or null
  int kvflags;      // FORGE_NORM_QK / FORGE_ROPE for the keys, FORGE_NORM_V for the values
  void* kcw;        // the caches, written
  void* vcw;
};

// Eight fp32 values: two 16-byte loads when the caller's tables allow it (a block-uniform
// flag), else scalar loads of the same values.
__device__ __forceinline__ void load_f32x8_any(const float* ptr, float* out, bool vec) {
  if (vec) {
    load_f32x8(ptr, out);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = ptr[e];
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Visible key range [kmin, kmax] of the query at absolute position qpos.
__device__ __forceinline__ void visible_range(int64_t qpos, int window, int64_t max_len,
                                              int64_t& kmin, int64_t& kmax) {
  kmax = qpos < max_len - 1 ? qpos : max_len - 1;
  kmin = window > 0 ? qpos - window + 1 : 0;
  if (kmin < 0) kmin = 0;
}

__device__ __forceinline__ void visible_range32(int qpos, int window, int max_len, int& kmin,
                                                int& kmax) {
  kmax = qpos < max_len - 1 ? qpos : max_len - 1;
  kmin = window > 0 ? qpos - window + 1 : 0;
  if (kmin < 0) kmin = 0;
}

// q . k over one lane's 16 bytes. bf16/fp16: packed dot2 on the raw pairs (products
// exact in fp32); fp32: four FMAs.
template <typename T>
__device__ __forceinline__ float dot16(const uint4& qraw, const uint4& kraw, float acc) {
  const unsigned qa[4] = {qraw.x, qraw.y, qraw.z, qraw.w};
  const unsigned ka[4] = {kraw.x, kraw.y, kraw.z, kraw.w};
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(__uint_as_float(qa[j]), __uint_as_float(ka[j]), acc);
  } else if constexpr (__is_same(T, bf16)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qa[j]),
                                            __builtin_bit_cast(bf16x2_t, ka[j]), acc, false);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qa[j]),
                                   __builtin_bit_cast(f16x2_t, ka[j]), acc, false);
  }
  return acc;
}

// 16 bytes of V as VEC floats (bf16 -> fp32 is a shift / mask of the raw bits).
template <typename T>
__device__ __forceinline__ void unpack_v(const uint4& raw, float* out) {
  if constexpr (__is_same(T, bf16)) {
    const unsigned w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = __uint_as_float(w[j] << 16);
      out[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  } else {
    unpack16<T>(raw, out);
  }
}

template <typename T>
__device__ __forceinline__ uint4 load_nt(const T* p) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// VEC consecutive fp32 values: 16-byte loads when the caller's tables allow it (a
// block-uniform flag), else scalar loads of the same values.
template <int VEC>
__device__ __forceinline__ void load_f32_row(const float* ptr, float* out, bool vec) {
  if (vec) {
#pragma unroll
    for (int i = 0; i < VEC; i += 4) {
      const float4 a = *reinterpret_cast<const float4*>(ptr + i);
      out[i] = a.x; out[i + 1] = a.y; out[i + 2] = a.z; out[i + 3] = a.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = ptr[e];
  }
}

// Value of lane li ^ (LPR/2) of an aligned LPR-lane group (the NEOX RoPE partner). For
// 16-lane groups that is a rotation of each DPP row by 8; otherwise a cross-lane shuffle.
template <int LPR>
__device__ __forceinline__ float rope_partner(float x) {
  if constexpr (LPR == 16) {
    constexpr int kDppRowRor8 = 0x128;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowRor8, 0xF, 0xF, false));
  } else {
    return __shfl_xor(x, LPR / 2, kWave);
  }
}

// The q side of one work unit, in two steps so that its loads go out ahead of the K/V
// prefetch and their latency overlaps it: fetch() requests the raw 16-byte slice of every
// row (a row past the end re-reads the last row; its results are never written) and, when the tables
// are held (TABLES: up to two rows), the gain slice and each row's cos/sin slices;
// finish() applies the optional fused RMSNorm + RoPE and rounds once to T (the dtype the
// reference's q has when SDPA reads it), returning the raw 16 bytes (packed pairs for
// dot2). Without TABLES the table loads happen in finish().
template <typename T, int D, int ROWS>
struct QRows {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int LPR = D / VEC;
  static constexpr bool TABLES = ROWS <= 2;
  static constexpr int TW = TABLES ? VEC : 1;
  uint4 raw[ROWS];
  float w[TW];
  float c[TABLES ? ROWS : 1][TW], s[TABLES ? ROWS : 1][TW];

  __device__ __forceinline__ void fetch(const SplitParams& p, int b, int kvh, int rb, int li) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      int flat = rb * ROWS + r;
      flat = flat < p.rows_total ? flat : p.rows_total - 1;
      raw[r] = load16(static_cast<const T*>(p.q) + b * p.sqb + (kvh * p.G + flat % p.G) * p.sqh +
                      (flat / p.G) * p.sqt + li * VEC);
    }
    if constexpr (TABLES) {
      if ((p.flags & FORGE_NORM_QK) && p.qw) load_f32_row<VEC>(p.qw + li * VEC, w, p.vec_tables);
      if (p.flags & FORGE_ROPE) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
          int flat = rb * ROWS + r;
          flat = flat < p.rows_total ? flat : p.rows_total - 1;
          const int64_t off = b * p.csb + (flat / p.G) * p.cst + li * VEC;
          load_f32_row<VEC>(p.cos + off, c[r], p.vec_tables);
          load_f32_row<VEC>(p.sin + off, s[r], p.vec_tables);
        }
      }
    }
  }

  __device__ __forceinline__ uint4 finish(const SplitParams& p, int b, int rb, int r, int li) const {
    if (!(p.flags & (FORGE_NORM_QK | FORGE_ROPE))) return raw[r];
    float q[VEC];
    unpack16<T>(raw[r], q);
    const int flat = rb * ROWS + r < p.rows_total ? rb * ROWS + r : p.rows_total - 1;
    const int t = flat / p.G;
    if (p.flags & FORGE_NORM_QK) {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss += q[e] * q[e];
      ss = group_sum<LPR>(ss);
      const float rs = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
      for (int e = 0; e < VEC; ++e) q[e] *= rs;
      if (p.qw) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) q[e] *= TABLES ? w[e % TW] : p.qw[li * VEC + e];
      }
    }
    if (p.flags & FORGE_ROPE) {
      // NEOX pairing c <-> c + D/2: the partner slice is in lane li ^ (LPR/2).
      const float* cr = p.cos + b * p.csb + t * p.cst + li * VEC;
      const float* sr = p.sin + b * p.csb + t * p.cst + li * VEC;
      const bool first_half = li < LPR / 2;
      float y[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float partner = rope_partner<LPR>(q[e]);
        const float ce = TABLES ? c[r % (TABLES ? ROWS : 1)][e % TW] : cr[e];
        const float se = TABLES ? s[r % (TABLES ? ROWS : 1)][e % TW] : sr[e];
        y[e] = first_half ? q[e] * ce - partner * se : q[e] * ce + partner * se;
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) q[e] = y[e];
    }
    return pack16<T>(q);
  }
};

// One lane's 16-byte slice of a new key or value row (the group of LPR lanes holds the
// row), normalised (gain w, if any) and rotated like forge_kv_append's row kernel: the
// per-lane sum runs over the pairs (c, c + D/2) in the same order, the group sum over the
// same lane pattern, the fmas are the same explicit ones and nothing else is contracted,
// so the two produce the same bits. Every lane of the group must take part (cross-lane
// steps).
template <typename T, int D>
__device__ __forceinline__ uint4 new_row_slice(uint4 raw, bool norm, const float* w, float eps,
                                               const float* cr, const float* sr, int li) {
#pragma clang fp contract(off)
  constexpr int VEC = 16 / sizeof(T);
  constexpr int LPR = D / VEC;
  if (!norm && !cr) return raw;
  float x[VEC];
  unpack16<T>(raw, x);
  const bool first_half = li < LPR / 2;
  if (norm) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float o = rope_partner<LPR>(x[e]);
      const float a = first_half ? x[e] : o, z = first_half ? o : x[e];
      ss += fmaf(a, a, z * z);
    }
    ss = group_sum<LPR / 2>(ss);
    const float rs = rsqrtf(fmaf(ss, 1.0f / (float)D, eps));
#pragma unroll
    for (int e = 0; e < VEC; ++e) x[e] *= rs;
    if (w) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] *= w[li * VEC + e];
    }
  }
  if (cr) {
    float y[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float o = rope_partner<LPR>(x[e]);
      const float ce = cr[li * VEC + e], se = sr[li * VEC + e];
      y[e] = first_half ? fmaf(x[e], ce, -(o * se)) : fmaf(x[e], ce, o * se);
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) y[e] = fp32_result(y[e]);
    return pack16<T>(y);
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) x[e] = fp32_result(x[e]);
  return pack16<T>(x);
}

// Buffer resource of one (batch row, KV head) slab of the cache (gfx9 raw buffer: stride
// 0, range `bytes`). A load at a byte offset >= the range returns zeros without touching
// memory, which is how the split-K loop skips keys outside a unit's range while still
// issuing every load (kSkipOffset).
constexpr unsigned kBufferConfig = 0x00020000u;

// s_waitcnt immediate (gfx9 layout) that waits until at most the K and V loads of `ITERS`
// prefetched iterations (2 * NK each) are in flight; exp and lgkm counts left at maximum.
template <int ITERS, int NK> constexpr int kWaitPrefetch() {
  constexpr int n = 2 * NK * ITERS;
  static_assert(n < 64, "vmcnt is 6 bits");
  return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14);
}
constexpr unsigned kSkipOffset = 0x80000000u;  // beyond every slab (host check: < 2^31 bytes)
constexpr int kNonTemporal = 2;                // cache policy of the streaming loads (nt)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t slab_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kBufferConfig);
}

__device__ __forceinline__ uint4 load_slab(__amdgpu_buffer_rsrc_t rs, unsigned off) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, kNonTemporal));
  return make_uint4(v.x, v.y, v.z, v.w);
}

constexpr int kSplitWaves = kSplitThreads / kWave;

// LDS of the block-level merge, reused by every unit a block processes.
template <int D, int ROWS> struct SplitShared {
  float o[kSplitWaves][ROWS][D];
  float m[kSplitWaves][ROWS];
  float l[kSplitWaves][ROWS];
};

// One work unit: rows rb*ROWS .. of KV head kvh of batch row b (whose first new token
// sits at position `base`), keys of chunk c. The caller guarantees the block is converged
// (the unit may leave early, block-uniformly) and passes block-uniform arguments.
template <typename T, int D, int ROWS>
__device__ __forceinline__ void split_unit(const SplitParams& p, const int b, const int base,
                                           const int kvh, const int rb, const int c_in,
                                           SplitShared<D, ROWS>& sh, int* ticket = nullptr) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int LPR = D / VEC;  // lanes per key row
  static_assert(LPR >= 2 && LPR <= kWave && (LPR & (LPR - 1)) == 0, "bad head dim");
  constexpr int NG = kSplitThreads / LPR;  // key groups per block
  constexpr int NK = kSplitNK;
  constexpr int KPI = NG * NK;  // keys per block iteration
  constexpr int NWAVES = kSplitWaves;

  const int tid = threadIdx.x;
  const int li = tid % LPR;
  const int g = tid / LPR;
  const int wave = tid / kWave;

  // Rows of this block and their visible key ranges; the union [kmin_rb, kmax_rb] and
  // the intersection [lo_all, hi_all] over the valid rows.
  int kmin[ROWS], kmax[ROWS];
  int kmin_rb = INT_MAX, kmax_rb = -1, lo_all = -1, hi_all = INT_MAX;
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int flat = rb * ROWS + r;
    if (flat < p.rows_total) {
      visible_range32(base + flat / p.G, p.window, (int)p.max_len, kmin[r], kmax[r]);
      kmin_rb = kmin[r] < kmin_rb ? kmin[r] : kmin_rb;
      kmax_rb = kmax[r] > kmax_rb ? kmax[r] : kmax_rb;
      lo_all = kmin[r] > lo_all ? kmin[r] : lo_all;
      hi_all = kmax[r] < hi_all ? kmax[r] : hi_all;
    } else {
      kmin[r] = INT_MAX;
      kmax[r] = -1;
    }
  }
  const int c = p.span_chunks ? kmin_rb / p.chunk + c_in : c_in;  // absolute chunk
  const int c0 = c * p.chunk;
  if (c >= p.max_chunks || c0 > kmax_rb || c0 + p.chunk - 1 < kmin_rb) {  // block-uniform
    if (ticket && tid == 0) *ticket = atomicAdd(p.ws_ctr, 1);
    return;
  }
  const int iters = p.chunk / KPI;

  // New positions in this chunk (forge_attn_decode_append): [n_lo, n_hi], block-uniform.
  // The host takes this path only when one row block covers all of a KV head's query rows,
  // so this unit is the only one of the launch that reads these cache rows. It makes them
  // and writes them before its loads: lane group g handles the keys c0 + g (mod NG), both
  // here and in the stream below, so every lane later loads exactly the 16 bytes it stored
  // (a thread reads its own earlier write), and nothing extra stays live in the loop.
  if (p.kn) {
    int n_lo = base > c0 ? base : c0;
    int n_hi = base + p.T - 1 < c0 + p.chunk - 1 ? base + p.T - 1 : c0 + p.chunk - 1;
    if (n_hi > (int)p.max_len - 1) n_hi = (int)p.max_len - 1;
    if (n_lo <= n_hi) {  // block-uniform
      const int first = n_lo + (((g - (n_lo - c0)) % NG) + NG) % NG;  // this group's first
      const int64_t slab = b * p.skb + kvh * p.skh;
#pragma unroll
      for (int j = 0; j < kNewPerLane; ++j) {
        const int pp = first + j * NG;
        const int t = (pp <= n_hi ? pp : n_hi) - base;  // a row of the call, for every lane
        const T* kr = static_cast<const T*>(p.kn) + b * p.sknb + kvh * p.sknh + t * p.sknt + li * VEC;
        const T* vr = static_cast<const T*>(p.vn) + b * p.svnb + kvh * p.svnh + t * p.svnt + li * VEC;
        const bool rope = p.kvflags & FORGE_ROPE;
        const float* cr = rope ? p.cos + b * p.csb + t * p.cst : nullptr;
        const float* sr = rope ? p.sin + b * p.csb + t * p.cst : nullptr;
        const uint4 nk = new_row_slice<T, D>(load16(kr), p.kvflags & FORGE_NORM_QK, p.kw, p.eps, cr, sr, li);
        const uint4 nv = new_row_slice<T, D>(load16(vr), p.kvflags & FORGE_NORM_V, nullptr, p.eps,
                                             nullptr, nullptr, li);
        if (pp <= n_hi) {
          store16(static_cast<T*>(p.kcw) + slab + (int64_t)pp * p.sks + li * VEC, nk);
          store16(static_cast<T*>(p.vcw) + slab + (int64_t)pp * p.sks + li * VEC, nv);
        }
      }
      // the stores complete before the stream below loads the same rows
      __builtin_amdgcn_s_waitcnt(0);
      asm volatile("" ::: "memory");
    }
  }

  int it_first = kmin_rb > c0 ? (kmin_rb - c0) / KPI : 0;
  int it_last = (kmax_rb - c0) / KPI;
  if (it_last > iters - 1) it_last = iters - 1;

  // the persistent grid's next work ticket (the counter's old value; the caller adds the
  // grid size): nothing reads it before the unit's merge, so its round trip hides under
  // the unit
  if (ticket && tid == 0) *ticket = atomicAdd(p.ws_ctr, 1);

  QRows<T, D, ROWS> qr;
  qr.fetch(p, b, kvh, rb, li);

  // One (b, kv head) slab of the cache as a buffer; byte offsets inside it fit in 31 bits
  // (host check), so kSkipOffset lies beyond it.
  const int64_t slab = b * p.skb + kvh * p.skh;
  const unsigned row_bytes = (unsigned)p.sks * (unsigned)sizeof(T);
  const unsigned slab_bytes = (unsigned)(p.max_len - 1) * row_bytes + (unsigned)(D * sizeof(T));
  const __amdgpu_buffer_rsrc_t krs = slab_rsrc(static_cast<const T*>(p.kc) + slab, slab_bytes);
  const __amdgpu_buffer_rsrc_t vrs = slab_rsrc(static_cast<const T*>(p.vc) + slab, slab_bytes);
  const unsigned lane_bytes = (unsigned)(li * VEC * sizeof(T));

  // Loads of iteration `it`. Every load is issued, whatever the branch: keys outside
  // [kmin_rb, kmax_rb] and the iterations past it_last (the pipeline's tail, never
  // computed) read zeros through kSkipOffset, without memory traffic. With no load behind
  // a branch the compiler counts the loads in flight exactly, and an iteration waits only
  // for its own data, not for the prefetch issued just before it.
  auto load_iter = [&](int it, uint4* kr, uint4* vr) {
    const int kb0 = c0 + it * KPI;
    const bool live = it <= it_last;
#pragma unroll
    for (int u = 0; u < NK; ++u) {
      const int kp = kb0 + u * NG + g;
      const bool in = live && kp >= kmin_rb && kp <= kmax_rb;
      const unsigned off = in ? (unsigned)kp * row_bytes + lane_bytes : kSkipOffset;
      kr[u] = load_slab(krs, off);
      vr[u] = load_slab(vrs, off);
    }
  };

  constexpr int PF = split_pf<ROWS>();
  uint4 kbuf[PF][NK], vbuf[PF][NK];
#pragma unroll
  for (int j = 0; j < PF; ++j) load_iter(it_first + j, kbuf[j], vbuf[j]);

  // (A row past the end holds a copy of the last row; its results are never written.)
  uint4 q[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) q[r] = qr.finish(p, b, rb, r, li);
  // Everything but the prefetch has landed. Said explicitly so that the compiler's count
  // of loads in flight at the loop head does not include q/table loads that only some
  // (flag-dependent) paths consumed; otherwise it waits for every load there.
  __builtin_amdgcn_s_waitcnt(kWaitPrefetch<PF, NK>());

  float m[ROWS], l[ROWS], o[ROWS][VEC];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    m[r] = kNegInf;
    l[r] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[r][e] = 0.0f;
  }

  auto compute_iter = [&](int it, const uint4* kr, const uint4* vr) {
    const int kb0 = c0 + it * KPI;
    const bool full = kb0 >= lo_all && kb0 + KPI - 1 <= hi_all;  // every row sees every key
    float s[ROWS][NK];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
#pragma unroll
      for (int u = 0; u < NK; ++u) s[r][u] = group_sum<LPR>(dot16<T>(q[r], kr[u], 0.0f)) * p.scale_log2;
    }
    if (!full) {
#pragma unroll
      for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int u = 0; u < NK; ++u) {
          const int kp = kb0 + u * NG + g;
          if (kp < kmin[r] || kp > kmax[r]) s[r][u] = kNegInf;
        }
    }
    float vf[NK][VEC];
#pragma unroll
    for (int u = 0; u < NK; ++u) unpack_v<T>(vr[u], vf[u]);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float mx = s[r][0];
#pragma unroll
      for (int u = 1; u < NK; ++u) mx = fmaxf(mx, s[r][u]);
      if (mx > m[r] + kRescaleLog2) {  // (m = -inf: first visible key)
        const float alpha = m[r] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m[r] - mx);
        l[r] *= alpha;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[r][e] *= alpha;
        m[r] = mx;
      }
      float psum = 0.0f;
      float pu[NK];
#pragma unroll
      for (int u = 0; u < NK; ++u) {
        pu[u] = s[r][u] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(s[r][u] - m[r]);
        psum += pu[u];
      }
      l[r] += psum;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float acc = o[r][e];
#pragma unroll
        for (int u = 0; u < NK; ++u) acc = fmaf(pu[u], vf[u][e], acc);
        o[r][e] = acc;
      }
    }
  };

  // Rotating register pipeline: iteration it reads buffer (it - it_first) % PF, which is
  // refilled with iteration it + PF right after, so PF - 1 iterations are in flight while
  // one is computed. Whole rounds of PF iterations run without an exit in between (an exit
  // that rejoins the loop's latch would make the compiler wait for every load at the loop
  // head); the last < PF iterations, already requested, follow.
  const int n_it = it_last - it_first + 1;
  const int it_tail = it_first + n_it / PF * PF;
  for (int it = it_first; it < it_tail; it += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      compute_iter(it + j, kbuf[j], vbuf[j]);
      // From 3 rows on, the accumulators are pinned final here, so this iteration's V
      // registers are dead before their refill: left alone, the compiler sinks the V
      // accumulation below the refill, keeps the refilled V rows in other registers and
      // copies them back at the latch, which waits for all but the newest iteration's loads
      // once per round (C4 lengths, 16 q / 8 KV heads, T = 4: 986 against 1028 us per step;
      // at 1-2 rows the same pin measured within noise, so it is left out).
      if constexpr (ROWS > 2) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
          for (int e = 0; e < VEC; ++e) asm volatile("" : "+v"(o[r][e]));
      }
      // The refill stays below the compute, so the buffer keeps its registers across the
      // loop (no copies at the latch, which would wait for every load in flight).
      __builtin_amdgcn_sched_barrier(0);
      load_iter(it + j + PF, kbuf[j], vbuf[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < PF - 1; ++j)
    if (it_tail + j <= it_last) compute_iter(it_tail + j, kbuf[j], vbuf[j]);

  // Merge the groups of this wave: butterfly over lane distances LPR .. 32.
#pragma unroll
  for (int dist = LPR; dist < kWave; dist <<= 1) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const float m_o = __shfl_xor(m[r], dist, kWave);
      const float l_o = __shfl_xor(l[r], dist, kWave);
      const float m_n = fmaxf(m[r], m_o);
      const float a_s = rescale(m[r], m_n);
      const float a_o = rescale(m_o, m_n);
      l[r] = l[r] * a_s + l_o * a_o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float o_o = __shfl_xor(o[r][e], dist, kWave);
        o[r][e] = o[r][e] * a_s + o_o * a_o;
      }
      m[r] = m_n;
    }
  }
  if (tid % kWave < LPR) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) sh.o[wave][r][li * VEC + e] = o[r][e];
      if (li == 0) {
        sh.m[wave][r] = m[r];
        sh.l[wave][r] = l[r];
      }
    }
  }
  __syncthreads();

  // Merge the waves in order 0..3 and write the row's result for this chunk.
  for (int idx = tid; idx < ROWS * D; idx += kSplitThreads) {
    const int r = idx / D;
    const int e = idx % D;
    const int flat = rb * ROWS + r;
    if (flat >= p.rows_total) continue;
    const int t = flat / p.G;
    const int h = kvh * p.G + flat % p.G;
    int rkmin, rkmax;
    visible_range32(base + t, p.window, (int)p.max_len, rkmin, rkmax);
    if (c0 > rkmax || c0 + p.chunk - 1 < rkmin) continue;  // this chunk is outside the row
    float M = sh.m[0][r];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) M = fmaxf(M, sh.m[w][r]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
      const float a = rescale(sh.m[w][r], M);
      L = L + a * sh.l[w][r];
      O = O + a * sh.o[w][r][e];
    }
    const int cmin = rkmin / p.chunk;
    const int cmax = rkmax / p.chunk;
    if (cmin == cmax) {
      T* dst = static_cast<T*>(p.out) + b * p.sob + t * p.sot + h * p.soh;
      dst[e] = from_f32<T>(O / L);
    } else {
      const int64_t rowid = ((int64_t)b * p.H + h) * p.T + t;
      const int64_t slot = rowid * p.max_chunks + c;
      p.ws_o[slot * D + e] = O;
      if (e == 0) p.ws_ml[slot] = make_float2(M, L);
    }
  }
}

// Split-K kernel. Persistent mode (p.persist, used when positions come from device
// memory): a fixed grid of kPersistBlocksPerCU blocks per CU; every block derives the
// per-row chunk ranges from the device positions (so the launch needs no host knowledge
// of ragged lengths and stays graph-safe), builds the prefix sum of work units per batch row in LDS, and takes units
// by ticket from a counter in the workspace (zeroed by a one-thread kernel launched just
// before): blocks on CUs that stream faster take more units, so all blocks finish
// together. Units are ordered (row b, KV head x row block, chunk) with the chunk fastest,
// so the units in flight stream neighbouring chunks of a few (b, kv head) slabs, and no
// block is spent on chunks past a row's end.
// Grid mode (batches too large for the LDS prefix): one block per (chunk, head x row
// block, batch row), as before.
constexpr int kPersistMaxRows = 2048;
constexpr int kLastClasses = 16;  // size classes of the rows' last chunks (the hand-out order)

// Size class (0 .. kLastClasses - 1) of the last chunk of a row whose first new token sits at
// `base`: the chunk holding its last visible key, cut to the row's visible keys; 0 also for
// a row with no visible key.
__device__ __forceinline__ int last_chunk_class(const SplitParams& p, int base) {
  int lo, hi0, lo1, hi;
  visible_range32(base, p.window, (int)p.max_len, lo, hi0);
  visible_range32(base + p.T - 1, p.window, (int)p.max_len, lo1, hi);
  const int cmin = lo / p.chunk;
  int cmax = hi / p.chunk;
  if (cmax > p.max_chunks - 1) cmax = p.max_chunks - 1;
  if (hi < lo || cmax < cmin) return 0;
  const int c_lo = cmax * p.chunk > lo ? cmax * p.chunk : lo;
  const int c_hi = (cmax + 1) * p.chunk - 1 < hi ? (cmax + 1) * p.chunk - 1 : hi;
  return (int)(((int64_t)(c_hi - c_lo + 1) * kLastClasses - 1) / p.chunk);
}

// The persistent grids hand out the rows' last chunks at the end, largest first: the blocks
// that run out of work first take the longest of them, which shortens the launch's tail
// (a ragged batch's last chunks are a random part of a chunk each). A counting sort of the
// B rows by class (counts[] holds each class's rows, cls[] each row's class): sh_last[i] is
// the row of the i-th last chunk. Stable (row order within a class), since every block of a
// launch must derive the same unit -> row map. Called by the whole block.
__device__ __forceinline__ void order_last_chunks(int B, int* counts, const unsigned char* cls, int* sh_last) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    int run = 0;
    for (int k = kLastClasses - 1; k >= 0; --k) {
      const int c = counts[k];
      counts[k] = run;
      run += c;
    }
  }
  __syncthreads();
  if (tid < kWave) {  // wave 0, 64 rows at a time; lane k keeps the running count of class k
    int run = 0;
    for (int b0 = 0; b0 < B; b0 += kWave) {
      const int b = b0 + tid;
      const int c = b < B ? (int)cls[b] : -1;
      unsigned long long left = __ballot(c >= 0);
      int slot = 0;
      while (left) {  // one pass per class present among these rows
        const int c0 = __builtin_amdgcn_readlane(c, __builtin_ctzll(left));
        const unsigned long long same = __ballot(c == c0);
        const int placed = __builtin_amdgcn_readlane(run, c0);
        if (c == c0) slot = counts[c0] + placed + __popcll(same & ((1ull << tid) - 1));
        if (tid == c0) run += __popcll(same);
        left &= ~same;
      }
      if (b < B) sh_last[slot] = b;
    }
  }
  __syncthreads();
}

// Occupancy target: more waves hide more HBM latency, fewer leave registers for the
// accumulators of ROWS query rows and the pipeline's buffers (the persistent grid holds two
// blocks per CU, two waves per SIMD, whatever the target).
template <int ROWS> constexpr int split_waves_per_eu() { return ROWS <= 2 ? 3 : 2; }

template <typename T, int D, int ROWS>
__global__ __launch_bounds__(kSplitThreads) __attribute__((amdgpu_waves_per_eu(split_waves_per_eu<ROWS>())))
void splitk_kernel(SplitParams p) {
  __shared__ SplitShared<D, ROWS> sh;
  if (!p.persist) {
    // Positions fit in 32 bits (host check: max_len < 2^30).
    const int base = (int)row_base(p.row_pos, p.pos_dev, p.pos0, blockIdx.z);
    // chunks in reverse: a row's last chunk, whose unit also makes the step's new keys
    // (forge_attn_decode_append) and so starts its stream later, is dispatched first
    split_unit<T, D, ROWS>(p, blockIdx.z, base, blockIdx.y % p.K, blockIdx.y / p.K,
                           (int)gridDim.x - 1 - (int)blockIdx.x, sh);
    return;
  }
  __shared__ int sh_pref[kPersistMaxRows + 1];
  __shared__ int sh_base[kPersistMaxRows];  // first new token's position of each row
  __shared__ int sh_nch[kPersistMaxRows];
  __shared__ int sh_last[kPersistMaxRows];     // rows by the size of their last chunk, largest first
  __shared__ unsigned char sh_cls[kPersistMaxRows];
  __shared__ int sh_count[kLastClasses];
  const int tid = threadIdx.x;
  const int n_rb = (p.rows_total + ROWS - 1) / ROWS;
  const int per_row = p.K * n_rb;  // (kv head, row block) pairs per chunk
  if (tid < kLastClasses) sh_count[tid] = 0;
  __syncthreads();
  // chunk range of each batch row: union of its T queries' visible keys
  for (int b = tid; b < p.B; b += kSplitThreads) {
    const int base = (int)row_base(p.row_pos, p.pos_dev, p.pos0, b);
    sh_base[b] = base;
    int lo, hi0, lo1, hi;
    visible_range32(base, p.window, (int)p.max_len, lo, hi0);
    visible_range32(base + p.T - 1, p.window, (int)p.max_len, lo1, hi);
    const int cmin = lo / p.chunk;
    int cmax = hi / p.chunk;
    if (cmax > p.max_chunks - 1) cmax = p.max_chunks - 1;
    sh_nch[b] = (hi >= lo && cmax >= cmin) ? cmax - cmin + 1 : 0;
    const int cls = last_chunk_class(p, base);
    sh_cls[b] = (unsigned char)cls;
    atomicAdd(&sh_count[cls], 1);
  }
  __syncthreads();
  order_last_chunks(p.B, sh_count, sh_cls, sh_last);
  // exclusive prefix sum of units per row (wave 0: lane l scans a contiguous segment)
  if (tid < kWave) {
    const int seg = (p.B + kWave - 1) / kWave;
    const int r0 = tid * seg;
    const int r1 = r0 + seg < p.B ? r0 + seg : p.B;
    int sum = 0;
    for (int r = r0; r < r1; ++r) sum += (sh_nch[r] > 0 ? sh_nch[r] - 1 : 0) * per_row;
    int incl = sum;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (tid >= d) incl += v;
    }
    int run = incl - sum;
    for (int r = r0; r < r1; ++r) {
      sh_pref[r] = run;
      run += (sh_nch[r] > 0 ? sh_nch[r] - 1 : 0) * per_row;
    }
    if (tid == kWave - 1) sh_pref[p.B] = incl;
  }
  __syncthreads();
  // Units [0, body) are every row's chunks but its last, (row, KV head x row block, chunk)
  // with the chunk fastest, each row's from its second-to-last chunk down; units
  // [body, total) are the rows' last chunks, (row in sh_last's order, KV head x row block).
  // A ragged batch's last chunks are partial (a random part of a chunk each), so handing
  // them out last, largest first, shortens the units left when blocks run out of work.
  const int body = sh_pref[p.B];
  const int total = body + p.B * per_row;
  // Block i starts with unit i; after that units go by ticket (grid + an atomic counter
  // in the workspace, which the host zeroes before the launch), so a block on a CU that
  // streams faster takes more of them. A block fetches its next ticket when it starts a
  // unit and reads it after the unit's merge.
  // Two ticket slots, alternating by iteration: a unit may return early without a block
  // barrier, so thread 0 can write the next ticket while a slower wave has not yet read
  // the one before; with the slots alternating it writes the other slot, and the barrier
  // at the end of every iteration keeps the waves within one iteration of each other.
  __shared__ int sh_ticket[2];
  int parity = 0;
  // (LDS values are block-uniform; readfirstlane lets the compiler keep the unit's
  // coordinates, and the cache slab's buffer descriptors built from them, in scalar
  // registers.)
  for (int u = blockIdx.x; u < total; u = __builtin_amdgcn_readfirstlane(sh_ticket[parity]), parity ^= 1) {
    int next = 0;  // split_unit sets it on every path
    int lo, pr, cidx;  // row, (KV head, row block), chunk counted from the row's first
    if (u < body) {
      lo = 0;
      int hi = p.B - 1;  // last row with sh_pref[row] <= u
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (__builtin_amdgcn_readfirstlane(sh_pref[mid]) <= u) lo = mid;
        else hi = mid - 1;
      }
      const int o = u - __builtin_amdgcn_readfirstlane(sh_pref[lo]);
      const int n = __builtin_amdgcn_readfirstlane(sh_nch[lo]) - 1;  // >= 1 here
      pr = o / n;
      cidx = n - 1 - o % n;
    } else {
      // a row with no visible key has no last chunk either: cidx -1 lies before every key,
      // and the unit returns at once
      const int q = u - body;
      lo = __builtin_amdgcn_readfirstlane(sh_last[q / per_row]);
      pr = q % per_row;
      cidx = __builtin_amdgcn_readfirstlane(sh_nch[lo]) - 1;
    }
    const int base = __builtin_amdgcn_readfirstlane(sh_base[lo]);
    int kmin, kmax;
    visible_range32(base, p.window, (int)p.max_len, kmin, kmax);  // the row's first chunk
    split_unit<T, D, ROWS>(p, lo, base, pr % p.K, pr / p.K, kmin / p.chunk + cidx, sh, &next);
    if (tid == 0) sh_ticket[parity] = (int)gridDim.x + next;
    __syncthreads();  // the next unit reuses the merge LDS; the ticket is visible
  }
}

// Zeroes the work ticket of the next persistent launch on this stream (a kernel rather
// than a memset, so that the call can be captured into a graph).
__global__ void ticket_reset_kernel(int* ctr) {
  if (threadIdx.x == 0) ctr[0] = 0;
}

// One block (4 waves) per (b, h, t) row: wave w merges chunks w, w+4, ... of the row
// (8 at a time, loads issued together), then the 4 wave results are merged in order.
template <typename T, int D>
__global__ __launch_bounds__(256) void combine_kernel(SplitParams p) {
  constexpr int EPL = D >= kWave ? D / kWave : 1;  // elements per lane
  constexpr int NWAVES = 4;
  constexpr int UNROLL = 8;
  __shared__ float sh_o[NWAVES][D];
  __shared__ float sh_m[NWAVES], sh_l[NWAVES];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  // the split kernel has finished with the work ticket: leave it zero for the next call on
  // this workspace (FORGE_WS_ZEROED)
  if (blockIdx.x == 0 && threadIdx.x == 0 && p.ws_ctr) *p.ws_ctr = 0;
  const int64_t row = blockIdx.x;  // == (b*H + h)*T + t
  const int t = (int)(row % p.T);
  const int b = (int)(row / ((int64_t)p.T * p.H));
  const int64_t base = row_base(p.row_pos, p.pos_dev, p.pos0, b);
  int64_t kmin, kmax;
  visible_range(base + t, p.window, p.max_len, kmin, kmax);
  if (kmax < kmin) return;
  const int64_t cmin = kmin / p.chunk;
  int64_t cmax = kmax / p.chunk;
  if (cmax > p.max_chunks - 1) cmax = p.max_chunks - 1;
  if (cmin >= cmax) return;  // single chunk: the split kernel wrote the output
  const int64_t slot0 = row * p.max_chunks;

  float M = kNegInf;
  for (int64_t c = cmin + threadIdx.x; c <= cmax; c += 256) M = fmaxf(M, p.ws_ml[slot0 + c].x);
  M = group_max<kWave>(M);
  if (lane == 0) sh_m[wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(sh_m[0], sh_m[1]), fmaxf(sh_m[2], sh_m[3]));
  __syncthreads();

  const bool active = lane * EPL < D;
  float L = 0.0f, O[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) O[i] = 0.0f;
  for (int64_t c = cmin + wave; c <= cmax; c += NWAVES * UNROLL) {
    float2 ml[UNROLL];
    float ov[UNROLL][EPL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t cc = c + (int64_t)u * NWAVES;
      if (cc <= cmax) {
        ml[u] = p.ws_ml[slot0 + cc];
        const float* src = p.ws_o + (slot0 + cc) * D + lane * EPL;
#pragma unroll
        for (int i = 0; i < EPL; ++i) ov[u][i] = active ? src[i] : 0.0f;
      } else {
        ml[u] = make_float2(kNegInf, 0.0f);
#pragma unroll
        for (int i = 0; i < EPL; ++i) ov[u][i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const float a = rescale(ml[u].x, M);
      L = L + a * ml[u].y;
#pragma unroll
      for (int i = 0; i < EPL; ++i) O[i] = O[i] + a * ov[u][i];
    }
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) sh_o[wave][lane * EPL + i] = O[i];
  }
  if (lane == 0) sh_l[wave] = L;
  __syncthreads();
  if (wave != 0 || !active) return;
  const float Lt = ((sh_l[0] + sh_l[1]) + sh_l[2]) + sh_l[3];
  const int h = (int)((row / p.T) % p.H);
  T* dst = static_cast<T*>(p.out) + b * p.sob + t * p.sot + h * p.soh + lane * EPL;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane * EPL + i;
    const float Ot = ((sh_o[0][e] + sh_o[1][e]) + sh_o[2][e]) + sh_o[3][e];
    dst[i] = from_f32<T>(Ot / Lt);
  }
}

// ---------------------------------------------------------------------------------------
// Verify / decode for wide head groups (G = H/K >= 4, bf16/fp16, head dim 128 or 256) on
// MFMA. There the G*T query rows of one KV head make a small GEMM rather than a GEMV, and
// the VALU split-K kernel above spends its time on per-score lane reductions. One block
// (4 waves) takes one unit of the same split as above: (batch row, KV head, block of up
// to 32 rows, chunk of keys at absolute positions), writing the same outputs/partials for
// the same combine kernel. The path is chosen by (dtype, head dim, G) only, never by T, so
// a verify row and the decode of that token run the same code.
//
//   * K and V tiles of 32 keys go from HBM into LDS with direct loads (two stages), the
//     same swizzled layouts as the prefill kernel. Every wave computes the whole score tile
//     S^T = K . Q^T (32 keys x 32 rows on v_mfma_f32_32x32x16) with Q^T in registers, and
//     owns D/4 output channels of O^T = V^T . P^T, so the waves never merge: the running
//     (m, l) they keep are identical.
//   * Lane l owns row l % 32 (a query head and token); the row's visible key range comes
//     from its position as in the split kernel, so masks, windows and ragged rows match.
template <int D> struct VerifyTile {
  static constexpr int WAVES = 4;
  static constexpr int ROWS = 32;
  static constexpr int BN = 32;                 // keys per tile
  static constexpr int NCH = D / 8;
  static constexpr int ROWB = 2 * D;
  static constexpr int TILEB = BN * ROWB;
  static constexpr int LOADS = TILEB / (WAVES * 1024);
  // LDS stages of K and V: three tiles in flight; at head dim 512 (32 KB tiles) two stages
  // (one tile in flight), the most that fits beside the tables
  static constexpr int STAGES = D >= 512 ? 2 : 4;
  static constexpr int MIN_G = D >= 512 ? 8 : 4;          // query heads per KV head the path takes
  static constexpr int MAX_TOK = ROWS / MIN_G + 1;        // tokens under one unit's rows
  // q gains, cos rows and sin rows (fp32), each region padded to whole KB (the DMA unit)
  static constexpr int TAB_G = (4 * D + 1023) / 1024 * 1024;
  static constexpr int TAB_R = (MAX_TOK * 4 * D + 1023) / 1024 * 1024;
  static constexpr int TAB_BYTES = TAB_G + 2 * TAB_R;
  static constexpr int LDS_BYTES = STAGES * 2 * TILEB + TAB_BYTES;
  static constexpr int DW = D / WAVES;          // output channels per wave
  static_assert(LOADS * WAVES * 1024 == TILEB, "tile must split into whole wave loads");
  static_assert(DW % 32 == 0, "a wave owns whole 32-channel MFMA blocks");
};

typedef __bf16 v_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 v_f16x8 __attribute__((ext_vector_type(8)));
typedef float v_floatx16 __attribute__((ext_vector_type(16)));
typedef short v_i16x4 __attribute__((ext_vector_type(4)));

template <typename T> struct VMfma;
template <> struct VMfma<bf16> {
  typedef v_bf16x8 vec;
  static __device__ __forceinline__ v_floatx16 run(vec a, vec b, v_floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct VMfma<f16> {
  typedef v_f16x8 vec;
  static __device__ __forceinline__ v_floatx16 run(vec a, vec b, v_floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// XOR swizzles of the 16-byte chunk index by key row (conflict-free operand reads; the
// same as the prefill kernel's for head dim >= 128).
__device__ __forceinline__ int vswz_k(int row) { return row & 15; }
__device__ __forceinline__ int vswz_v(int row) { return (row & 3) << 2; }

// Wait until at most N vector-memory loads of this wave are outstanding (they retire in
// issue order, so everything issued before the last N has landed).
template <int N> __device__ __forceinline__ void vwait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 0..63");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One unit of the MFMA verify path: rows rb*32 .. of KV head kvh of batch row b (whose first
// new token sits at position `base`), keys of chunk c_in (absolute; with p.span_chunks,
// counted from the unit's first visible chunk). The caller passes block-uniform arguments
// and a converged block; the unit may leave early, block-uniformly, and uses all of the
// dynamic LDS `smem`. This form fills the LDS stages with direct loads; it serves head dim
// 512 on the persistent grid (per-row positions), and verify_unit_staged below every other
// case.
template <typename T, int D>
__device__ __forceinline__ void verify_unit_dma(const SplitParams& p, char* smem, const int b,
                                                const int base, const int kvh, const int rb,
                                                const int c_in) {
  using V8 = typename VMfma<T>::vec;
  using TL = VerifyTile<D>;
  constexpr int BN = TL::BN;
  constexpr int KSTEPS = D / 16;
  constexpr int DBW = TL::DW / 32;  // 32-channel blocks per wave

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int n = lane & 31;
  const int hi = lane >> 5;

  // this lane's row and its visible keys; the unit's key span (union over valid rows)
  const int flat = rb * TL::ROWS + n;
  const bool valid = flat < p.rows_total;
  const int t = valid ? flat / p.G : 0;
  const int h = kvh * p.G + (valid ? flat % p.G : 0);
  int kmin = INT_MAX, kmax = -1;
  if (valid) visible_range32(base + t, p.window, (int)p.max_len, kmin, kmax);
  // union over the unit's rows: both ends of a visible range grow with the position, so it
  // runs from the first row's start to the last row's end (tokens rb*32/G .. of the unit)
  int umin, umax, dummy;
  {
    const int r_hi = rb * TL::ROWS + TL::ROWS - 1 < p.rows_total - 1 ? rb * TL::ROWS + TL::ROWS - 1 : p.rows_total - 1;
    visible_range32(base + rb * TL::ROWS / p.G, p.window, (int)p.max_len, umin, dummy);
    visible_range32(base + r_hi / p.G, p.window, (int)p.max_len, dummy, umax);
  }
  // keys every valid row of the unit sees: the last token's first key to the first token's last
  int kmin_all, kmax_all;
  {
    const int r_hi = rb * TL::ROWS + TL::ROWS - 1 < p.rows_total - 1 ? rb * TL::ROWS + TL::ROWS - 1 : p.rows_total - 1;
    visible_range32(base + r_hi / p.G, p.window, (int)p.max_len, kmin_all, dummy);
    visible_range32(base + rb * TL::ROWS / p.G, p.window, (int)p.max_len, dummy, kmax_all);
  }
  const int c = p.span_chunks ? umin / p.chunk + c_in : c_in;  // absolute chunk
  const int c0 = c * p.chunk;
  if (c >= p.max_chunks || c0 > umax || c0 + p.chunk - 1 < umin) return;  // block-uniform

  // New positions in this chunk (forge_attn_decode_append; the host takes this path when the
  // unit's row block holds all of the KV head's query rows, so this block is the only reader
  // of these cache rows): make them (a group of D / 8 lanes per row), write them, and wait
  // for every wave's writes before any tile load.
  if (p.kn) {
    int n_lo = base > c0 ? base : c0;
    int n_hi = base + p.T - 1 < c0 + p.chunk - 1 ? base + p.T - 1 : c0 + p.chunk - 1;
    if (n_hi > (int)p.max_len - 1) n_hi = (int)p.max_len - 1;
    if (n_lo <= n_hi) {  // block-uniform
      constexpr int VEC = 16 / sizeof(T);
      constexpr int LPR = D / VEC;
      constexpr int RPP = 256 / LPR;  // rows per pass of the block
      const int li = tid % LPR, rr = tid / LPR;
      const int64_t slab = b * p.skb + kvh * p.skh;
      for (int p0 = n_lo; p0 <= n_hi; p0 += RPP) {
        const int pp = p0 + rr;
        const int tt = (pp <= n_hi ? pp : n_hi) - base;  // a row of the call, for every lane
        const T* kr = static_cast<const T*>(p.kn) + b * p.sknb + kvh * p.sknh + tt * p.sknt + li * VEC;
        const T* vr = static_cast<const T*>(p.vn) + b * p.svnb + kvh * p.svnh + tt * p.svnt + li * VEC;
        const bool krope = p.kvflags & FORGE_ROPE;
        const float* cr = krope ? p.cos + b * p.csb + tt * p.cst : nullptr;
        const float* sr = krope ? p.sin + b * p.csb + tt * p.cst : nullptr;
        const uint4 nk = new_row_slice<T, D>(load16(kr), p.kvflags & FORGE_NORM_QK, p.kw, p.eps, cr, sr, li);
        const uint4 nv = new_row_slice<T, D>(load16(vr), p.kvflags & FORGE_NORM_V, nullptr, p.eps,
                                             nullptr, nullptr, li);
        if (pp <= n_hi) {
          store16(static_cast<T*>(p.kcw) + slab + (int64_t)pp * p.sks + li * VEC, nk);
          store16(static_cast<T*>(p.vcw) + slab + (int64_t)pp * p.sks + li * VEC, nv);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  int t_first = umin > c0 ? (umin - c0) / BN : 0;
  int t_last = (umax - c0) / BN;
  if (t_last > p.chunk / BN - 1) t_last = p.chunk / BN - 1;
  const int ntiles = t_last - t_first + 1;

  // direct loads of tile i (key0 = c0 + (t_first + i)*BN) into stage i % STAGES; rows past
  // the unit's last key read row umax (masked)
  const char* kgb = reinterpret_cast<const char*>(static_cast<const T*>(p.kc) + b * p.skb + kvh * p.skh);
  const char* vgb = reinterpret_cast<const char*>(static_cast<const T*>(p.vc) + b * p.skb + kvh * p.skh);
  const int rstride = (int)p.sks * 2;
  auto issue = [&](int i) {
    if (i >= ntiles) return;
    const int key0 = c0 + (t_first + i) * BN;
    const int rows_left = umax - key0 + 1;
    const unsigned kdst = lds_offset(smem + (2 * (i % TL::STAGES)) * TL::TILEB + wave * TL::LOADS * 1024);
    const unsigned vdst = kdst + TL::TILEB;
    const char* kt = kgb + (int64_t)key0 * rstride;
    const char* vt = vgb + (int64_t)key0 * rstride;
#pragma unroll
    for (int j = 0; j < TL::LOADS; ++j) {
      const int slot = (wave * TL::LOADS + j) * 64 + lane;
      const int row = slot / TL::NCH, pch = slot % TL::NCH;
      const int rr = row < rows_left ? row : rows_left - 1;
      lds_dma16(kt, (unsigned)(rr * rstride + ((pch ^ vswz_k(row)) << 4)), kdst + j * 1024);
      lds_dma16(vt, (unsigned)(rr * rstride + ((pch ^ vswz_v(row)) << 4)), vdst + j * 1024);
    }
  };

  // ---- prologue: the unit's q rows, q gains and RoPE rows, and the first STAGES - 1 tiles.
  // Loads retire in issue order, so the small loads go out FIRST: waiting for them (a
  // vmcnt of the tile loads issued after them) leaves the tiles streaming while q is
  // normalised and rotated. With small_dma (aligned tables, offsets within 32 bits) they
  // are DMA'd straight into LDS: raw q rows into the V slot of the last stage, tables into
  // `tab`; otherwise they go through registers and wait for the tiles too.
  const bool gains = (p.flags & FORGE_NORM_QK) && p.qw;
  const bool rope = (p.flags & FORGE_ROPE) != 0;
  const int tok_lo = rb * TL::ROWS / p.G;
  const int tok_hi = (rb * TL::ROWS + TL::ROWS - 1 < p.rows_total - 1 ? rb * TL::ROWS + TL::ROWS - 1 : p.rows_total - 1) / p.G;
  const int ntok = tok_hi - tok_lo + 1;  // <= MAX_TOK for G >= 4
  char* tab_b = smem + TL::STAGES * 2 * TL::TILEB;  // [gains | cos rows | sin rows], regions padded
  float* tab = reinterpret_cast<float*>(tab_b);
  const float* tab_cos = reinterpret_cast<const float*>(tab_b + TL::TAB_G);
  const float* tab_sin = reinterpret_cast<const float*>(tab_b + TL::TAB_G + TL::TAB_R);
  T* qs = reinterpret_cast<T*>(smem + (2 * (TL::STAGES - 1)) * TL::TILEB);        // normalised [ROWS][D]
  T* qraw = reinterpret_cast<T*>(smem + (2 * (TL::STAGES - 1) + 1) * TL::TILEB);  // raw [ROWS][D]
  static_assert(TL::ROWS * D * 2 == TL::TILEB, "the raw q rows fill one tile slot");
  // The q math is split over the waves: this lane normalises and rotates row
  // qr = 8 * wave + lane / 8 of the unit, first-half channels qx .. qx + QCH - 1 and their
  // RoPE partners qx + D/2. Rows past the end read row 0 of head kvh * G and are zeroed.
  constexpr int QCH = D / 16;  // first-half channels per lane, 8 lanes per row
  const int qr = 8 * wave + (lane >> 3);
  const int qx = QCH * (lane & 7);
  const int qflat = rb * TL::ROWS + qr;
  const bool qvalid = qflat < p.rows_total;
  const int qtok = qvalid ? qflat / p.G : 0;
  uint4 qa[QCH / 8], qz[QCH / 8];
  if (p.small_dma) {
    // raw q rows: instruction j of this wave fills bytes [(wave * QI + j) KB, +1 KB) of qraw
    constexpr int QI = TL::TILEB / 1024 / TL::WAVES;
    const char* qb = static_cast<const char*>(p.q) + (int64_t)b * p.sqb * (int64_t)sizeof(T);
#pragma unroll
    for (int j = 0; j < QI; ++j) {
      const int inst = wave * QI + j;
      const int off = inst * 1024 + 16 * lane;
      const int r = off / (2 * D), cb = off % (2 * D);
      const int fl = rb * TL::ROWS + r;
      const bool ok = fl < p.rows_total;
      const int64_t src = ((int64_t)(kvh * p.G + (ok ? fl % p.G : 0)) * p.sqh +
                           (int64_t)(ok ? fl / p.G : 0) * p.sqt) * (int64_t)sizeof(T) + cb;
      lds_dma16(qb, (unsigned)src, lds_offset(qraw) + inst * 1024);
    }
    // table rows, 1 KB per instruction, instruction i of the block on wave i % WAVES; lanes
    // past a region's last row re-read its last 16 bytes into the region's padding
    int inst0 = 0;
    auto dma_rows = [&](const float* src, int64_t stride, int rows, unsigned dst) {
      const int bytes = rows * 4 * D;
      const int ninst = (bytes + 1023) / 1024;
      for (int i = 0; i < ninst; ++i) {
        if ((inst0 + i) % TL::WAVES != wave) continue;
        int off = i * 1024 + 16 * lane;
        if (off > bytes - 16) off = bytes - 16;
        const int r = off / (4 * D), cb = off % (4 * D);
        lds_dma16(src, (unsigned)(r * stride * 4 + cb), dst + i * 1024);
      }
      inst0 += ninst;
    };
    if (gains) dma_rows(p.qw, 0, 1, lds_offset(tab_b));
    if (rope) {
      const int64_t row0 = b * p.csb + (int64_t)tok_lo * p.cst;
      dma_rows(p.cos + row0, p.cst, ntok, lds_offset(tab_b + TL::TAB_G));
      dma_rows(p.sin + row0, p.cst, ntok, lds_offset(tab_b + TL::TAB_G + TL::TAB_R));
    }
#pragma unroll
    for (int i = 0; i < TL::STAGES - 1; ++i) issue(i);
    // this wave's small loads have landed once at most its tile loads remain
    const int pro_tiles = ntiles < TL::STAGES - 1 ? ntiles : TL::STAGES - 1;
    static_assert(TL::STAGES - 1 == 3 || TL::STAGES - 1 == 1, "one wait per prologue tile count");
    if (TL::STAGES - 1 == 3 && pro_tiles >= 3) vwait_vm<(TL::STAGES - 1 == 3 ? 6 : 2) * TL::LOADS>();
    else if (TL::STAGES - 1 == 3 && pro_tiles == 2) vwait_vm<(TL::STAGES - 1 == 3 ? 4 : 2) * TL::LOADS>();
    else vwait_vm<2 * TL::LOADS>();
    __syncthreads();  // every wave's q rows and tables are in LDS (tiles may be in flight)
    const T* qrow = qraw + qr * D + qx;
#pragma unroll
    for (int j = 0; j < QCH / 8; ++j) {
      qa[j] = *reinterpret_cast<const uint4*>(qrow + 8 * j);
      qz[j] = *reinterpret_cast<const uint4*>(qrow + D / 2 + 8 * j);
    }
  } else {
#pragma unroll
    for (int i = 0; i < TL::STAGES - 1; ++i) issue(i);
    {
      const int qh = kvh * p.G + (qvalid ? qflat % p.G : 0);
      const T* src = static_cast<const T*>(p.q) + b * p.sqb + qh * p.sqh + qtok * p.sqt + qx;
#pragma unroll
      for (int j = 0; j < QCH / 8; ++j) {
        qa[j] = load16(src + 8 * j);
        qz[j] = load16(src + D / 2 + 8 * j);
      }
    }
    // every table value's load goes out before the first store (one round trip)
    constexpr int NV = ((1 + 2 * TL::MAX_TOK) * D + TL::WAVES * kWave - 1) / (TL::WAVES * kWave);
    const int nrow = (gains ? 1 : 0) + (rope ? 2 * ntok : 0);
    float v[NV];
    int dsti[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int idx = tid + j * TL::WAVES * kWave;
      dsti[j] = -1;
      v[j] = 0.0f;
      if (idx < nrow * D) {
        const int r = idx / D, x = idx % D;
        const int rr = gains ? r : r + 1;  // table row: 0 gains, 1..ntok cos, ntok+1.. sin
        if (rr == 0) {
          v[j] = p.qw[x];
          dsti[j] = x;
        } else {
          const int k = (rr - 1) % ntok;
          v[j] = (rr <= ntok ? p.cos : p.sin)[b * p.csb + (int64_t)(tok_lo + k) * p.cst + x];
          dsti[j] = (rr <= ntok ? TL::TAB_G : TL::TAB_G + TL::TAB_R) / 4 + k * D + x;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (dsti[j] >= 0) tab[dsti[j]] = v[j];
    __syncthreads();  // tables in LDS (the tile loads may still be in flight)
  }

  // Fused RMSNorm + RoPE of this lane's q values in fp32, one rounding (as the split
  // kernel's q prologue), staged as T in the K slot of the last stage (not loaded until the
  // loop's first barrier); then every wave reads the Q^T operands of its lane's row n:
  // channels 16s + 8hi + e.
  {
    float a[QCH], z[QCH];
#pragma unroll
    for (int j = 0; j < QCH / 8; ++j) {
      unpack16<T>(qa[j], a + 8 * j);
      unpack16<T>(qz[j], z + 8 * j);
    }
    if (!qvalid) {
#pragma unroll
      for (int e = 0; e < QCH; ++e) a[e] = z[e] = 0.0f;
    }
    float rs = 1.0f;  // RMSNorm factor (1 without FORGE_NORM_QK)
    if (p.flags & FORGE_NORM_QK) {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < QCH; ++e) ss += a[e] * a[e] + z[e] * z[e];
      ss += __shfl_xor(ss, 1, kWave);
      ss += __shfl_xor(ss, 2, kWave);
      ss += __shfl_xor(ss, 4, kWave);
      rs = rsqrtf(ss / (float)D + p.eps);
    }
#pragma unroll
    for (int j = 0; j < QCH / 8; ++j) {
      const int x = qx + 8 * j;
      float* aj = a + 8 * j;
      float* zj = z + 8 * j;
      if (gains) {
        float wa[8], wz[8];
        load_f32x8(tab + x, wa);
        load_f32x8(tab + x + D / 2, wz);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          aj[e] = aj[e] * rs * wa[e];
          zj[e] = zj[e] * rs * wz[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          aj[e] *= rs;
          zj[e] *= rs;
        }
      }
      if (rope && qvalid) {
        const float* cr = tab_cos + (qtok - tok_lo) * D;
        const float* sr = tab_sin + (qtok - tok_lo) * D;
        float c1[8], s1[8], c2[8], s2[8];
        load_f32x8(cr + x, c1);
        load_f32x8(sr + x, s1);
        load_f32x8(cr + x + D / 2, c2);
        load_f32x8(sr + x + D / 2, s2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float a0 = aj[e], z0 = zj[e];
          aj[e] = a0 * c1[e] - z0 * s1[e];
          zj[e] = z0 * c2[e] + a0 * s2[e];
        }
      }
      *reinterpret_cast<uint4*>(qs + qr * D + x) = pack16<T>(aj);
      *reinterpret_cast<uint4*>(qs + qr * D + D / 2 + x) = pack16<T>(zj);
    }
  }
  __syncthreads();  // the block's q rows are in LDS
  V8 qreg[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) qreg[s] = *reinterpret_cast<const V8*>(qs + n * D + 16 * s + 8 * hi);

  // LDS read offsets within a tile (as the prefill kernel's)
  const int k_rd = n * TL::ROWB;
  const int k_sw = vswz_k(n);
  const int g = lane >> 4, kq = (lane >> 2) & 3, qq = lane & 3;
  const int v_row = 4 * (g >> 1) + kq;
  const int v_sw = vswz_v(v_row);
  const int v_chlo = 2 * (g & 1) + (qq >> 1);
  const int v_byte = 8 * (qq & 1);

  v_floatx16 oacc[DBW];
#pragma unroll
  for (int d = 0; d < DBW; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.0f;
  float m_run = kNegInf, l_run = 0.0f;
  const float cl2 = p.scale_log2;

  for (int i = 0; i < ntiles; ++i) {
    // tile i has landed once at most the loads of the tiles issued after it remain
    const int after = ntiles - 1 - i < TL::STAGES - 2 ? ntiles - 1 - i : TL::STAGES - 2;
    if (after >= 2) vwait_vm<4 * TL::LOADS>();
    else if (after == 1) vwait_vm<2 * TL::LOADS>();
    else vwait_vm<0>();
    __syncthreads();  // every wave's share; the stage of tile i - 1 is free
    issue(i + TL::STAGES - 1);
    const int key0 = c0 + (t_first + i) * BN;
    const char* kl = smem + (2 * (i % TL::STAGES)) * TL::TILEB + k_rd;
    const char* vl = smem + (2 * (i % TL::STAGES) + 1) * TL::TILEB;

    // S^T = K . Q^T for the 32 keys of the tile: four accumulation chains over the k-steps
    // (a chain of dependent MFMAs issues at half rate), added in a fixed order
    v_floatx16 sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int x = 0; x < 16; ++x) sc[j][x] = 0.0f;
    {
      // K operands of k-step s + 2 read before the MFMA of step s (see verify_unit_staged)
      auto kread = [&](int st) { return *reinterpret_cast<const V8*>(kl + (((2 * st + hi) ^ k_sw) << 4)); };
      V8 k0 = kread(0), k1 = kread(1), k2 = k1;
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        if (s + 2 < KSTEPS) {
          k2 = kread(s + 2);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        sc[s & 3] = VMfma<T>::run(k0, qreg[s], sc[s & 3]);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        k0 = k1;
        k1 = k2;
      }
    }
    v_floatx16 sacc;
#pragma unroll
    for (int x = 0; x < 16; ++x) sacc[x] = (sc[0][x] + sc[1][x]) + (sc[2][x] + sc[3][x]);

    // element x of this lane is key key0 + 8(x/4) + 4hi + x%4 of row n; tiles every valid
    // row sees whole skip the mask (as in verify_unit_staged, the same values either way)
    float mx = kNegInf;
    const bool whole = key0 >= kmin_all && key0 + BN - 1 <= kmax_all;
    if (!whole) {
      const int lo = kmin - key0 - 4 * hi, top = kmax - key0 - 4 * hi;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int ce = 8 * (x >> 2) + (x & 3);
        sacc[x] = (ce >= lo && ce <= top) ? sacc[x] : kNegInf;
      }
    }
#pragma unroll
    for (int x = 0; x < 16; ++x) mx = fmaxf(mx, sacc[x]);
    mx = max_xor32(mx) * cl2;
    if (mx > m_run + kRescaleLog2) {  // (m = -inf: first visible key)
      const float alpha = m_run == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m_run - mx);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DBW; ++d)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[d][x] *= alpha;
      m_run = mx;
    }
    const float neg_m = -m_run;
    float rs = 0.0f;
    if (whole) {
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[x], cl2, neg_m));
        sacc[x] = pv;
        rs += pv;
      }
    } else {
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float pv = sacc[x] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sacc[x], cl2, neg_m));
        sacc[x] = pv;
        rs += pv;
      }
    }
    l_run += rs;

    // O^T += V^T . P^T over this wave's channels (two 16-key MFMA steps)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      V8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = from_f32<T>(sacc[8 * hf + e]);
      const char* vrow0 = vl + (16 * hf + v_row) * TL::ROWB + v_byte;
#pragma unroll
      for (int d = 0; d < DBW; ++d) {
        const int ch = ((4 * (wave * DBW + d) + v_chlo) ^ v_sw) << 4;
        const v_i16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v_i16x4*)(vrow0 + ch));
        const v_i16x4 vup = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v_i16x4*)(vrow0 + 8 * TL::ROWB + ch));
        typedef short i16x8 __attribute__((ext_vector_type(8)));
        const i16x8 av = __builtin_shufflevector(vlo, vup, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[d] = VMfma<T>::run(__builtin_bit_cast(V8, av), pb, oacc[d]);
      }
    }
  }

  // The row's total over the two lane halves; the chunk's result: final output when the
  // row's visible keys lie in this chunk only, else an fp32 partial (m, l, o).
  l_run += __shfl_xor(l_run, 32, kWave);
  if (!valid || c0 > kmax || c0 + p.chunk - 1 < kmin) return;
  const int cmin = kmin / p.chunk, cmax = kmax / p.chunk;
  // lane holds channels wave*DW + 32d + 8i + 4hi + j of row n
  if (cmin == cmax) {
    const float inv_l = 1.0f / l_run;
    T* dst = static_cast<T*>(p.out) + b * p.sob + t * p.sot + h * p.soh + wave * TL::DW;
#pragma unroll
    for (int d = 0; d < DBW; ++d)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[32 * d + 8 * ii + 4 * hi + j] = from_f32<T>(oacc[d][4 * ii + j] * inv_l);
  } else {
    const int64_t rowid = ((int64_t)b * p.H + h) * p.T + t;
    const int64_t slot = rowid * p.max_chunks + c;
    float* dst = p.ws_o + slot * D + wave * TL::DW;
#pragma unroll
    for (int d = 0; d < DBW; ++d)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        *reinterpret_cast<float4*>(dst + 32 * d + 8 * ii + 4 * hi) =
            make_float4(oacc[d][4 * ii], oacc[d][4 * ii + 1], oacc[d][4 * ii + 2], oacc[d][4 * ii + 3]);
    if (wave == 0 && hi == 0) p.ws_ml[slot] = make_float2(m_run, l_run);
  }
}

// Head dims 128 and 256, and 512 on the dense grid: the K and V tiles go from HBM into
// registers (16-byte non-temporal loads, two tiles in flight) and the threads write them
// into two LDS stages with the same swizzled layouts. A CU streams about 23-30 GB/s through
// direct-to-LDS loads whatever the waves and depth, against 36-48 GB/s through registers
// (7.3 against 5.9 TB/s over the chip), and the q rows and tables, loaded first into
// registers, no longer queue behind the tiles. LDS: two stages of K and V, the normalised q
// rows (chunk-swizzled by row, so the Q^T operand reads are conflict-free) and the tables.
template <int D> struct StagedTile {
  static constexpr int WAVES = 4;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int ROWS = 32;
  static constexpr int BN = 32;                                 // keys per tile
  static constexpr int NCH = D / 8;                             // 16-byte chunks per key row
  static constexpr int ROWB = 2 * D;
  static constexpr int TILEB = BN * ROWB;                       // one K (or V) tile
  static constexpr int PER = TILEB / (THREADS * 16);            // pieces per thread per tile
  static constexpr int MAX_TOK = ROWS / VerifyTile<D>::MIN_G + 1;
  static constexpr int TAB_G = (4 * D + 1023) / 1024 * 1024;
  static constexpr int TAB_R = (MAX_TOK * 4 * D + 1023) / 1024 * 1024;
  static constexpr int QS_OFF = 4 * TILEB;                      // after [K0 | V0 | K1 | V1]
  // the tables are read only by the q prologue, before tile 1 is written into stage 1: they
  // share its bytes, so a block takes 80 KB at head dim 256 and a CU holds two
  static constexpr int TAB_OFF = 2 * TILEB;
  static constexpr int LDS_BYTES = QS_OFF + ROWS * ROWB;
  // Q^T operands: all in registers at 128; at 256 read from the q rows in LDS per tile; at
  // 512 the score tile is split over the waves by k-steps (SPLIT_S) and each wave holds its
  // quarter of the operands in registers
  static constexpr bool Q_REGS = D <= 128;
  static constexpr bool SPLIT_S = D >= 512;
  // score accumulation chains: two at 256 (two waves per SIMD, registers short); four at 512
  // (one per wave), added as verify_unit_dma adds its four, so both forms give the same bits
  static constexpr int NCHAIN = D == 256 ? 2 : 4;
  static constexpr int NR = 2;                     // register sets of tiles in flight
  static constexpr int DW = D / WAVES;
  static_assert(PER * THREADS * 16 == TILEB, "a tile splits into whole 16-byte pieces per thread");
  static_assert(NCH >= 16, "the K swizzle spans 16 chunks");
  static_assert(TAB_G + 2 * TAB_R <= 2 * TILEB, "the tables fit in stage 1");
};

template <typename T, int D>
__device__ __forceinline__ void verify_unit_staged(const SplitParams& p, char* smem, const int b,
                                                   const int base, const int kvh, const int rb,
                                                   const int c_in) {
  using V8 = typename VMfma<T>::vec;
  using TL = StagedTile<D>;
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  constexpr int BN = TL::BN;
  constexpr int KSTEPS = D / 16;
  constexpr int DBW = TL::DW / 32;  // 32-channel blocks per wave

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int n = lane & 31;
  const int hi = lane >> 5;

  // this lane's row and its visible keys; the unit's key span (union over valid rows)
  const int flat = rb * TL::ROWS + n;
  const bool valid = flat < p.rows_total;
  const int t = valid ? flat / p.G : 0;
  const int h = kvh * p.G + (valid ? flat % p.G : 0);
  int kmin = INT_MAX, kmax = -1;
  if (valid) visible_range32(base + t, p.window, (int)p.max_len, kmin, kmax);
  int umin, umax, dummy;
  {
    const int r_hi = rb * TL::ROWS + TL::ROWS - 1 < p.rows_total - 1 ? rb * TL::ROWS + TL::ROWS - 1 : p.rows_total - 1;
    visible_range32(base + rb * TL::ROWS / p.G, p.window, (int)p.max_len, umin, dummy);
    visible_range32(base + r_hi / p.G, p.window, (int)p.max_len, dummy, umax);
  }
  // keys every valid row of the unit sees: the last token's first key to the first token's last
  int kmin_all, kmax_all;
  {
    const int r_hi = rb * TL::ROWS + TL::ROWS - 1 < p.rows_total - 1 ? rb * TL::ROWS + TL::ROWS - 1 : p.rows_total - 1;
    visible_range32(base + r_hi / p.G, p.window, (int)p.max_len, kmin_all, dummy);
    visible_range32(base + rb * TL::ROWS / p.G, p.window, (int)p.max_len, dummy, kmax_all);
  }
  const int c = p.span_chunks ? umin / p.chunk + c_in : c_in;  // absolute chunk
  const int c0 = c * p.chunk;
  if (c >= p.max_chunks || c0 > umax || c0 + p.chunk - 1 < umin) return;  // block-uniform

  // New positions in this chunk (forge_attn_decode_append): made and written before any
  // tile load, as in verify_unit_dma.
  if (p.kn) {
    int n_lo = base > c0 ? base : c0;
    int n_hi = base + p.T - 1 < c0 + p.chunk - 1 ? base + p.T - 1 : c0 + p.chunk - 1;
    if (n_hi > (int)p.max_len - 1) n_hi = (int)p.max_len - 1;
    if (n_lo <= n_hi) {  // block-uniform
      constexpr int VEC = 16 / sizeof(T);
      constexpr int LPR = D / VEC;
      constexpr int RPP = 256 / LPR;
      const int li = tid % LPR, rr = tid / LPR;
      const int64_t slab = b * p.skb + kvh * p.skh;
      for (int p0 = n_lo; p0 <= n_hi; p0 += RPP) {
        const int pp = p0 + rr;
        const int tt = (pp <= n_hi ? pp : n_hi) - base;
        const T* kr = static_cast<const T*>(p.kn) + b * p.sknb + kvh * p.sknh + tt * p.sknt + li * VEC;
        const T* vr = static_cast<const T*>(p.vn) + b * p.svnb + kvh * p.svnh + tt * p.svnt + li * VEC;
        const bool krope = p.kvflags & FORGE_ROPE;
        const float* cr = krope ? p.cos + b * p.csb + tt * p.cst : nullptr;
        const float* sr = krope ? p.sin + b * p.csb + tt * p.cst : nullptr;
        const uint4 nk = new_row_slice<T, D>(load16(kr), p.kvflags & FORGE_NORM_QK, p.kw, p.eps, cr, sr, li);
        const uint4 nv = new_row_slice<T, D>(load16(vr), p.kvflags & FORGE_NORM_V, nullptr, p.eps,
                                             nullptr, nullptr, li);
        if (pp <= n_hi) {
          store16(static_cast<T*>(p.kcw) + slab + (int64_t)pp * p.sks + li * VEC, nk);
          store16(static_cast<T*>(p.vcw) + slab + (int64_t)pp * p.sks + li * VEC, nv);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  int t_first = umin > c0 ? (umin - c0) / BN : 0;
  int t_last = (umax - c0) / BN;
  if (t_last > p.chunk / BN - 1) t_last = p.chunk / BN - 1;
  const int ntiles = t_last - t_first + 1;

  // ---- q rows, q gains and RoPE rows first (registers), then the first two tiles. Loads
  // retire in issue order, so q is usable after one round trip while the tiles stream.
  const bool gains = (p.flags & FORGE_NORM_QK) && p.qw;
  const bool rope = (p.flags & FORGE_ROPE) != 0;
  const int tok_lo = rb * TL::ROWS / p.G;
  const int tok_hi = (rb * TL::ROWS + TL::ROWS - 1 < p.rows_total - 1 ? rb * TL::ROWS + TL::ROWS - 1 : p.rows_total - 1) / p.G;
  const int ntok = tok_hi - tok_lo + 1;  // <= MAX_TOK for G >= MIN_G
  char* qs_b = smem + TL::QS_OFF;       // normalised q rows [ROWS][D], chunk c of row r at c ^ (r & 15)
  char* tab_b = smem + TL::TAB_OFF;     // [gains | cos rows | sin rows], regions padded
  float* tab = reinterpret_cast<float*>(tab_b);
  const float* tab_cos = reinterpret_cast<const float*>(tab_b + TL::TAB_G);
  const float* tab_sin = reinterpret_cast<const float*>(tab_b + TL::TAB_G + TL::TAB_R);
  // q math split over the waves: this lane normalises and rotates row qr = 8 * wave + lane / 8,
  // first-half channels qx .. qx + QCH - 1 and their RoPE partners qx + D/2
  constexpr int QCH = D / 16;
  const int qr = 8 * wave + (lane >> 3);
  const int qx = QCH * (lane & 7);
  const int qflat = rb * TL::ROWS + qr;
  const bool qvalid = qflat < p.rows_total;
  const int qtok = qvalid ? qflat / p.G : 0;
  uint4 qa[QCH / 8], qz[QCH / 8];
  {
    const int qh = kvh * p.G + (qvalid ? qflat % p.G : 0);
    const T* src = static_cast<const T*>(p.q) + b * p.sqb + qh * p.sqh + qtok * p.sqt + qx;
#pragma unroll
    for (int j = 0; j < QCH / 8; ++j) {
      qa[j] = load16(src + 8 * j);
      qz[j] = load16(src + D / 2 + 8 * j);
    }
  }
  // Tables as rows [gains | ntok cos rows | ntok sin rows] (rows present per the flags): with
  // 16-byte aligned tables (p.vec_tables) thread tid loads 4 floats of row ps * RPP + tid / V4R
  // per pass, else single floats. (Index math per value, with a division by ntok, cost about
  // as much as the loads' round trip.)
  constexpr int V4R = D / 4;                       // 16-byte pieces per table row
  constexpr int RPP = TL::THREADS / V4R;           // rows per pass
  constexpr int NPASS = (1 + 2 * TL::MAX_TOK + RPP - 1) / RPP;
  const int nrow = (gains ? 1 : 0) + (rope ? 2 * ntok : 0);
  const float* cos0 = rope ? p.cos + b * p.csb + (int64_t)tok_lo * p.cst : nullptr;
  const float* sin0 = rope ? p.sin + b * p.csb + (int64_t)tok_lo * p.cst : nullptr;
  // table row r of this call: source row, and its float offset in `tab`
  auto tab_src = [&](int r) {
    const int rr = gains ? r : r + 1;  // 0 gains, 1..ntok cos, ntok+1.. sin
    return rr == 0 ? p.qw : rr <= ntok ? cos0 + (int64_t)(rr - 1) * p.cst : sin0 + (int64_t)(rr - 1 - ntok) * p.cst;
  };
  auto tab_dst = [&](int r) {
    const int rr = gains ? r : r + 1;
    return rr == 0 ? 0 : rr <= ntok ? TL::TAB_G / 4 + (rr - 1) * D : (TL::TAB_G + TL::TAB_R) / 4 + (rr - 1 - ntok) * D;
  };
  float4 tv[NPASS];
  const int tx = 4 * (tid % V4R);
  if (p.vec_tables) {
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int r = ps * RPP + tid / V4R;
      if (r < nrow) tv[ps] = *reinterpret_cast<const float4*>(tab_src(r) + tx);
    }
  } else {
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int r = ps * RPP + tid / V4R;
      if (r < nrow) {
        const float* src = tab_src(r) + tx;
        tv[ps] = make_float4(src[0], src[1], src[2], src[3]);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the small loads ahead of the tile loads

  // piece j of this thread: 16-byte chunk ch of key row `row` of the tile, written to LDS
  // chunk position ch ^ swizzle(row); rows past the unit's last key re-read that key (masked)
  const char* kgb = reinterpret_cast<const char*>(static_cast<const T*>(p.kc) + b * p.skb + kvh * p.skh);
  const char* vgb = reinterpret_cast<const char*>(static_cast<const T*>(p.vc) + b * p.skb + kvh * p.skh);
  const int rstride = (int)p.sks * 2;
  // byte offset of piece j within a full tile (32-bit, from a block-uniform tile base)
  unsigned poff[TL::PER];
#pragma unroll
  for (int j = 0; j < TL::PER; ++j) {
    const int slot = j * TL::THREADS + tid;
    poff[j] = (unsigned)((slot / TL::NCH) * rstride + (slot % TL::NCH) * 16);
  }
  auto load_tile = [&](int i, u4 (&kr)[TL::PER], u4 (&vr)[TL::PER]) {
    const int key0 = c0 + (t_first + i) * BN;
    const int rows_left = umax - key0 + 1;  // block-uniform
    const char* kt = kgb + (int64_t)key0 * rstride;
    const char* vt = vgb + (int64_t)key0 * rstride;
    if (rows_left >= BN) {
#pragma unroll
      for (int j = 0; j < TL::PER; ++j) {
        kr[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(kt + poff[j]));
        vr[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(vt + poff[j]));
      }
    } else {
#pragma unroll
      for (int j = 0; j < TL::PER; ++j) {
        const int slot = j * TL::THREADS + tid;
        const int row = slot / TL::NCH, ch = slot % TL::NCH;
        const unsigned off = (unsigned)((row < rows_left ? row : rows_left - 1) * rstride + ch * 16);
        kr[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(kt + off));
        vr[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(vt + off));
      }
    }
  };
  auto store_tile = [&](int stage, const u4 (&kr)[TL::PER], const u4 (&vr)[TL::PER]) {
    char* kd = smem + (2 * stage) * TL::TILEB;
    char* vd = kd + TL::TILEB;
#pragma unroll
    for (int j = 0; j < TL::PER; ++j) {
      const int slot = j * TL::THREADS + tid;
      const int row = slot / TL::NCH, ch = slot % TL::NCH;
      *reinterpret_cast<u4*>(kd + row * TL::ROWB + ((ch ^ vswz_k(row)) << 4)) = kr[j];
      *reinterpret_cast<u4*>(vd + row * TL::ROWB + ((ch ^ vswz_v(row)) << 4)) = vr[j];
    }
  };
  // NR register sets: tile i sits in set i % NR until it moves to LDS, so NR tiles are in
  // flight while one is computed (about 96 KB per CU either way: three sets of one block at
  // head dim 256, two sets of each of two blocks at 128; fewer bytes in flight leave a CU
  // below its share of the HBM bandwidth)
  constexpr int NR = TL::NR;
  u4 r0k[TL::PER], r0v[TL::PER], r1k[TL::PER], r1v[TL::PER], r2k[NR > 2 ? TL::PER : 1], r2v[NR > 2 ? TL::PER : 1];
  // Tile 0 goes out with the q rows and tables; the later tiles wait for them: every block
  // of the launch requests its q rows at once, and more tile requests issued with them
  // would put each block's q behind the whole launch's first tiles (5 us at C5's global
  // layer with three tiles, against about one round trip alone).
  load_tile(0, r0k, r0v);
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int r = ps * RPP + tid / V4R;
    if (r < nrow) *reinterpret_cast<float4*>(tab + tab_dst(r) + tx) = tv[ps];
  }
  __builtin_amdgcn_sched_barrier(0);
  if (ntiles > 1) load_tile(1, r1k, r1v);
  if constexpr (NR > 2) {
    if (ntiles > 2) load_tile(2, r2k, r2v);
  }
  __syncthreads();  // tables in LDS

  // Fused RMSNorm + RoPE of this lane's q values in fp32, one rounding (as the split kernel's
  // q prologue), stored as T in the swizzled q rows.
  {
    float a[QCH], z[QCH];
#pragma unroll
    for (int j = 0; j < QCH / 8; ++j) {
      unpack16<T>(qa[j], a + 8 * j);
      unpack16<T>(qz[j], z + 8 * j);
    }
    if (!qvalid) {
#pragma unroll
      for (int e = 0; e < QCH; ++e) a[e] = z[e] = 0.0f;
    }
    float rs = 1.0f;
    if (p.flags & FORGE_NORM_QK) {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < QCH; ++e) ss += a[e] * a[e] + z[e] * z[e];
      ss += __shfl_xor(ss, 1, kWave);
      ss += __shfl_xor(ss, 2, kWave);
      ss += __shfl_xor(ss, 4, kWave);
      rs = rsqrtf(ss / (float)D + p.eps);
    }
#pragma unroll
    for (int j = 0; j < QCH / 8; ++j) {
      const int x = qx + 8 * j;
      float* aj = a + 8 * j;
      float* zj = z + 8 * j;
      if (gains) {
        float wa[8], wz[8];
        load_f32x8(tab + x, wa);
        load_f32x8(tab + x + D / 2, wz);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          aj[e] = aj[e] * rs * wa[e];
          zj[e] = zj[e] * rs * wz[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          aj[e] *= rs;
          zj[e] *= rs;
        }
      }
      if (rope && qvalid) {
        const float* cr = tab_cos + (qtok - tok_lo) * D;
        const float* sr = tab_sin + (qtok - tok_lo) * D;
        float c1[8], s1[8], c2[8], s2[8];
        load_f32x8(cr + x, c1);
        load_f32x8(sr + x, s1);
        load_f32x8(cr + x + D / 2, c2);
        load_f32x8(sr + x + D / 2, s2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float a0 = aj[e], z0 = zj[e];
          aj[e] = a0 * c1[e] - z0 * s1[e];
          zj[e] = z0 * c2[e] + a0 * s2[e];
        }
      }
      const int sw = qr & 15;
      *reinterpret_cast<uint4*>(qs_b + qr * TL::ROWB + (((x / 8) ^ sw) << 4)) = pack16<T>(aj);
      *reinterpret_cast<uint4*>(qs_b + qr * TL::ROWB + ((((x + D / 2) / 8) ^ sw) << 4)) = pack16<T>(zj);
    }
  }
  store_tile(0, r0k, r0v);
  if (ntiles > NR) load_tile(NR, r0k, r0v);
  __syncthreads();  // q rows and tile 0 in LDS

  // Q^T operand of k-step s: channels 16s + 8hi .. of row n
  const char* q_rd = qs_b + n * TL::ROWB;
  const int q_sw = n & 15;
  auto qop = [&](int s) { return *reinterpret_cast<const V8*>(q_rd + (((2 * s + hi) ^ q_sw) << 4)); };
  // At head dim 512 the score tile is split over the waves by k-steps: wave w computes chain
  // w of verify_unit_dma's four (k-steps w, w + 4, ...), holds only those Q^T operands, and
  // the four partial tiles meet in LDS (the q rows' bytes, free once every wave holds its
  // operands) and are added as verify_unit_dma adds its chains, so both forms give the same
  // bits. A wave then reads 8 rather than 32 K operands per tile and issues 8 score MFMAs.
  constexpr bool SPLIT_S = TL::SPLIT_S;
  constexpr int QR = TL::Q_REGS ? KSTEPS : SPLIT_S ? KSTEPS / TL::WAVES : 1;
  V8 qreg[QR];
  if constexpr (TL::Q_REGS) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) qreg[s] = qop(s);
  } else if constexpr (SPLIT_S) {
#pragma unroll
    for (int j = 0; j < QR; ++j) qreg[j] = qop(wave + TL::WAVES * j);
    __syncthreads();  // every wave holds its operands: the q rows' bytes take the partial tiles
  }
  char* part = smem + TL::QS_OFF;  // [wave][4][64 lanes] float4 partial score tiles

  // LDS read offsets within a tile (as verify_unit_dma's)
  const int k_rd = n * TL::ROWB;
  const int k_sw = vswz_k(n);
  const int g = lane >> 4, kq = (lane >> 2) & 3, qq = lane & 3;
  const int v_row = 4 * (g >> 1) + kq;
  const int v_sw = vswz_v(v_row);
  const int v_chlo = 2 * (g & 1) + (qq >> 1);
  const int v_byte = 8 * (qq & 1);

  v_floatx16 oacc[DBW];
#pragma unroll
  for (int d = 0; d < DBW; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.0f;
  float m_run = kNegInf, l_run = 0.0f;
  const float cl2 = p.scale_log2;

  // One tile: compute tile i from stage i % 2, then move tile i + 1 from its registers (nk,
  // nv: set (i + 1) % NR) into the other stage (free since the last barrier) and reuse those
  // registers for tile i + 1 + NR.
  auto step = [&](int i, u4 (&nk)[TL::PER], u4 (&nv)[TL::PER]) {
    const int stage = i & 1;
    const int key0 = c0 + (t_first + i) * BN;
    const char* kl = smem + (2 * stage) * TL::TILEB + k_rd;
    const char* vl = smem + (2 * stage + 1) * TL::TILEB;

    // S^T = K . Q^T for the 32 keys of the tile: NCHAIN accumulation chains over the k-steps
    // (a chain of dependent MFMAs issues at half rate), added in a fixed order
    // The operands of k-step s + 2 are read before the MFMA of step s is issued (three
    // register sets), so the LDS latency hides under two MFMAs; the scheduling groups pin
    // that order (left alone, the compiler reads each step's operands just before its MFMA
    // and waits for them: one LDS round trip per MFMA).
    v_floatx16 sacc;
    if constexpr (SPLIT_S) {
      v_floatx16 sw;
#pragma unroll
      for (int x = 0; x < 16; ++x) sw[x] = 0.0f;
      auto kread = [&](int st) { return *reinterpret_cast<const V8*>(kl + (((2 * st + hi) ^ k_sw) << 4)); };
      V8 k0 = kread(wave), k1 = kread(wave + TL::WAVES), k2 = k1;
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        if (j + 2 < QR) {
          k2 = kread(wave + TL::WAVES * (j + 2));
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        sw = VMfma<T>::run(k0, qreg[j], sw);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        k0 = k1;
        k1 = k2;
      }
      float4* pw = reinterpret_cast<float4*>(part + wave * 4096) + lane;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) pw[64 * qd] = make_float4(sw[4 * qd], sw[4 * qd + 1], sw[4 * qd + 2], sw[4 * qd + 3]);
      __syncthreads();  // the four partial tiles in LDS
      v_floatx16 pt[TL::WAVES];
#pragma unroll
      for (int w = 0; w < TL::WAVES; ++w)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const float4 v = reinterpret_cast<const float4*>(part + w * 4096)[64 * qd + lane];
          pt[w][4 * qd] = v.x;
          pt[w][4 * qd + 1] = v.y;
          pt[w][4 * qd + 2] = v.z;
          pt[w][4 * qd + 3] = v.w;
        }
#pragma unroll
      for (int x = 0; x < 16; ++x) sacc[x] = (pt[0][x] + pt[1][x]) + (pt[2][x] + pt[3][x]);
    } else {
      v_floatx16 sc[TL::NCHAIN];
#pragma unroll
      for (int j = 0; j < TL::NCHAIN; ++j)
#pragma unroll
        for (int x = 0; x < 16; ++x) sc[j][x] = 0.0f;
      {
        constexpr int RD = TL::Q_REGS ? 1 : 2;  // LDS reads per k-step
        auto kread = [&](int st) { return *reinterpret_cast<const V8*>(kl + (((2 * st + hi) ^ k_sw) << 4)); };
        auto qget = [&](int st) { return TL::Q_REGS ? qreg[TL::Q_REGS ? st : 0] : qop(st); };
        V8 k0 = kread(0), k1 = kread(1), k2 = k1;
        V8 q0 = qget(0), q1 = qget(1), q2 = q1;
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * RD, 0);
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st) {
          if (st + 2 < KSTEPS) {
            k2 = kread(st + 2);
            q2 = qget(st + 2);
            __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
          }
          sc[st % TL::NCHAIN] = VMfma<T>::run(k0, q0, sc[st % TL::NCHAIN]);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          k0 = k1;
          k1 = k2;
          q0 = q1;
          q1 = q2;
        }
      }
#pragma unroll
      for (int x = 0; x < 16; ++x)
        sacc[x] = TL::NCHAIN == 4 ? (sc[0][x] + sc[1][x]) + (sc[2][x] + sc[TL::NCHAIN - 1][x]) : sc[0][x] + sc[1][x];
    }

    // element x of this lane is key key0 + 8(x/4) + 4hi + x%4 of row n. A tile every valid
    // row of the unit sees whole (block-uniform) skips the mask and the masked-key tests; both
    // forms compute the same values bit for bit (the max over raw scores, scaled once; weights
    // exp2(fma(s, c, -m))), so a tile's path never changes a row's result.
    float mx = kNegInf;
    const bool whole = key0 >= kmin_all && key0 + BN - 1 <= kmax_all;
    if (!whole) {
      const int lo = kmin - key0 - 4 * hi, top = kmax - key0 - 4 * hi;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int ce = 8 * (x >> 2) + (x & 3);
        sacc[x] = (ce >= lo && ce <= top) ? sacc[x] : kNegInf;
      }
    }
#pragma unroll
    for (int x = 0; x < 16; ++x) mx = fmaxf(mx, sacc[x]);
    mx = max_xor32(mx) * cl2;
    if (mx > m_run + kRescaleLog2) {  // (m = -inf: first visible key)
      const float alpha = m_run == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m_run - mx);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DBW; ++d)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[d][x] *= alpha;
      m_run = mx;
    }
    const float neg_m = -m_run;
    float rs = 0.0f;
    if (whole) {
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[x], cl2, neg_m));
        sacc[x] = pv;
        rs += pv;
      }
    } else {
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float pv = sacc[x] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sacc[x], cl2, neg_m));
        sacc[x] = pv;
        rs += pv;
      }
    }
    l_run += rs;

    // O^T += V^T . P^T over this wave's channels (two 16-key MFMA steps)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      V8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = from_f32<T>(sacc[8 * hf + e]);
      const char* vrow0 = vl + (16 * hf + v_row) * TL::ROWB + v_byte;
#pragma unroll
      for (int d = 0; d < DBW; ++d) {
        const int ch = ((4 * (wave * DBW + d) + v_chlo) ^ v_sw) << 4;
        const v_i16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v_i16x4*)(vrow0 + ch));
        const v_i16x4 vup = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v_i16x4*)(vrow0 + 8 * TL::ROWB + ch));
        typedef short i16x8 __attribute__((ext_vector_type(8)));
        const i16x8 av = __builtin_shufflevector(vlo, vup, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[d] = VMfma<T>::run(__builtin_bit_cast(V8, av), pb, oacc[d]);
      }
    }
    if (i + 1 < ntiles) {
      store_tile(stage ^ 1, nk, nv);
      if (i + 1 + NR < ntiles) load_tile(i + 1 + NR, nk, nv);
    }
    __syncthreads();  // tile i + 1 in LDS; the stage of tile i is free
  };
  if constexpr (NR > 2) {
    for (int i = 0; i < ntiles; i += 3) {
      step(i, r1k, r1v);
      if (i + 1 < ntiles) step(i + 1, r2k, r2v);
      if (i + 2 < ntiles) step(i + 2, r0k, r0v);
    }
  } else {
    for (int i = 0; i < ntiles; i += 2) {
      step(i, r1k, r1v);
      if (i + 1 < ntiles) step(i + 1, r0k, r0v);
    }
  }

  // The row's total over the two lane halves; the chunk's result: final output when the
  // row's visible keys lie in this chunk only, else an fp32 partial (m, l, o).
  l_run += __shfl_xor(l_run, 32, kWave);
  if (!valid || c0 > kmax || c0 + p.chunk - 1 < kmin) return;
  const int cmin = kmin / p.chunk, cmax = kmax / p.chunk;
  // lane holds channels wave*DW + 32d + 8i + 4hi + j of row n
  if (cmin == cmax) {
    const float inv_l = 1.0f / l_run;
    T* dst = static_cast<T*>(p.out) + b * p.sob + t * p.sot + h * p.soh + wave * TL::DW;
#pragma unroll
    for (int d = 0; d < DBW; ++d)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[32 * d + 8 * ii + 4 * hi + j] = from_f32<T>(oacc[d][4 * ii + j] * inv_l);
  } else {
    const int64_t rowid = ((int64_t)b * p.H + h) * p.T + t;
    const int64_t slot = rowid * p.max_chunks + c;
    float* dst = p.ws_o + slot * D + wave * TL::DW;
#pragma unroll
    for (int d = 0; d < DBW; ++d)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        *reinterpret_cast<float4*>(dst + 32 * d + 8 * ii + 4 * hi) =
            make_float4(oacc[d][4 * ii], oacc[d][4 * ii + 1], oacc[d][4 * ii + 2], oacc[d][4 * ii + 3]);
    if (wave == 0 && hi == 0) p.ws_ml[slot] = make_float2(m_run, l_run);
  }
}

// The staged form at every head dim, except the persistent grid at 512: there the staged
// form's 160 KB of LDS leaves no room for the grid's bookkeeping, and the direct-load form
// (150 KB) computes the same values bit for bit.
template <int D, bool PERSIST> constexpr bool verify_staged() { return D <= 256 || !PERSIST; }

template <typename T, int D, bool PERSIST>
__device__ __forceinline__ void verify_unit(const SplitParams& p, char* smem, const int b,
                                            const int base, const int kvh, const int rb,
                                            const int c_in) {
  if constexpr (verify_staged<D, PERSIST>()) verify_unit_staged<T, D>(p, smem, b, base, kvh, rb, c_in);
  else verify_unit_dma<T, D>(p, smem, b, base, kvh, rb, c_in);
}

// Dynamic LDS of the MFMA verify kernels.
template <int D, bool PERSIST> constexpr int verify_lds_bytes() {
  return verify_staged<D, PERSIST>() ? StagedTile<D>::LDS_BYTES : VerifyTile<D>::LDS_BYTES;
}

// Rows of a persistent MFMA verify launch held in LDS (their first new position, the prefix
// sums of their units and the hand-out order of their last chunks): under 8 KB, within the
// 80 KB a block may use for two blocks per CU at head dim 128.
constexpr int kVerifyPersistRows = 512;

// MFMA verify kernel, dense grid: one block per (chunk, KV head x row block, batch row).
// Waves per SIMD: two at head dims 128 and 256, so a CU may hold two blocks (the second
// block's waves run while the first one's wait on LDS reads and dependent MFMAs); at 512 one
// (160 KB of LDS per block, and two register sets of 32 KB tiles per wave).
template <int D> constexpr int verify_waves_per_eu() { return D >= 512 ? 1 : 2; }
// The persistent grid's bookkeeping (under 8 KB of static LDS) leaves one block per CU at 256,
// whose waves may then use the whole register file of their SIMD.
template <int D> constexpr int verify_persist_waves_per_eu() { return D >= 256 ? 1 : 2; }
constexpr int kVerifyPersistStaticLds = 8 * 1024;

template <typename T, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(verify_waves_per_eu<D>())))
void verify_mfma_kernel(SplitParams p) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int b = blockIdx.z;
  verify_unit<T, D, false>(p, smem, b, (int)row_base(p.row_pos, p.pos_dev, p.pos0, b), blockIdx.y % p.K,
                    blockIdx.y / p.K, blockIdx.x);
}

// MFMA verify kernel, persistent (per-row positions in device memory): verify_blocks_per_cu
// blocks per CU take the units (row, KV head x row block, chunk) of every row's own chunk range by
// ticket, as splitk_kernel does, so a ragged batch spends no blocks on chunks past a row's
// end and the blocks that stream faster take more units. (A kernel of its own: with both
// grids in one, the dense grid's registers grew from 150 to 212 at head dim 128.)
template <typename T, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(verify_persist_waves_per_eu<D>())))
void verify_mfma_persistent_kernel(SplitParams p) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  __shared__ int sh_pref[kVerifyPersistRows + 1];
  __shared__ int sh_base[kVerifyPersistRows];
  __shared__ int sh_last[kVerifyPersistRows];
  __shared__ unsigned char sh_cls[kVerifyPersistRows];
  __shared__ int sh_count[kLastClasses];
  __shared__ int sh_ticket[2];
  static_assert(sizeof(int) * (3 * kVerifyPersistRows + kLastClasses + 3) + kVerifyPersistRows <=
                    kVerifyPersistStaticLds, "bookkeeping LDS");
  const int tid = threadIdx.x;
  constexpr int ROWS = VerifyTile<D>::ROWS;
  const int per_row = p.K * ((p.rows_total + ROWS - 1) / ROWS);
  // chunks of each row: the union of its T queries' visible keys (wave 0 scans the rows)
  auto row_chunks = [&](int base) {
    int lo, hi0, lo1, hi;
    visible_range32(base, p.window, (int)p.max_len, lo, hi0);
    visible_range32(base + p.T - 1, p.window, (int)p.max_len, lo1, hi);
    const int cmin = lo / p.chunk;
    int cmax = hi / p.chunk;
    if (cmax > p.max_chunks - 1) cmax = p.max_chunks - 1;
    return (hi >= lo && cmax >= cmin) ? cmax - cmin + 1 : 0;
  };
  if (tid < kLastClasses) sh_count[tid] = 0;
  __syncthreads();
  for (int b = tid; b < p.B; b += blockDim.x) {
    const int base = (int)row_base(p.row_pos, p.pos_dev, p.pos0, b);
    sh_base[b] = base;
    const int cls = last_chunk_class(p, base);
    sh_cls[b] = (unsigned char)cls;
    atomicAdd(&sh_count[cls], 1);
  }
  __syncthreads();
  // units [0, body): every row's chunks but its last, (row, KV head x row block, chunk) with
  // the chunk fastest, each row's from its second-to-last chunk down; [body, total): the
  // rows' last chunks, largest first (as in splitk_kernel)
  if (tid < kWave) {
    const int seg = (p.B + kWave - 1) / kWave;
    const int r0 = tid * seg;
    const int r1 = r0 + seg < p.B ? r0 + seg : p.B;
    int sum = 0;
    for (int r = r0; r < r1; ++r) {
      const int n = row_chunks(sh_base[r]);
      sum += (n > 0 ? n - 1 : 0) * per_row;
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (tid >= d) incl += v;
    }
    int run = incl - sum;
    for (int r = r0; r < r1; ++r) {
      sh_pref[r] = run;
      const int n = row_chunks(sh_base[r]);
      run += (n > 0 ? n - 1 : 0) * per_row;
    }
    if (tid == kWave - 1) sh_pref[p.B] = incl;
  }
  order_last_chunks(p.B, sh_count, sh_cls, sh_last);
  const int body = sh_pref[p.B];
  const int total = body + p.B * per_row;
  // Block i starts with unit i, then takes units by ticket; the ticket slots alternate, as
  // in splitk_kernel (a unit may leave without a block barrier).
  int parity = 0;
  for (int u = blockIdx.x; u < total; u = __builtin_amdgcn_readfirstlane(sh_ticket[parity]), parity ^= 1) {
    int next = 0;
    if (tid == 0) next = atomicAdd(p.ws_ctr, 1);  // read after the unit: its round trip hides
    int lo, pr, cidx;  // row, (KV head, row block), chunk counted from the row's first
    if (u < body) {
      lo = 0;
      int hi = p.B - 1;  // last row with sh_pref[row] <= u
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (__builtin_amdgcn_readfirstlane(sh_pref[mid]) <= u) lo = mid;
        else hi = mid - 1;
      }
      const int o = u - __builtin_amdgcn_readfirstlane(sh_pref[lo]);
      const int n = row_chunks(__builtin_amdgcn_readfirstlane(sh_base[lo])) - 1;  // >= 1 here
      pr = o / n;
      cidx = n - 1 - o % n;
    } else {
      // a row with no visible key has no last chunk either: cidx -1 lies before every key,
      // and the unit returns at once
      const int q = u - body;
      lo = __builtin_amdgcn_readfirstlane(sh_last[q / per_row]);
      pr = q % per_row;
      cidx = row_chunks(__builtin_amdgcn_readfirstlane(sh_base[lo])) - 1;
    }
    const int base = __builtin_amdgcn_readfirstlane(sh_base[lo]);
    int kmin, kmax;
    visible_range32(base, p.window, (int)p.max_len, kmin, kmax);  // the row's first chunk
    verify_unit<T, D, true>(p, smem, lo, base, pr % p.K, pr / p.K, kmin / p.chunk + cidx);
    if (tid == 0) sh_ticket[parity] = (int)gridDim.x + next;
    __syncthreads();  // the next unit reuses the LDS stages and tables; the ticket is visible
  }
}

// ---------------------------------------------------------------- host side
static int vec_of(int dtype) { return dtype == FORGE_F32 ? 4 : 8; }

// Query rows per split-K block: up to 8, and up to 4 at head dim 512, where the block's
// merge buffer (4 waves x rows x D fp32) would otherwise exceed the 64 KB of static LDS.
template <int D> constexpr int split_max_rows() { return D >= 512 ? 4 : 8; }
static int rows_per_block(int rows_total, int D) {
  const int cap = D >= 512 ? split_max_rows<512>() : split_max_rows<256>();
  if (rows_total >= cap) return cap;
  int r = 1;
  while (r < rows_total) r <<= 1;
  return r;
}

static int keys_per_iter(int dtype, int D) { return (kSplitThreads / (D / vec_of(dtype))) * kSplitNK; }

// Head dims of the split-K kernel: a key row is held by D / (16 bytes) lanes, at most a
// wave, so 512 needs 2-byte elements (bf16/fp16: the full-attention layers of Gemma 4,
// reference kv_cache.py:12-13).
static bool head_dim_ok(int dtype, int D) {
  return D == 32 || D == 64 || D == 128 || D == 256 || (D == 512 && dtype != FORGE_F32);
}

// The MFMA path (verify_mfma_kernel) serves bf16/fp16 head dim 128/256 with G >= 4 query
// heads per KV head, whatever T is (so verify and decode of one model share it).
// Blocks of the MFMA verify kernel one CU holds (its LDS, 160 KB per CU, is the limit; the
// persistent kernel adds its static bookkeeping).
static int verify_blocks_per_cu(int D, bool persist = false) {
  const int lds = persist ? (D == 512   ? verify_lds_bytes<512, true>()
                             : D == 256 ? verify_lds_bytes<256, true>()
                                        : verify_lds_bytes<128, true>()) + kVerifyPersistStaticLds
                          : (D == 512   ? verify_lds_bytes<512, false>()
                             : D == 256 ? verify_lds_bytes<256, false>()
                                        : verify_lds_bytes<128, false>());
  const int n = (160 * 1024) / lds;
  return n < 1 ? 1 : (n > 2 ? 2 : n);
}

static bool use_verify_mfma(int dtype, int D, int G) {
  return dtype != FORGE_F32 && (((D == 128 || D == 256) && G >= VerifyTile<128>::MIN_G) ||
                                (D == 512 && G >= VerifyTile<512>::MIN_G));
}
constexpr int kVerifyRows = 32;

// Default chunk. It does not depend on T, so decode and verify calls of one model get the
// same chunk boundaries (and a verify row equals the decode of that token bit for bit);
// with a sliding window, pass the span a row can see (window + kMaxVerifyT).
constexpr int kMaxVerifyT = 16;
static int64_t chunk_span(int64_t max_kv_len, int window) {
  return window > 0 && window + kMaxVerifyT < max_kv_len ? window + kMaxVerifyT : max_kv_len;
}

// CUs of the current device (256 where no device answers, e.g. a host-only build check).
static int device_cus() {
  int ncu = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
    ncu = 256;
  return ncu;
}

// MFMA verify path: the smallest multiple of 32 keys that puts every unit into one round of
// the device's block slots (CUs x blocks per CU): with one more unit than slots, the last
// few full units run as a second round and double the kernel's time. (rows of T = 1, as
// the module asks.)
static int verify_round_chunk(int B, int H, int K, int D, int64_t max_kv_len) {
  const int T = 1;
  const int G = H / K;
  const int64_t pairs = (int64_t)B * K * ((G * T + kVerifyRows - 1) / kVerifyRows);
  const int64_t len = max_kv_len > 0 ? max_kv_len : 1;
  // At head dim 256 a CU holds two blocks, but one unit per CU writes half the fp32 partials
  // (C5 global layer, 8 x 8196 keys: 288-key chunks 27.2-28.0 us per call against 30.5-30.9 at
  // 160-192 keys, same box)
  const int64_t slots = (int64_t)(D == 256 ? 1 : verify_blocks_per_cu(D)) * device_cus();
  const int64_t per_pair = slots / pairs > 1 ? slots / pairs : 1;  // chunks per (b, kv head, rows)
  int64_t chunk = (len + per_pair - 1) / per_pair;
  chunk = (chunk + 31) / 32 * 32;
  // A shorter unit is mostly prologue: at least two tiles where the staged pipeline keeps two
  // in flight (C5 window 1024: 64-key chunks 14.9 us, 96-key 15.4 us, 32-key 17.3 us); three at
  // head dim 512, whose direct loads keep one tile in flight.
  static_assert(VerifyTile<128>::BN == StagedTile<128>::BN && VerifyTile<128>::BN == VerifyTile<512>::BN &&
                StagedTile<256>::BN == VerifyTile<512>::BN, "one tile shape for every head dim");
  const int min_tiles = D >= 512 ? 3 : StagedTile<128>::NR;
  const int64_t min_chunk = (int64_t)min_tiles * VerifyTile<128>::BN;
  return (int)(chunk < min_chunk ? min_chunk : chunk);
}

// Longest chunk of the MFMA verify path on the dense grid (per-row positions beyond the
// persistent grid's rows, and the host-position rule's cap): a ragged batch's long rows
// would otherwise be few long units that finish last (C4 lengths at 32 q / 8 KV heads:
// 1012 us per decode step at 512-key chunks against 1205 us for one chunk per row; 28 q /
// 4 KV heads, 32 rows: 208 against 304 us; 8 q / 1 KV head, T = 4, 32 rows: 72 against
// 90 us; 256-key chunks were as fast or slower, 1024 slower for all three).
constexpr int kMaxVerifyChunk = 512;
// The same on the persistent grid (per-row positions, up to kVerifyPersistRows rows), whose
// tickets leave no block idle behind a long row: there fewer, longer units win (C4 lengths
// at 32 q / 8 KV heads: 688.5 us per decode step at 1024-key chunks against 723.6 at 512
// and 712.1 at 2048; T = 5 verify 794.3 against 853.1; 28 q / 4 KV heads, 32 rows: 186.0
// against 192.6; 8 q / 1 KV head, T = 4: 58.7 against 66.2 us, and 77.0 at 2048).
constexpr int kMaxVerifyChunkPersist = 1024;

static int auto_chunk(int dtype, int B, int /*T*/, int H, int K, int D, int64_t max_kv_len) {
  const int T = 1;
  const int G = H / K;
  if (use_verify_mfma(dtype, D, G)) {
    const int chunk = verify_round_chunk(B, H, K, D, max_kv_len);
    const int cap = B <= kVerifyPersistRows ? kMaxVerifyChunkPersist : kMaxVerifyChunk;
    return chunk < cap ? chunk : cap;
  }
  const int rows = rows_per_block(G * T, D);
  const int64_t n_rb = (G * T + rows - 1) / rows;
  const int64_t pairs = (int64_t)B * K * n_rb;
  // At least 4 block iterations per unit (a one-iteration unit spends most of its time in
  // the q prologue and the merge), then larger, up to 1024 keys, while at least one unit
  // per CU remains: fewer, longer units spend less on prologues, merges and partials, and
  // the cap keeps the units a ragged batch's longest rows leave for the end short (C4 step:
  // 609.5 us at 1024-key chunks, 610.6 at 768, 615.0 at 512; attention call 630 us at 2048).
  const int kpi = keys_per_iter(dtype, D);
  int chunk = kpi;
  const int64_t len = max_kv_len > 0 ? max_kv_len : 1;
  const int ncu = device_cus();
  while (chunk * 2 <= max_chunk_keys(kpi) &&
         (chunk < 4 * kpi || pairs * ((len + chunk * 2 - 1) / (chunk * 2)) >= ncu))
    chunk *= 2;
  return chunk;
}

// Default chunk for calls whose rows all start at one host position (the dense grid). Every
// row has the same length, so there is no ragged tail to balance and the chunk can be as
// long as the per-CU work allows: with U = pairs x chunks-per-row units spread over the
// CUs, a CU streams ceil(U / CUs) chunks, and the rule takes the longest chunk within 2% of
// the least such per-CU length (no split at all when the pairs already fill the CUs: C3
// decode, 256 (row, KV head) pairs of 8192 keys, 159 us per call against 171 us at 512-key
// chunks, which also pay for the partials and the combine launch). Like auto_chunk it
// ignores T. The MFMA verify path keeps its own rule.
static int uniform_chunk(int dtype, int B, int H, int K, int D, int64_t max_kv_len) {
  const int G = H / K;
  if (use_verify_mfma(dtype, D, G)) {
    // rows split four ways or more: as below, a capacity far above the rows' length must
    // not leave one long unit per row (C5's 8 rows in caches of 131072 would get 4096-key
    // chunks, 24 units)
    const int chunk = verify_round_chunk(B, H, K, D, max_kv_len);
    const int64_t pairs = (int64_t)B * K * ((G + kVerifyRows - 1) / kVerifyRows);
    const bool split = pairs * 4 <= (int64_t)verify_blocks_per_cu(D) * device_cus();
    return split && chunk > kMaxVerifyChunk ? kMaxVerifyChunk : chunk;
  }
  const int rows = rows_per_block(G, D);
  const int64_t pairs = (int64_t)B * K * ((G + rows - 1) / rows);
  const int kpi = keys_per_iter(dtype, D);
  const int64_t min_chunk = 4 * (int64_t)kpi;  // at least 4 block iterations per unit
  const int64_t len = max_kv_len > 0 ? max_kv_len : 1;
  const int64_t ncu = device_cus();
  int64_t best = -1, best_cost = 0;
  for (int64_t c = 1; c <= 4096; ++c) {  // chunks per row, longest chunk first
    const int64_t chunk = ((len + c - 1) / c + kpi - 1) / kpi * kpi;
    if (c > 1 && chunk < min_chunk) break;
    const int64_t per_row = (len + chunk - 1) / chunk;
    const int64_t cost = (pairs * per_row + ncu - 1) / ncu * chunk;  // keys per CU
    if (best < 0 || cost * 50 < best_cost * 49) {  // shorter chunks only if 2% better
      best = chunk;
      best_cost = cost;
    }
  }
  // With fewer pairs than CUs every row must be split to fill them. The span is a cache's
  // capacity, which a row may be far from reaching, so the chunk stays at most as long as
  // the general rule's (a capacity of 32768 at C2's 64 pairs would otherwise give 8192-key
  // chunks, one unit per row of 2049 keys: 30.9 us per call against 19.9 us).
  if (pairs < ncu && best > max_chunk_keys(kpi)) best = max_chunk_keys(kpi);
  return best > INT_MAX ? INT_MAX / kpi * kpi : (int)best;
}

// Persistent split-K blocks per CU. Fewer concurrent streams read HBM faster: on C4-shaped
// ragged decode 2 blocks per CU (each with a deeper prefetch) beat filling the CU.
constexpr int kPersistBlocksPerCU = 2;

// Persistent blocks of `kernel` for the current device: CUs x min(occupancy,
// kPersistBlocksPerCU), cached per (device, kernel); host queries only, so the launch stays
// graph-capturable.
static int resident_blocks(const void* kernel) {
  struct Entry { int dev; const void* k; int n; };
  static Entry cache[64];
  static int used = 0;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].dev == dev && cache[i].k == kernel) return cache[i].n;
  int ncu = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kSplitThreads, 0) != hipSuccess) return 0;
  if (per_cu > kPersistBlocksPerCU) per_cu = kPersistBlocksPerCU;
  const int n = ncu * (per_cu > 0 ? per_cu : 1);
  if (used < 64) cache[used++] = Entry{dev, kernel, n};
  return n;
}

// Dense grid over the chunks of the call: with a window, a unit's rows see at most
// window + T - 1 keys, so the grid covers that many chunks counted from each unit's first
// visible one (p.span_chunks) instead of every chunk of max_kv_len.
static int dense_chunks(SplitParams& p) {
  p.span_chunks = 0;
  if (p.window > 0) {
    const int64_t span = ((int64_t)p.window + p.T - 1 + p.chunk - 1) / p.chunk + 1;
    if (span < p.max_chunks) p.span_chunks = (int)span;
  }
  return p.span_chunks ? p.span_chunks : p.max_chunks;
}

template <typename T, int D>
static int launch_split_d(SplitParams p, int rows, hipStream_t s) {
  const int n_rb = (p.rows_total + rows - 1) / rows;
  const void* kern = nullptr;
  switch (rows) {
    case 1: kern = reinterpret_cast<const void*>(&splitk_kernel<T, D, 1>); break;
    case 2: kern = reinterpret_cast<const void*>(&splitk_kernel<T, D, 2>); break;
    case 4: kern = reinterpret_cast<const void*>(&splitk_kernel<T, D, 4>); break;
    case 8:
      if constexpr (split_max_rows<D>() >= 8) {
        kern = reinterpret_cast<const void*>(&splitk_kernel<T, D, 8>);
        break;
      }
      return set_error("internal: rows per block");
    default: return set_error("internal: rows per block");
  }
  dim3 grid;
  // Persistent only for per-row lengths (ragged rows): there it saves the blocks a dense
  // grid would spend past each row's end. With one position for every row, host-known or on
  // the device (graph steps), the dense grid is faster (C3 decode with the position on the
  // device: 163.7 us against 186.5 us persistent; 169.8 against 186.4 us in a cache of 4x
  // the rows' length), and the hardware's dynamic block dispatch balances uneven per-CU
  // bandwidth better than a fixed assignment does.
  if (p.row_pos != nullptr && p.B <= kPersistMaxRows && p.ws_ctr) {
    const int64_t upper = (int64_t)p.B * p.K * n_rb * p.max_chunks;
    int blocks = resident_blocks(kern);
    if (blocks <= 0) return set_error("forge_attn_decode: cannot query the device");
    if (upper < blocks) blocks = (int)upper;
    if ((int64_t)p.B * p.K * n_rb * p.max_chunks >= (1LL << 31))
      return set_error("forge_attn_decode: too many work units");
    p.persist = 1;
    grid = dim3((unsigned)blocks);
    if (!p.ws_zeroed) {
      hipLaunchKernelGGL(ticket_reset_kernel, dim3(1), dim3(64), 0, s, p.ws_ctr);
      const int st0 = check_launch();
      if (st0) return st0;
    }
  } else {
    if ((int64_t)p.K * n_rb > 65535 || p.B > 65535) return set_error("grid too large");
    p.persist = 0;
    grid = dim3((unsigned)dense_chunks(p), (unsigned)(p.K * n_rb), (unsigned)p.B);
  }
  switch (rows) {
#define FORGE_ROWS(R) \
  case R: hipLaunchKernelGGL((splitk_kernel<T, D, R>), grid, dim3(kSplitThreads), 0, s, p); break;
    FORGE_ROWS(1) FORGE_ROWS(2) FORGE_ROWS(4)
#undef FORGE_ROWS
    case 8:
      if constexpr (split_max_rows<D>() >= 8)
        hipLaunchKernelGGL((splitk_kernel<T, D, 8>), grid, dim3(kSplitThreads), 0, s, p);
      break;
  }
  int st = check_launch();
  if (st || p.max_chunks < 2) return st;
  const int64_t nrows = (int64_t)p.B * p.H * p.T;
  if (nrows > 0x7fffffff) return set_error("too many rows");
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3((unsigned)nrows), dim3(256), 0, s, p);
  return check_launch();
}

template <typename T, int D>
static int launch_verify_d(SplitParams p, hipStream_t s) {
  constexpr int LDS = verify_lds_bytes<D, false>();
  constexpr int LDS_P = verify_lds_bytes<D, true>();
  static bool attr_set = false;  // raise the dynamic LDS limit once per kernel
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&verify_mfma_kernel<T, D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, LDS) != hipSuccess ||
        hipFuncSetAttribute(reinterpret_cast<const void*>(&verify_mfma_persistent_kernel<T, D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, LDS_P) != hipSuccess)
      return set_error("forge_attn_decode: cannot reserve the LDS the kernel needs");
    attr_set = true;
  }
  const int n_rb = (p.rows_total + kVerifyRows - 1) / kVerifyRows;
  dim3 grid;
  // Persistent for per-row lengths. One device-held position for every row (a graph step)
  // keeps the dense grid: its rows end together, and the persistent launch's ticket reset
  // and set-up cost C5 (8 rows) 35.2 against 29.1 us per graph-replayed call.
  if (p.row_pos != nullptr && p.B <= kVerifyPersistRows && p.ws_ctr) {
    const int64_t upper = (int64_t)p.B * p.K * n_rb * p.max_chunks;
    if (upper >= (1LL << 31)) return set_error("forge_attn_decode: too many work units");
    int64_t blocks = (int64_t)verify_blocks_per_cu(D, true) * device_cus();
    if (upper < blocks) blocks = upper;
    p.persist = 1;
    grid = dim3((unsigned)blocks);
    if (!p.ws_zeroed) {
      hipLaunchKernelGGL(ticket_reset_kernel, dim3(1), dim3(64), 0, s, p.ws_ctr);
      const int st0 = check_launch();
      if (st0) return st0;
    }
  } else {
    if ((int64_t)p.K * n_rb > 65535 || p.B > 65535) return set_error("grid too large");
    p.persist = 0;
    grid = dim3((unsigned)dense_chunks(p), (unsigned)(p.K * n_rb), (unsigned)p.B);
  }
  if (p.persist)
    hipLaunchKernelGGL((verify_mfma_persistent_kernel<T, D>), grid, dim3(256), LDS_P, s, p);
  else
    hipLaunchKernelGGL((verify_mfma_kernel<T, D>), grid, dim3(256), LDS, s, p);
  int st = check_launch();
  if (st || p.max_chunks < 2) return st;
  const int64_t nrows = (int64_t)p.B * p.H * p.T;
  if (nrows > 0x7fffffff) return set_error("too many rows");
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3((unsigned)nrows), dim3(256), 0, s, p);
  return check_launch();
}

template <typename T>
static int launch_verify(const SplitParams& p, int D, hipStream_t s) {
  return D == 128 ? launch_verify_d<T, 128>(p, s)
                  : D == 256 ? launch_verify_d<T, 256>(p, s) : launch_verify_d<T, 512>(p, s);
}

template <typename T>
static int launch_split(const SplitParams& p, int D, int rows, hipStream_t s) {
  switch (D) {
    case 32: return launch_split_d<T, 32>(p, rows, s);
    case 64: return launch_split_d<T, 64>(p, rows, s);
    case 128: return launch_split_d<T, 128>(p, rows, s);
    case 256: return launch_split_d<T, 256>(p, rows, s);
    case 512:
      if constexpr (sizeof(T) == 2) return launch_split_d<T, 512>(p, rows, s);
      return set_error("forge_attn_decode: head dim 512 needs bf16 or fp16");
    default: return set_error("forge_attn_decode: head dim must be 32, 64, 128 or 256 (or 512 in bf16/fp16)");
  }
}

}  // namespace forge

using namespace forge;

extern "C" int forge_attn_decode_chunk(int dtype, int B, int T, int H, int K, int D,
                                       int64_t max_kv_len) {
  if (K <= 0 || H % K || !head_dim_ok(dtype, D) || T <= 0) return 0;
  return auto_chunk(dtype, B, T, H, K, D, max_kv_len);
}

extern "C" int forge_attn_decode_chunk_uniform(int dtype, int B, int T, int H, int K, int D,
                                               int64_t max_kv_len) {
  if (K <= 0 || H % K || !head_dim_ok(dtype, D) || T <= 0 || B <= 0) return 0;
  return uniform_chunk(dtype, B, H, K, D, max_kv_len);
}

// Workspace of a call with `slots` (row, chunk) partials: the persistent grid's work ticket
// (256 bytes), fp32 (m, l) pairs and fp32 partial outputs.
static size_t workspace_for(int64_t slots, int D) {
  const size_t ml = ((size_t)slots * sizeof(float2) + 255) / 256 * 256;
  const size_t o = ((size_t)slots * D * sizeof(float) + 255) / 256 * 256;
  return ml + o + 256;
}

extern "C" size_t forge_attn_decode_workspace_bytes(int dtype, int B, int T, int H, int K,
                                                    int D, int64_t max_kv_len, int chunk) {
  if (chunk <= 0) chunk = (K > 0 && H % K == 0) ? auto_chunk(dtype, B, T, H, K, D, max_kv_len) : 64;
  const int64_t max_chunks = (max_kv_len + chunk - 1) / chunk;
  if (max_chunks < 2) return 0;
  return workspace_for((int64_t)B * H * T * max_chunks, D);
}

namespace {

// Checks the arguments of a decode call and fills everything of p but the workspace.
// Returns 0, or the status of set_error.
int decode_setup(SplitParams& p, int dtype, int B, int T, int H, int K, int D, const void* q,
                 int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight, float eps,
                 int flags, const float* cos, const float* sin, int64_t s_cos_b, int64_t s_cos_t,
                 const void* k_cache, const void* v_cache, int64_t skb, int64_t skh, int64_t sks,
                 int64_t max_len, const int32_t* row_pos, const int64_t* pos_dev, int64_t pos0,
                 int64_t max_kv_len, int window, float scale, int chunk, void* out, int64_t sob,
                 int64_t sot, int64_t soh) {
  if (dtype != FORGE_F32 && dtype != FORGE_BF16 && dtype != FORGE_F16)
    return set_error("unknown dtype code");
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0) return set_error("sizes must be positive");
  if (H % K) return set_error("n_heads must be a multiple of the KV heads");
  if (!head_dim_ok(dtype, D))
    return set_error("forge_attn_decode: head dim must be 32, 64, 128 or 256 (or 512 in bf16/fp16)");
  if (!q || !k_cache || !v_cache || !out) return set_error("null tensor pointer");
  if ((flags & FORGE_ROPE) && (!cos || !sin)) return set_error("FORGE_ROPE needs cos and sin");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16)
    return set_error("forge_attn_decode: q and the caches must be 16-byte aligned");
  const int vec = vec_of(dtype);
  if ((sqb | sqh | sqt | skb | skh | sks) % vec)
    return set_error("forge_attn_decode: q/cache strides must be multiples of 16 bytes");
  if (max_len <= 0 || max_len >= (1LL << 30)) return set_error("cache length must be in [1, 2^30)");
  const int64_t esize = dtype == FORGE_F32 ? 4 : 2;
  if (sks * (max_len + 1) * esize >= (1LL << 31))
    return set_error("forge_attn_decode: one (batch, kv head) slab of the cache must span < 2^31 bytes");
  if (max_kv_len <= 0 || max_kv_len > max_len) max_kv_len = max_len;
  if (!row_pos && !pos_dev && (pos0 < 0 || pos0 + T > max_len))
    return set_error("KV cache full: pos + T exceeds the cache length");
  if (!row_pos && !pos_dev && pos0 + T > max_kv_len) max_kv_len = pos0 + T;
  if (window < 0) return set_error("window must be >= 0");
  const bool mfma_path = use_verify_mfma(dtype, D, H / K);
  const int kpi = mfma_path ? 32 : keys_per_iter(dtype, D);
  if (chunk <= 0) chunk = auto_chunk(dtype, B, T, H, K, D, chunk_span(max_kv_len, window));
  if (chunk % kpi) return set_error("chunk must be a multiple of the keys per block iteration");

  p = SplitParams{};
  p.q = q;
  p.sqb = sqb;
  p.sqh = sqh;
  p.sqt = sqt;
  p.qw = q_weight;
  p.eps = eps;
  p.flags = flags;
  p.cos = cos;
  p.sin = sin;
  p.csb = s_cos_b;
  p.cst = s_cos_t;
  p.kc = k_cache;
  p.vc = v_cache;
  p.skb = skb;
  p.skh = skh;
  p.sks = sks;
  p.max_len = max_len;
  p.row_pos = row_pos;
  p.pos_dev = pos_dev;
  p.pos0 = pos0;
  p.B = B;
  p.T = T;
  p.H = H;
  p.K = K;
  p.G = H / K;
  p.rows_total = p.G * T;
  p.window = window;
  p.scale_log2 = scale * kLog2e;
  p.chunk = chunk;
  p.max_chunks = (int)((max_kv_len + chunk - 1) / chunk);
  p.out = out;
  p.sob = sob;
  p.sot = sot;
  p.soh = soh;
  p.vec_tables = ((uintptr_t)q_weight | (uintptr_t)cos | (uintptr_t)sin) % 16 == 0 &&
                 (cos == nullptr || (s_cos_b % 4 == 0 && s_cos_t % 4 == 0));
  // the MFMA verify kernel DMAs q rows (offsets from the batch row's start) and table rows
  // (from the unit's first token's row) with 32-bit byte offsets
  const int64_t q_span = ((int64_t)(H - 1) * sqh + (int64_t)(T - 1) * sqt + D) * esize;
  const int64_t tab_span = cos ? ((int64_t)T * s_cos_t + D) * 4 : 0;
  p.small_dma = p.vec_tables && q_span < (1LL << 31) && tab_span < (1LL << 31);
  return 0;
}

// Workspace bytes the call set up in p needs (0: one chunk per row, no partials).
size_t decode_need(const SplitParams& p, int D) {
  return p.max_chunks > 1 ? workspace_for((int64_t)p.B * p.H * p.T * p.max_chunks, D) : 0;
}

// Points p's work ticket and partials into `ws` (at least decode_need bytes). The ticket sits
// at offset 0 for every shape, so a workspace reused by calls of different shapes keeps it
// in one place (the combine kernel leaves it zero: FORGE_WS_ZEROED).
void decode_bind(SplitParams& p, int D, void* ws) {
  if (p.max_chunks < 2) return;
  const int64_t slots = (int64_t)p.B * p.H * p.T * p.max_chunks;
  const size_t ml = ((size_t)slots * sizeof(float2) + 255) / 256 * 256;
  p.ws_ctr = static_cast<int*>(ws);
  p.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + 256);
  p.ws_o = reinterpret_cast<float*>(static_cast<char*>(ws) + 256 + ml);
}

int decode_launch(const SplitParams& p, int dtype, int D, hipStream_t s) {
  if (use_verify_mfma(dtype, D, p.G))
    return dtype == FORGE_BF16 ? launch_verify<bf16>(p, D, s) : launch_verify<f16>(p, D, s);
  const int rows = rows_per_block(p.rows_total, D);
  switch (dtype) {
    case FORGE_F32: return launch_split<float>(p, D, rows, s);
    case FORGE_BF16: return launch_split<bf16>(p, D, rows, s);
    default: return launch_split<f16>(p, D, rows, s);
  }
}

}  // namespace

extern "C" int forge_attn_decode(int dtype, int B, int T, int H, int K, int D, const void* q,
                                 int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                                 float eps, int flags, const float* cos, const float* sin,
                                 int64_t s_cos_b, int64_t s_cos_t, const void* k_cache,
                                 const void* v_cache, int64_t skb, int64_t skh, int64_t sks,
                                 int64_t max_len, const int32_t* row_pos, const int64_t* pos_dev,
                                 int64_t pos0, int64_t max_kv_len, int window, float scale,
                                 int chunk, void* out, int64_t sob, int64_t sot, int64_t soh,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SplitParams p;
  const int st = decode_setup(p, dtype, B, T, H, K, D, q, sqb, sqh, sqt, q_weight, eps, flags, cos,
                              sin, s_cos_b, s_cos_t, k_cache, v_cache, skb, skh, sks, max_len,
                              row_pos, pos_dev, pos0, max_kv_len, window, scale, chunk, out, sob,
                              sot, soh);
  if (st) return st;
  const size_t need = decode_need(p, D);
  if (need && (!workspace || workspace_bytes < need)) return set_error("workspace too small");
  decode_bind(p, D, workspace);
  return decode_launch(p, dtype, D, (hipStream_t)stream);
}

// ---------------------------------------------------------------- decode with the cache write
extern "C" int forge_attn_decode_append(
    int dtype, int B, int T, int H, int K, int D, const void* q, int64_t sqb, int64_t sqh,
    int64_t sqt, const float* q_weight, float eps, int flags, const void* k, int64_t sknb,
    int64_t sknh, int64_t sknt, const void* v, int64_t svnb, int64_t svnh, int64_t svnt,
    const float* k_weight, int kv_flags, const float* cos, const float* sin, int64_t s_cos_b,
    int64_t s_cos_t, void* k_cache, void* v_cache, int64_t skb, int64_t skh, int64_t sks,
    int64_t max_len, const int32_t* row_pos, const int64_t* pos_dev, int64_t pos0,
    int64_t max_kv_len, int window, float scale, int chunk, void* out, int64_t sob, int64_t sot,
    int64_t soh, void* workspace, size_t workspace_bytes, int ws_flags, void* stream) {
  clear_error();
  SplitParams p;
  int st = decode_setup(p, dtype, B, T, H, K, D, q, sqb, sqh, sqt, q_weight, eps, flags, cos, sin,
                        s_cos_b, s_cos_t, k_cache, v_cache, skb, skh, sks, max_len, row_pos,
                        pos_dev, pos0, max_kv_len, window, scale, chunk, out, sob, sot, soh);
  if (st) return st;
  if (!k || !v) return set_error("forge_attn_decode_append: null k or v");
  if ((kv_flags & FORGE_ROPE) && (!cos || !sin)) return set_error("FORGE_ROPE needs cos and sin");
  const int vec = vec_of(dtype);
  const size_t need = decode_need(p, D);
  if (need && (!workspace || workspace_bytes < need)) return set_error("workspace too small");
  // In the attention kernel when one row block holds a KV head's G*T query rows (one unit
  // per chunk reads the new rows; on the split-K path a lane group also holds at most
  // kNewPerLane new keys) and the rows allow 16-byte slices; otherwise forge_kv_append's
  // kernel runs first.
  const int groups = kSplitThreads / (D / vec);
  const bool one_block = use_verify_mfma(dtype, D, p.G)
                             ? p.rows_total <= kVerifyRows
                             : T <= kNewPerLane * groups && rows_per_block(p.rows_total, D) >= p.rows_total;
  const bool fused = one_block &&
                     ((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_weight | (uintptr_t)cos | (uintptr_t)sin) % 16 == 0 &&
                     (sknb | sknh | sknt | svnb | svnh | svnt) % vec == 0;
  if (!fused) {
    st = forge_kv_append(dtype, B, T, K, D, k, sknb, sknh, sknt, v, svnb, svnh, svnt, k_cache, v_cache,
                         skb, skh, sks, max_len, row_pos, pos_dev, pos0, k_weight, eps, kv_flags, cos,
                         sin, s_cos_b, s_cos_t, stream);
    if (st) return st;
  } else {
    p.kn = k;
    p.vn = v;
    p.sknb = sknb;
    p.sknh = sknh;
    p.sknt = sknt;
    p.svnb = svnb;
    p.svnh = svnh;
    p.svnt = svnt;
    p.kw = k_weight;
    p.kvflags = kv_flags;
    p.kcw = k_cache;
    p.vcw = v_cache;
  }
  decode_bind(p, D, workspace);
  p.ws_zeroed = (ws_flags & FORGE_WS_ZEROED) ? 1 : 0;
  return decode_launch(p, dtype, D, (hipStream_t)stream);
}

// ---------------------------------------------------------------- allocation-free entry point
// For callers that cannot allocate device memory (code under graph capture that may not call
// hipMalloc, tight serving loops): the split-K partials and the work ticket live in this
// file-scope device array instead of a caller-provided workspace. Every device that loads the
// library holds its own copy until the process ends. Host code never uses the array's name as
// an address: its device address is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address goes to the kernels. All calls on one device share the
// array, so calls that overlap on one device (different streams, no ordering) race on it.
static __device__ __align__(256) unsigned char scratch[FORGE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, looked up on first use there.
void* scratch_address() {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    addr[dev] = ptr;
  }
  return addr[dev];
}

}  // namespace

extern "C" int forge_attn_decode_noalloc(int dtype, int B, int T, int H, int K, int D,
                                         const void* q, int64_t sqb, int64_t sqh, int64_t sqt,
                                         const float* q_weight, float eps, int flags,
                                         const float* cos, const float* sin, int64_t s_cos_b,
                                         int64_t s_cos_t, const void* k_cache,
                                         const void* v_cache, int64_t skb, int64_t skh,
                                         int64_t sks, int64_t max_len, const int32_t* row_pos,
                                         const int64_t* pos_dev, int64_t pos0,
                                         int64_t max_kv_len, int window, float scale, int chunk,
                                         void* out, int64_t sob, int64_t sot, int64_t soh,
                                         void* stream) {
  clear_error();
  SplitParams p;
  const int st = decode_setup(p, dtype, B, T, H, K, D, q, sqb, sqh, sqt, q_weight, eps, flags, cos,
                              sin, s_cos_b, s_cos_t, k_cache, v_cache, skb, skh, sks, max_len,
                              row_pos, pos_dev, pos0, max_kv_len, window, scale, chunk, out, sob,
                              sot, soh);
  if (st) return st;
  const size_t need = decode_need(p, D);
  if (need > (size_t)FORGE_NOALLOC_SCRATCH_BYTES) {
    char msg[200];
    snprintf(msg, sizeof msg,
             "forge_attn_decode_noalloc: this call needs %zu bytes of split-K scratch, more than "
             "the %d the library holds (use forge_attn_decode with a workspace, or a larger chunk)",
             need, FORGE_NOALLOC_SCRATCH_BYTES);
    return set_error(msg);
  }
  if (need) {
    void* ws = scratch_address();
    if (!ws) return set_error("forge_attn_decode_noalloc: cannot find the scratch array on this device");
    decode_bind(p, D, ws);   // the work ticket is zeroed by a kernel before the launch that uses it
  }
  return decode_launch(p, dtype, D, (hipStream_t)stream);
}
