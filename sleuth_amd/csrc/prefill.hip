// Causal prefill on bf16/fp16 MFMA (gfx950 v_mfma_f32_32x32x16_{bf16,f16}).
//
// A block of 4 waves owns BM = 128 queries of one (b, head); each wave owns 32 of them
// and keeps them for the whole block, together with its output accumulator. Key tiles
// of BN keys (64 for head dim <= 128, 32 for 256) stream through LDS:
//
//   * K and V tiles go from HBM straight into LDS with global_load_lds_dwordx4 (no
//     staging registers, no VALU). Each lane's 16 bytes land at LDS slot `lane`, so the
//     16-byte chunk a lane fetches decides the LDS layout: chunk c of key row r is stored
//     at chunk position c ^ swz(r), an XOR swizzle that keeps the MFMA operand reads
//     below free of bank conflicts. LDS stages (two for every head dim today): the loads
//     of tile j+1 are issued before tile j is computed, one barrier per tile separates
//     the stages, and two blocks share a CU so that its SIMDs interleave two independent
//     waves.
//   * Scores are computed transposed, S^T = K . Q^T: K is the MFMA A operand (128-bit
//     LDS reads), Q^T the B operand held in registers for the whole block. In the 32x32
//     accumulator layout each lane then owns ONE query (column l % 32) and 16 keys of a
//     32-key block (rows 8i + 4(l/32) + j), so the online softmax of a query needs a
//     single cross-lane exchange per tile (lane l <-> l ^ 32) for the running max, and
//     none for the running sum (the two halves are added once at the end).
//   * P^T is fed to the second MFMA (O^T = V^T . P^T) straight from the score registers:
//     MFMA k index 8hi + 4i' + j stands for key 16*half + 8i' + 4hi + j, exactly the keys
//     the lane already holds. The matching V^T operand is read from the row-major V tile
//     with ds_read_b64_tr_b16 (gfx950's transposing LDS read: within each 16-lane group,
//     lane i receives element i % 4 of the 4-element rows addressed by lanes 4k + i / 4,
//     k = 0..3), two reads of 4 keys per MFMA.
//   * The running max only moves when a score exceeds it by 2^8 (log2 units), so the
//     rescale of the accumulator is rare; weights stay <= 2^8, safe in bf16/fp16.
//
// Q gets the per-head RMSNorm and RoPE in its load (fp32 math, one rounding), like
// fused_ops._head_kernel (fused_ops.py:53-85); K and V come from the cache, where
// forge_kv_append wrote them already normalised.
#include "common.h"
#include "forge_internal.h"

namespace forge {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ floatx16 run(vec a, vec b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ floatx16 run(vec a, vec b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

struct PrefillParams {
  const void* q;
  int64_t sqb, sqh, sqt;
  const float* qw;
  float eps;
  int flags;
  const float* cos;
  const float* sin;
  int64_t cst;
  const void* k;
  const void* v;
  int64_t skb, skh, sks;
  int64_t offset;
  int B, T, H, K, G;
  int nqt;       // query tiles per (b, head)
  int xcd_map;   // 1: blocks of one (b, kv head) pair run on one XCD (B*K % 8 == 0)
  int window;
  float scale_log2;
  void* out;
  int64_t sob, sot, soh;
  // Document masking (forge_attn_prefill_docs): query t of row b also sees no key before
  // position doc_lo[b * sdb + t], the first of its document (non-decreasing in t); or null.
  const int32_t* doc_lo;
  int64_t sdb;
};

constexpr float kLazyLog2 = 8.0f;

// Block shape per head dim: WAVES waves of 32 queries each, STAGES LDS stages of one K
// and one V tile of BN keys (loads run STAGES - 1 tiles ahead of the compute).
template <int D> struct Tile {
  static constexpr int WAVES = 4;
  static constexpr int STAGES = 2;
  static constexpr int BM = 32 * WAVES;                // queries per block
  static constexpr int BN = D >= 256 ? 32 : 64;        // keys per tile
  static constexpr int NCH = D / 8;                    // 16-byte chunks per key row
  static constexpr int ROWB = 2 * D;                   // bytes per key row
  static constexpr int TILEB = BN * ROWB;              // bytes of one K (or V) tile
  static constexpr int LOADS = TILEB / (WAVES * 1024);   // 16-byte loads per lane per tile
  static constexpr int LDS_BYTES = STAGES * 2 * TILEB;
  static_assert(LOADS * WAVES * 1024 == TILEB, "tile must split into whole wave loads");
};

// XOR swizzles of the 16-byte chunk index by key row (see the reads below).
template <int D> __device__ __forceinline__ int swz_k(int row) {
  return row & ((D / 8 >= 16 ? 16 : D / 8) - 1);
}
template <int D> __device__ __forceinline__ int swz_v(int row) {
  return D / 8 >= 16 ? (row & 3) << 2 : ((row >> 1) & 1) << 2;
}

// Wait until at most N vector-memory loads of this wave are outstanding (loads retire in
// issue order, so everything issued before the last N has landed).
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N == 0 || N == 2 || N == 4 || N == 8, "add the count");
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}

// Q rows of one wave as MFMA B operands: load, fused RMSNorm + RoPE (fp32, one rounding).
// Lane (n, hi) holds channels 16s + 8hi + e of query i_q; gains and RoPE rows come in
// 16-byte loads.
template <typename T, int D>
__device__ __forceinline__ void load_q(const PrefillParams& p, int b, int h, int i_q, bool valid_q,
                                       int hi, typename Mfma<T>::vec (&qreg)[D / 16]) {
  constexpr int KSTEPS = D / 16;
  float qf[KSTEPS][8];
  const T* src = static_cast<const T*>(p.q) + b * p.sqb + h * p.sqh + (int64_t)i_q * p.sqt;
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    if (valid_q) {
      unpack16<T>(load16(src + 16 * s + 8 * hi), qf[s]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = 0.0f;
    }
  }
  if (p.flags & FORGE_NORM_QK) {
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += qf[s][e] * qf[s][e];
    ss += __shfl_xor(ss, 32, kWave);
    const float rs = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] *= rs;
    if (p.qw) {
      float w[KSTEPS][8];
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) load_f32x8(p.qw + 16 * s + 8 * hi, w[s]);
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[s][e] *= w[s][e];
    }
  }
  if ((p.flags & FORGE_ROPE) && valid_q) {
    const float* cr = p.cos + (int64_t)i_q * p.cst;
    const float* sr = p.sin + (int64_t)i_q * p.cst;
#pragma unroll
    for (int s = 0; s < KSTEPS / 2; ++s) {
      const int x = 16 * s + 8 * hi;  // first-half channels x..x+7; partners x + D/2
      float c1[8], s1[8], c2[8], s2[8];
      load_f32x8(cr + x, c1);
      load_f32x8(sr + x, s1);
      load_f32x8(cr + x + D / 2, c2);
      load_f32x8(sr + x + D / 2, s2);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = qf[s][e], z = qf[s + KSTEPS / 2][e];
        qf[s][e] = a * c1[e] - z * s1[e];
        qf[s + KSTEPS / 2][e] = z * c2[e] + a * s2[e];
      }
    }
  }
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) qreg[s][e] = from_f32<T>(qf[s][e]);
}

template <typename T, int D>
__global__ __launch_bounds__(Tile<D>::WAVES * 64) __attribute__((amdgpu_waves_per_eu(D >= 256 ? 1 : 2)))
void prefill_kernel(PrefillParams p) {
  using V8 = typename Mfma<T>::vec;
  using TL = Tile<D>;
  constexpr int BN = TL::BN;
  constexpr int kBM = TL::BM;
  constexpr int KB = BN / 32;       // 32-key blocks per tile
  constexpr int KSTEPS = D / 16;    // MFMA k-steps over the head dim (scores)
  constexpr int DB = D / 32;        // 32-channel blocks of the output
  constexpr int HALVES = BN / 16;   // 16-key MFMA steps of P.V

  extern __shared__ __attribute__((aligned(1024))) char smem[];  // [stage][K|V][TILEB]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int n = lane & 31;
  const int hi = lane >> 5;

  // ---- block -> (query tile, head, batch). Heavy (late) causal tiles first. With
  // xcd_map, block i runs on XCD i % 8 and all blocks of one (b, kv head) pair share an
  // XCD, so the K/V they all read stays in that XCD's L2.
  int qt, b, kvh, gq;
  {
    const int bid = blockIdx.x;
    const int P = p.B * p.K;
    if (p.xcd_map) {
      const int x = bid & 7, local = bid >> 3;
      const int per = (P >> 3) * p.G;  // (pair, head) combinations per XCD
      const int rank = local / per, rest = local % per;
      qt = p.nqt - 1 - rank;
      const int pair = (rest / p.G) * 8 + x;
      gq = rest % p.G;
      b = pair / p.K;
      kvh = pair % p.K;
    } else {
      const int HB = p.H * p.B;
      qt = p.nqt - 1 - bid / HB;
      const int hb = bid % HB;
      const int pair = hb % P;
      gq = hb / P;
      b = pair / p.K;
      kvh = pair % p.K;
    }
  }
  const int h = kvh * p.G + gq;

  const int i_q = qt * kBM + wave * 32 + n;  // this lane's query (index into T)
  const bool valid_q = i_q < p.T;
  const int64_t qpos = p.offset + i_q;
  const int64_t S = p.offset + p.T;

  // ---- key tiles of the block, and the first stage's loads (issued before the Q math)
  const int64_t q_first = p.offset + (int64_t)qt * kBM;
  const int64_t q_last_idx =
      (int64_t)qt * kBM + kBM - 1 < p.T - 1 ? (int64_t)qt * kBM + kBM - 1 : p.T - 1;
  const int64_t blk_kmax = p.offset + q_last_idx;
  int64_t blk_kmin = p.window > 0 ? q_first - p.window + 1 : 0;
  if (blk_kmin < 0) blk_kmin = 0;
  // with documents: the block's first query starts the earliest document of the block
  const int32_t* dl = p.doc_lo ? p.doc_lo + b * p.sdb : nullptr;
  if (dl) {
    const int64_t d0 = __builtin_amdgcn_readfirstlane(dl[(int64_t)qt * kBM]);
    if (d0 > blk_kmin) blk_kmin = d0;
  }
  const int kt_begin = (int)(blk_kmin / BN);
  const int kt_end = (int)(blk_kmax / BN);

  const T* kg = static_cast<const T*>(p.k) + b * p.skb + kvh * p.skh;
  const T* vg = static_cast<const T*>(p.v) + b * p.skb + kvh * p.skh;

  // Per-lane source byte offsets of the direct loads within a tile: load i of this wave
  // fills LDS slots (wave*LOADS + i)*64 + lane, i.e. key row slot / NCH and swizzled
  // chunk slot % NCH. The tile base is wave-uniform (scalar registers).
  int ld_koff[TL::LOADS], ld_voff[TL::LOADS];
#pragma unroll
  for (int i = 0; i < TL::LOADS; ++i) {
    const int slot = (wave * TL::LOADS + i) * 64 + lane;
    const int row = slot / TL::NCH, pch = slot % TL::NCH;
    ld_koff[i] = (int)(row * p.sks * 2) + (pch ^ swz_k<D>(row)) * 16;
    ld_voff[i] = (int)(row * p.sks * 2) + (pch ^ swz_v<D>(row)) * 16;
  }
  const char* kgb = reinterpret_cast<const char*>(kg);
  const char* vgb = reinterpret_cast<const char*>(vg);
  // The loads are issued from inline asm (lds_dma16), so the compiler does not hold the
  // LDS reads of the current stage back until the next stage's loads have landed; the
  // loop waits for them itself (wait_vm before the barrier).
  auto issue = [&](int kt, int stage) {
    const int64_t key0 = (int64_t)kt * BN;
    const char* kt_base = kgb + key0 * p.sks * 2;
    const char* vt_base = vgb + key0 * p.sks * 2;
    const unsigned kdst = lds_offset(smem + (2 * stage) * TL::TILEB + wave * TL::LOADS * 1024);
    const unsigned vdst = kdst + TL::TILEB;
    if (key0 + BN <= S) {
#pragma unroll
      for (int i = 0; i < TL::LOADS; ++i) {
        lds_dma16(kt_base, (unsigned)ld_koff[i], kdst + i * 1024);
        lds_dma16(vt_base, (unsigned)ld_voff[i], vdst + i * 1024);
      }
    } else {
      // last, partial tile: rows past the end are masked; they read row S - 1 instead
#pragma unroll
      for (int i = 0; i < TL::LOADS; ++i) {
        const int slot = (wave * TL::LOADS + i) * 64 + lane;
        const int row = slot / TL::NCH, pch = slot % TL::NCH;
        const int64_t key = key0 + row < S ? key0 + row : S - 1;
        const unsigned rb = (unsigned)((key - key0) * p.sks * 2);
        lds_dma16(kt_base, rb + (pch ^ swz_k<D>(row)) * 16, kdst + i * 1024);
        lds_dma16(vt_base, rb + (pch ^ swz_v<D>(row)) * 16, vdst + i * 1024);
      }
    }
  };
  issue(kt_begin, 0);
#pragma unroll
  for (int j = 1; j < TL::STAGES - 1; ++j)
    if (kt_begin + j <= kt_end) issue(kt_begin + j, j);

  // ---- Q: load, fused RMSNorm + RoPE, one rounding, kept as MFMA B operands.
  V8 qreg[KSTEPS];
  load_q<T, D>(p, b, h, i_q, valid_q, hi, qreg);

  // this wave's query span (tile skipping and the mask-free fast path); positions fit
  // in 32 bits (host check)
  const int w_first = qt * kBM + wave * 32;
  const int w_last = w_first + 31 < p.T - 1 ? w_first + 31 : p.T - 1;
  const bool wave_any = w_first < p.T;
  const int off = (int)p.offset;
  const int wq_lo = off + w_first, wq_hi = off + w_last;
  const int S32 = (int)S;
  const int qpos32 = (int)qpos;
  // document starts: this lane's query's, and the first (smallest) and last (largest) of the
  // wave's queries (loads of rows past T read row T - 1; those lanes are masked anyway)
  int d_lane = 0, d_wfirst = 0, d_wlast = 0;
  if (dl) {
    d_lane = dl[i_q < p.T ? i_q : p.T - 1];
    d_wfirst = __builtin_amdgcn_readfirstlane(d_lane);
    d_wlast = __builtin_amdgcn_readlane(d_lane, w_last - w_first > 0 ? w_last - w_first : 0);
  }

  // LDS read offsets (bytes within a stage buffer).
  // K operand: row 32kb + n, chunk 2s + hi, swizzled by row & 15 == n & 15.
  const int k_rd = n * TL::ROWB;
  const int k_sw = swz_k<D>(n);
  // V^T operand (tr reads): source lane role g = lane/16, kq = (lane/4)%4, qq = lane%4
  // addresses key row 16*half + 8i' + 4(g/2) + kq, channel 32db + 16(g%2) + 4qq.
  const int g = lane >> 4, kq = (lane >> 2) & 3, qq = lane & 3;
  const int v_row = 4 * (g >> 1) + kq;
  const int v_sw = swz_v<D>(v_row);  // rows differ from v_row by multiples of 8: same swizzle
  const int v_chlo = 2 * (g & 1) + (qq >> 1);  // chunk within the 32-channel block (0..3)
  const int v_byte = 8 * (qq & 1);

  floatx16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.0f;
  float m_run = kNegInf, l_run = 0.0f;
  const float c = p.scale_log2;

  for (int kt = kt_begin; kt <= kt_end; ++kt) {
    const int idx = kt - kt_begin;
    const int stage = idx % TL::STAGES;
    // Tile kt has landed once at most the loads of the tiles issued after it remain.
    if (TL::STAGES == 3 && kt + 1 <= kt_end) wait_vm<2 * TL::LOADS>();
    else wait_vm<0>();
    __syncthreads();  // tile kt is in LDS for every wave; the stage of tile kt-1 is free
    if (kt + TL::STAGES - 1 <= kt_end) issue(kt + TL::STAGES - 1, (idx + TL::STAGES - 1) % TL::STAGES);

    const int key0 = kt * BN;
    const bool wave_needs = wave_any && key0 <= wq_hi &&
                            (p.window <= 0 || key0 + BN - 1 > wq_lo - p.window) &&
                            key0 + BN - 1 >= d_wfirst;
    if (!wave_needs) continue;
    const bool full = key0 + BN - 1 <= wq_lo && key0 + BN - 1 < S32 &&
                      (p.window <= 0 || wq_hi - key0 < p.window) && w_last - w_first == 31 &&
                      key0 >= d_wlast;

    const char* kl = smem + (2 * stage) * TL::TILEB + k_rd;
    const char* vl = smem + (2 * stage + 1) * TL::TILEB;

    // ---- S^T = K . Q^T: KB independent accumulation chains. The K operands of step
    // st + 2 are read before the MFMAs of step st are issued (three register sets), so
    // the LDS latency hides under two steps of MFMAs; the scheduling groups pin that
    // order (left alone, the compiler reuses one register set and waits for every read).
    floatx16 sacc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) sacc[kb][x] = 0.0f;
    {
      auto kread = [&](int kb, int st) {
        return *reinterpret_cast<const V8*>(kl + kb * 32 * TL::ROWB + (((2 * st + hi) ^ k_sw) << 4));
      };
      V8 a0[KB], a1[KB], a2[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) a0[kb] = kread(kb, 0);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) a1[kb] = kread(kb, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * KB, 0);
#pragma unroll
      for (int st = 0; st < KSTEPS; ++st) {
        if (st + 2 < KSTEPS) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) a2[kb] = kread(kb, st + 2);
          __builtin_amdgcn_sched_group_barrier(0x100, KB, 0);
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sacc[kb] = Mfma<T>::run(a0[kb], qreg[st], sacc[kb]);
        __builtin_amdgcn_sched_group_barrier(0x008, KB, 0);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          a0[kb] = a1[kb];
          a1[kb] = a2[kb];
        }
      }
    }

    // ---- mask (boundary tiles only): element (kb, x) of this lane is key
    // key0 + 4hi + ce with ce = 32kb + 8(x/4) + x%4; it is visible iff lo <= ce <= hi.
    if (!full) {
      const int base = key0 + 4 * hi;
      const int top = (qpos32 < S32 - 1 ? qpos32 : S32 - 1) - base;
      const int lim_hi = valid_q ? top : -1;
      int lim_lo = p.window > 0 ? qpos32 - p.window + 1 - base : -(1 << 30);
      if (dl && d_lane - base > lim_lo) lim_lo = d_lane - base;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int ce = 32 * kb + 8 * (x >> 2) + (x & 3);
          sacc[kb][x] = (ce <= lim_hi && ce >= lim_lo) ? sacc[kb][x] : kNegInf;
        }
    }

    // ---- online softmax (base 2, scale folded into the exponent)
    float mxp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mxp[i] = sacc[0][4 * i];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = (kb == 0 ? 1 : 0); j < 4; ++j) mxp[i] = fmaxf(mxp[i], sacc[kb][4 * i + j]);
    }
    float mx = fmaxf(fmaxf(mxp[0], mxp[1]), fmaxf(mxp[2], mxp[3]));
    mx = max_xor32(mx);
    const float mxc = mx * c;
    if (mxc > m_run + kLazyLog2) {
      const float alpha = m_run == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m_run - mxc);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[d][x] *= alpha;
      m_run = mxc;
    }
    const float neg_m = m_run == kNegInf ? 0.0f : -m_run;  // all -inf so far: weights 0
    float rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[kb][x], c, neg_m));
        sacc[kb][x] = pv;
        rs[x & 3] += pv;
      }
    l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);

    // ---- O^T += V^T . P^T
#pragma unroll
    for (int hf = 0; hf < HALVES; ++hf) {
      const int kb = hf >> 1, half = hf & 1;
      V8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = from_f32<T>(sacc[kb][8 * half + e]);
      const char* vrow0 = vl + (16 * hf + v_row) * TL::ROWB + v_byte;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const int ch = ((4 * d + v_chlo) ^ v_sw) << 4;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vrow0 + ch));
        const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vrow0 + 8 * TL::ROWB + ch));
        typedef short i16x8 __attribute__((ext_vector_type(8)));
        const i16x8 av = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[d] = Mfma<T>::run(__builtin_bit_cast(V8, av), pb, oacc[d]);
      }
    }
  }

  l_run += __shfl_xor(l_run, 32, kWave);
  if (!valid_q) return;
  const float inv_l = 1.0f / l_run;
  T* dst = static_cast<T*>(p.out) + b * p.sob + (int64_t)i_q * p.sot + h * p.soh;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T vals[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vals[j] = from_f32<T>(oacc[d][4 * i + j] * inv_l);
      *reinterpret_cast<uint2*>(dst + d * 32 + 8 * i + 4 * hi) = *reinterpret_cast<uint2*>(vals);
    }
}

template <typename T, int D>
static int launch_prefill_d(PrefillParams p, hipStream_t s) {
  using TL = Tile<D>;
  static bool attr_set = false;  // raise the dynamic LDS limit once per kernel
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<T, D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, TL::LDS_BYTES) != hipSuccess)
      return set_error("forge_attn_prefill: cannot reserve the LDS the kernel needs");
    attr_set = true;
  }
  p.nqt = (p.T + TL::BM - 1) / TL::BM;
  if ((int64_t)p.nqt * p.H * p.B > 0x7fffffff) return set_error("grid too large");
  const dim3 grid((unsigned)((int64_t)p.nqt * p.H * p.B));
  hipLaunchKernelGGL((prefill_kernel<T, D>), grid, dim3(TL::WAVES * 64), TL::LDS_BYTES, s, p);
  return check_launch();
}

// ---------------------------------------------------------------- head dim 512
// Head dim 512 (Gemma 4's full-attention layers: 1 KV head of 512, reference
// kv_cache.py:12-13). A wave's 32 queries would need 128 registers of Q^T and 256 of output
// accumulators, so here the head dim is split over the block instead: a block of 4 waves
// owns 32 queries of one (b, head), and wave w holds channels 128w .. 128w + 127 of Q^T and
// of the output. Per key tile (32 keys, two LDS stages of 32 KB K + 32 KB V):
//   * each wave computes the partial scores of its channels, S_w^T = K[:, slice] . Q^T[slice]
//     (8 MFMAs), and stores them in LDS; after a barrier every wave adds the four partials
//     in the same order (waves 0..3), so all waves hold identical scores;
//   * every wave runs the same online softmax (the running max and sum are identical in
//     all waves) and accumulates its own 128 output channels, O^T += V^T[slice] . P^T
//     (8 MFMAs).
// The q RMSNorm sums the squares of the four slices through LDS in the same order; RoPE
// pairs channel c with c ^ 256, so each lane also loads its channels' partners.
struct WideTile {
  static constexpr int D = 512;
  static constexpr int WAVES = 4;
  static constexpr int BM = 32;                          // queries per block
  static constexpr int BN = 32;                          // keys per tile
  static constexpr int NCH = D / 8;
  static constexpr int ROWB = 2 * D;
  static constexpr int TILEB = BN * ROWB;                // 32 KB
  static constexpr int LOADS = TILEB / (WAVES * 1024);   // 8
  static constexpr int STAGES = 2;
  static constexpr int PART_BYTES = WAVES * 64 * 16 * 4; // the waves' partial scores
  static constexpr int SS_BYTES = WAVES * 32 * 4;        // the q slices' sums of squares
  static constexpr int LDS_BYTES = STAGES * 2 * TILEB + PART_BYTES + SS_BYTES;
};

template <typename T, int SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void prefill_wide_kernel(PrefillParams p) {
  using V8 = typename Mfma<T>::vec;
  using TL = WideTile;
  constexpr int D = TL::D;
  constexpr int BN = TL::BN;
  // SPLIT waves share a head, each with D / SPLIT channels; the block takes WAVES / SPLIT heads
  // of one KV head, so each K/V tile is loaded once for all of them
  static_assert(SPLIT == 4 || SPLIT == 2, "four quarter-slices of one head, or two halves of two");
  constexpr int HPB = TL::WAVES / SPLIT;     // heads per block
  constexpr int CW = D / SPLIT;              // channels per wave
  constexpr int CCH = CW / 8;                // 16-byte chunks per wave slice
  constexpr int KSTEPS = CW / 16;            // 16-channel MFMA k-steps over a wave's channels
  constexpr int DB = CW / 32;                // 32-channel output blocks per wave
  constexpr int HALVES = BN / 16;

  extern __shared__ __attribute__((aligned(1024))) char smem[];
  float* part = reinterpret_cast<float*>(smem + TL::STAGES * 2 * TL::TILEB);   // [wave][lane][16]
  float* sh_ss = part + TL::WAVES * 64 * 16;                                     // [wave][32]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int n = lane & 31;
  const int hi = lane >> 5;

  // block -> (query tile, head group, batch), heavy (late) causal tiles first; wave w takes
  // slice w % SPLIT of head HPB * hg + w / SPLIT
  const int HB = (p.H / HPB) * p.B;
  const int qt = p.nqt - 1 - (int)blockIdx.x / HB;
  const int hb = (int)blockIdx.x % HB;
  const int b = hb % p.B;
  const int slice = wave % SPLIT;
  const int h = (hb / p.B) * HPB + wave / SPLIT;
  const int kvh = h / p.G;
  const int wbase = wave - slice;  // the head's first wave

  const int i_q = qt * TL::BM + n;
  const bool valid_q = i_q < p.T;
  const int64_t S = p.offset + p.T;
  const int64_t q_first = p.offset + (int64_t)qt * TL::BM;
  const int q_last_idx = qt * TL::BM + TL::BM - 1 < p.T - 1 ? qt * TL::BM + TL::BM - 1 : p.T - 1;
  const int64_t blk_kmax = p.offset + q_last_idx;
  int64_t blk_kmin = p.window > 0 ? q_first - p.window + 1 : 0;
  if (blk_kmin < 0) blk_kmin = 0;
  const int32_t* dl = p.doc_lo ? p.doc_lo + b * p.sdb : nullptr;
  int d_lane = 0, d_first = 0, d_last = 0;
  if (dl) {
    d_lane = dl[i_q < p.T ? i_q : p.T - 1];
    d_first = __builtin_amdgcn_readfirstlane(d_lane);
    d_last = __builtin_amdgcn_readlane(d_lane, q_last_idx - qt * TL::BM);
    if (d_first > blk_kmin) blk_kmin = d_first;
  }
  const int kt_begin = (int)(blk_kmin / BN);
  const int kt_end = (int)(blk_kmax / BN);

  const char* kgb = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + b * p.skb + kvh * p.skh);
  const char* vgb = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + b * p.skb + kvh * p.skh);
  auto issue = [&](int kt, int stage) {
    const int64_t key0 = (int64_t)kt * BN;
    const char* kt_base = kgb + key0 * p.sks * 2;
    const char* vt_base = vgb + key0 * p.sks * 2;
    const unsigned kdst = lds_offset(smem + (2 * stage) * TL::TILEB + wave * TL::LOADS * 1024);
#pragma unroll
    for (int i = 0; i < TL::LOADS; ++i) {
      const int slot = (wave * TL::LOADS + i) * 64 + lane;
      const int row = slot / TL::NCH, pch = slot % TL::NCH;
      const int64_t key = key0 + row < S ? key0 + row : S - 1;   // rows past the end are masked
      const unsigned rb = (unsigned)((key - key0) * p.sks * 2);
      lds_dma16(kt_base, rb + (pch ^ swz_k<D>(row)) * 16, kdst + i * 1024);
      lds_dma16(vt_base, rb + (pch ^ swz_v<D>(row)) * 16, kdst + TL::TILEB + i * 1024);
    }
  };
  issue(kt_begin, 0);

  // ---- Q^T slice: channels CW slice + 16 s + 8 hi + e, RMSNorm over all 512 channels
  // (slice sums added through LDS in slice order), RoPE with the partner c ^ 256.
  V8 qreg[KSTEPS];
  {
    const int c0 = CW * slice + 8 * hi;
    const int pc0 = (CW * slice + 8 * hi) ^ 256;   // partner channels
    // raw slices stay packed (16 bf16/fp16 values per k-step in 8 registers); each k-step is
    // unpacked, normalised, rotated and rounded in turn
    uint4 rx[KSTEPS], rz[KSTEPS];
    const T* src = static_cast<const T*>(p.q) + b * p.sqb + h * p.sqh + (int64_t)(valid_q ? i_q : 0) * p.sqt;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      rx[s] = load16(src + c0 + 16 * s);
      rz[s] = load16(src + pc0 + 16 * s);
    }
    const bool norm = (p.flags & FORGE_NORM_QK) != 0;
    float rs = 1.0f;
    if (norm) {
      float ss = 0.0f;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        float x[8];
        unpack16<T>(rx[s], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      }
      ss += __shfl_xor(ss, 32, kWave);
      if (hi == 0) sh_ss[wave * 32 + n] = ss;
      __syncthreads();
      float tot = sh_ss[wbase * 32 + n];
#pragma unroll
      for (int w = 1; w < SPLIT; ++w) tot += sh_ss[(wbase + w) * 32 + n];
      rs = rsqrtf(tot / (float)D + p.eps);
    }
    const bool rope = (p.flags & FORGE_ROPE) && valid_q;
    const float* cr = rope ? p.cos + (int64_t)i_q * p.cst : nullptr;
    const float* sr = rope ? p.sin + (int64_t)i_q * p.cst : nullptr;
    const bool first_half = CW * slice < 256;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      float x[8], z[8];
      unpack16<T>(rx[s], x);
      unpack16<T>(rz[s], z);
      if (norm) {
        float wx[8], wz[8];
        if (p.qw) {
          load_f32x8(p.qw + c0 + 16 * s, wx);
          load_f32x8(p.qw + pc0 + 16 * s, wz);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] *= rs;
          z[e] *= rs;
          if (p.qw) {
            x[e] *= wx[e];
            z[e] *= wz[e];
          }
        }
      }
      if (rope) {
        float cv[8], sv[8];
        load_f32x8(cr + c0 + 16 * s, cv);
        load_f32x8(sr + c0 + 16 * s, sv);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = first_half ? x[e] * cv[e] - z[e] * sv[e] : x[e] * cv[e] + z[e] * sv[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) qreg[s][e] = from_f32<T>(valid_q ? x[e] : 0.0f);
    }
  }

  const int off = (int)p.offset;
  const int S32 = (int)S;
  const int qpos32 = (int)(p.offset + i_q);
  const int wq_lo = off + qt * TL::BM, wq_hi = off + q_last_idx;
  const int k_rd = n * TL::ROWB;
  const int k_sw = swz_k<D>(n);
  const int g = lane >> 4, kq = (lane >> 2) & 3, qq = lane & 3;
  const int v_row = 4 * (g >> 1) + kq;
  const int v_sw = swz_v<D>(v_row);
  const int v_chlo = 2 * (g & 1) + (qq >> 1);
  const int v_byte = 8 * (qq & 1);

  floatx16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.0f;
  float m_run = kNegInf, l_run = 0.0f;
  const float c = p.scale_log2;

  for (int kt = kt_begin; kt <= kt_end; ++kt) {
    const int stage = (kt - kt_begin) & 1;
    wait_vm<0>();
    __syncthreads();   // tile kt in LDS; every wave is done with tile kt - 1 and its partials
    if (kt + 1 <= kt_end) issue(kt + 1, stage ^ 1);
    const char* kl = smem + (2 * stage) * TL::TILEB + k_rd;
    const char* vl = smem + (2 * stage + 1) * TL::TILEB;

    // partial scores of this wave's channels
    floatx16 sp;
#pragma unroll
    for (int x = 0; x < 16; ++x) sp[x] = 0.0f;
#pragma unroll
    for (int st = 0; st < KSTEPS; ++st) {
      const V8 a = *reinterpret_cast<const V8*>(kl + ((CCH * slice + ((2 * st + hi) ^ k_sw)) << 4));
      sp = Mfma<T>::run(a, qreg[st], sp);
    }
    {
      float4* dst = reinterpret_cast<float4*>(part + (wave * 64 + lane) * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = make_float4(sp[4 * i], sp[4 * i + 1], sp[4 * i + 2], sp[4 * i + 3]);
    }
    __syncthreads();
    floatx16 sacc;
    {
      // the head's slices added in slice order (the same sums in every wave of the head)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float4 t = reinterpret_cast<const float4*>(part + (wbase * 64 + lane) * 16)[i];
#pragma unroll
        for (int w = 1; w < SPLIT; ++w) {
          const float4 u = reinterpret_cast<const float4*>(part + ((wbase + w) * 64 + lane) * 16)[i];
          t.x += u.x;
          t.y += u.y;
          t.z += u.z;
          t.w += u.w;
        }
        sacc[4 * i + 0] = t.x;
        sacc[4 * i + 1] = t.y;
        sacc[4 * i + 2] = t.z;
        sacc[4 * i + 3] = t.w;
      }
    }

    const int key0 = kt * BN;
    const bool full = key0 + BN - 1 <= wq_lo && key0 + BN - 1 < S32 &&
                      (p.window <= 0 || wq_hi - key0 < p.window) && q_last_idx - qt * TL::BM == TL::BM - 1 &&
                      key0 >= d_last;
    if (!full) {
      const int base = key0 + 4 * hi;
      const int top = (qpos32 < S32 - 1 ? qpos32 : S32 - 1) - base;
      const int lim_hi = valid_q ? top : -1;
      int lim_lo = p.window > 0 ? qpos32 - p.window + 1 - base : -(1 << 30);
      if (dl && d_lane - base > lim_lo) lim_lo = d_lane - base;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int ce = 8 * (x >> 2) + (x & 3);
        sacc[x] = (ce <= lim_hi && ce >= lim_lo) ? sacc[x] : kNegInf;
      }
    }
    float mx = sacc[0];
#pragma unroll
    for (int x = 1; x < 16; ++x) mx = fmaxf(mx, sacc[x]);
    mx = max_xor32(mx);
    const float mxc = mx * c;
    if (mxc > m_run + kLazyLog2) {
      const float alpha = m_run == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m_run - mxc);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[d][x] *= alpha;
      m_run = mxc;
    }
    const float neg_m = m_run == kNegInf ? 0.0f : -m_run;
    float rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[x], c, neg_m));
      sacc[x] = pv;
      rs[x & 3] += pv;
    }
    l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);

    // O^T += V^T . P^T over this wave's 128 channels
#pragma unroll
    for (int hf = 0; hf < HALVES; ++hf) {
      V8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = from_f32<T>(sacc[8 * hf + e]);
      const char* vrow0 = vl + (16 * hf + v_row) * TL::ROWB + v_byte;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const int ch = (CCH * slice + ((4 * d + v_chlo) ^ v_sw)) << 4;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vrow0 + ch));
        const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(vrow0 + 8 * TL::ROWB + ch));
        typedef short i16x8 __attribute__((ext_vector_type(8)));
        const i16x8 av = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[d] = Mfma<T>::run(__builtin_bit_cast(V8, av), pb, oacc[d]);
      }
    }
  }

  l_run += __shfl_xor(l_run, 32, kWave);
  if (!valid_q) return;
  const float inv_l = 1.0f / l_run;
  T* dst = static_cast<T*>(p.out) + b * p.sob + (int64_t)i_q * p.sot + h * p.soh + CW * slice;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T vals[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vals[j] = from_f32<T>(oacc[d][4 * i + j] * inv_l);
      *reinterpret_cast<uint2*>(dst + d * 32 + 8 * i + 4 * hi) = *reinterpret_cast<uint2*>(vals);
    }
}

template <typename T, int SPLIT>
static int launch_prefill_wide_s(PrefillParams p, hipStream_t s) {
  using TL = WideTile;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_wide_kernel<T, SPLIT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, TL::LDS_BYTES) != hipSuccess)
      return set_error("forge_attn_prefill: cannot reserve the LDS the kernel needs");
    attr_set = true;
  }
  constexpr int HPB = TL::WAVES / SPLIT;
  p.nqt = (p.T + TL::BM - 1) / TL::BM;
  if ((int64_t)p.nqt * (p.H / HPB) * p.B > 0x7fffffff) return set_error("grid too large");
  const dim3 grid((unsigned)((int64_t)p.nqt * (p.H / HPB) * p.B));
  hipLaunchKernelGGL((prefill_wide_kernel<T, SPLIT>), grid, dim3(TL::WAVES * 64), TL::LDS_BYTES, s, p);
  return check_launch();
}

// Two heads of one KV head per block (head dim in halves) where the group is even: each K/V
// tile is loaded once for both; else one head per block in quarter slices.
template <typename T>
static int launch_prefill_wide(PrefillParams p, hipStream_t s) {
  return p.G % 2 == 0 ? launch_prefill_wide_s<T, 2>(p, s) : launch_prefill_wide_s<T, 4>(p, s);
}

template <typename T>
static int launch_prefill(const PrefillParams& p, int D, hipStream_t s) {
  switch (D) {
    case 64: return launch_prefill_d<T, 64>(p, s);
    case 128: return launch_prefill_d<T, 128>(p, s);
    case 256: return launch_prefill_d<T, 256>(p, s);
    case 512: return launch_prefill_wide<T>(p, s);
    default: return set_error("forge_attn_prefill: head dim must be 64, 128, 256 or 512");
  }
}

}  // namespace forge

using namespace forge;

static int prefill_call(int dtype, int B, int T, int H, int K, int D, const void* q, int64_t sqb,
                        int64_t sqh, int64_t sqt, const float* q_weight, float eps, int flags,
                        const float* cos, const float* sin, int64_t s_cos_t, const void* k,
                        const void* v, int64_t skb, int64_t skh, int64_t sks, int64_t offset,
                        int window, float scale, void* out, int64_t sob, int64_t sot, int64_t soh,
                        const int32_t* doc_lo, int64_t sdb, void* stream) {
  if (dtype != FORGE_BF16 && dtype != FORGE_F16)
    return set_error("forge_attn_prefill: dtype must be bf16 or fp16 (use forge_attn_decode)");
  if (D != 64 && D != 128 && D != 256 && D != 512)
    return set_error("forge_attn_prefill: head dim must be 64, 128, 256 or 512");
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0) return set_error("sizes must be positive");
  if (H % K) return set_error("n_heads must be a multiple of the KV heads");
  if (offset < 0) return set_error("offset must be >= 0");
  if (window < 0) return set_error("window must be >= 0");
  if (!q || !k || !v || !out) return set_error("null tensor pointer");
  if ((flags & FORGE_ROPE) && (!cos || !sin)) return set_error("FORGE_ROPE needs cos and sin");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16)
    return set_error("forge_attn_prefill: tensors must be 16-byte aligned");
  if ((sqb | sqh | sqt | skb | skh | sks) % 8)
    return set_error("forge_attn_prefill: q/k/v strides must be multiples of 8 elements");
  if ((sob | sot | soh) % 4) return set_error("forge_attn_prefill: out strides must be multiples of 4");
  if (offset + (int64_t)T + 256 >= (1LL << 31)) return set_error("forge_attn_prefill: positions must fit in 31 bits");
  if (sks * 2 * 256 >= (1LL << 31)) return set_error("forge_attn_prefill: k/v row stride too large");
  if (((uintptr_t)q_weight | (uintptr_t)cos | (uintptr_t)sin) % 16 || (cos && s_cos_t % 4))
    return set_error("forge_attn_prefill: gain and RoPE rows must be 16-byte aligned");
  PrefillParams p{};
  p.q = q;
  p.sqb = sqb;
  p.sqh = sqh;
  p.sqt = sqt;
  p.qw = q_weight;
  p.eps = eps;
  p.flags = flags;
  p.cos = cos;
  p.sin = sin;
  p.cst = s_cos_t;
  p.k = k;
  p.v = v;
  p.skb = skb;
  p.skh = skh;
  p.sks = sks;
  p.offset = offset;
  p.B = B;
  p.T = T;
  p.H = H;
  p.K = K;
  p.G = H / K;
  p.xcd_map = (B * K) % 8 == 0 ? 1 : 0;
  p.window = window;
  p.scale_log2 = scale * kLog2e;
  p.out = out;
  p.sob = sob;
  p.sot = sot;
  p.soh = soh;
  p.doc_lo = doc_lo;
  p.sdb = sdb;
  hipStream_t s = (hipStream_t)stream;
  return dtype == FORGE_BF16 ? launch_prefill<bf16>(p, D, s) : launch_prefill<f16>(p, D, s);
}

extern "C" int forge_attn_prefill(int dtype, int B, int T, int H, int K, int D, const void* q,
                                  int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                                  float eps, int flags, const float* cos, const float* sin,
                                  int64_t s_cos_t, const void* k, const void* v, int64_t skb,
                                  int64_t skh, int64_t sks, int64_t offset, int window,
                                  float scale, void* out, int64_t sob, int64_t sot, int64_t soh,
                                  void* stream) {
  clear_error();
  return prefill_call(dtype, B, T, H, K, D, q, sqb, sqh, sqt, q_weight, eps, flags, cos, sin,
                      s_cos_t, k, v, skb, skh, sks, offset, window, scale, out, sob, sot, soh,
                      nullptr, 0, stream);
}

extern "C" int forge_attn_prefill_docs(int dtype, int B, int T, int H, int K, int D,
                                       const void* q, int64_t sqb, int64_t sqh, int64_t sqt,
                                       const float* q_weight, float eps, int flags,
                                       const float* cos, const float* sin, int64_t s_cos_t,
                                       const void* k, const void* v, int64_t skb, int64_t skh,
                                       int64_t sks, int64_t offset, int window, float scale,
                                       const int32_t* doc_start, int64_t s_doc_b, void* out,
                                       int64_t sob, int64_t sot, int64_t soh, void* stream) {
  clear_error();
  if (!doc_start) return set_error("forge_attn_prefill_docs: doc_start is null");
  if ((uintptr_t)doc_start % 4) return set_error("forge_attn_prefill_docs: doc_start must be 4-byte aligned");
  return prefill_call(dtype, B, T, H, K, D, q, sqb, sqh, sqt, q_weight, eps, flags, cos, sin,
                      s_cos_t, k, v, skb, skh, sks, offset, window, scale, out, sob, sot, soh,
                      doc_start, s_doc_b, stream);
}
