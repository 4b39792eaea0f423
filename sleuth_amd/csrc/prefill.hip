// Causal prefill on bf16/fp16 MFMA (gfx950 v_mfma_f32_32x32x16_{bf16,f16}).
//
// A block of 4 waves owns BM = 128 queries of one (b, head); each wave owns 32 of them.
// K and V tiles of BN = 64 keys are staged in LDS (the next tile is prefetched into
// registers while the current one is used) and shared by the 4 waves.
//
// Scores are computed transposed, S^T = K . Q^T, with K as the MFMA A operand (read
// row-major from LDS) and Q^T as the B operand (held in registers for the whole block).
// In the 32x32 accumulator layout every lane then owns ONE query (column l % 32) and 16
// of the 32 keys of a block (rows 8i + 4(l/32) + j), so the online softmax needs one
// cross-lane step per reduction (lane l <-> l ^ 32), and the output accumulator
// O^T = V^T . P^T has the same property: all 16 values of a lane belong to its query,
// so the rescale by exp(m_old - m_new) is a per-lane scalar.
//
// P^T is fed to the second MFMA straight from the score registers: lane (n, hi) holds
// keys {8i + 4hi + j}; the MFMA's k index 8hi + 4i' + j is mapped to key
// 16*half + 8i' + 4hi + j (i = 2*half + i'). V is written to LDS transposed (V^T, one
// row per head-dim channel) with its key columns permuted the same way, so each lane
// reads its 8 keys of V^T with one 128-bit LDS load.
//
// Q gets the per-head RMSNorm and RoPE in the load (fp32 math, one rounding), like
// fused_ops._head_kernel (fused_ops.py:53-85); K and V come from the cache, where
// forge_kv_append wrote them already normalised.
#include "common.h"
#include "forge_internal.h"

namespace forge {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
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
  int nqt;  // query tiles
  int window;
  float scale_log2;
  void* out;
  int64_t sob, sot, soh;
};

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kPad = 8;  // elements of padding per LDS row

// Column of key k (0..63 within a tile) in the permuted V^T rows.
__device__ __forceinline__ int vt_col(int k) {
  const int kb = k >> 5, kk = k & 31;
  const int half = kk >> 4, k16 = kk & 15;
  const int ip = k16 >> 3, hi = (k16 & 7) >> 2, j = k16 & 3;
  return kb * 32 + half * 16 + hi * 8 + ip * 4 + j;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillParams p) {
  using V8 = typename Mfma<T>::vec;
  constexpr int KSTEPS = D / 16;  // MFMA k-steps over the head dim (scores)
  constexpr int DB = D / 32;      // 32-channel blocks of the output
  constexpr int KCH = D / 8;      // 16-byte chunks per K/V row
  constexpr int KTOTAL = kBN * KCH;        // 16-byte K chunks per tile
  constexpr int VTOTAL = (kBN / 4) * KCH;  // V pieces of 4 keys x 8 channels per tile
  constexpr int KLOADS = (KTOTAL + 255) / 256;
  constexpr int VQUADS = (VTOTAL + 255) / 256;

  __shared__ __attribute__((aligned(16))) T sK[kBN][D + kPad];
  __shared__ __attribute__((aligned(16))) T sVt[D][kBN + kPad];

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int n = lane & 31;
  const int hi = lane >> 5;

  // Block -> (query tile, head, batch). Heavy (late) causal tiles go first; the heads
  // of one KV group and the batch rows are ordered so that blocks reading the same K/V
  // are 8 apart in launch order, i.e. on the same XCD (and its L2).
  const int HB = p.H * p.B;
  const int qt = p.nqt - 1 - (int)(blockIdx.x / HB);
  const int hb = blockIdx.x % HB;
  const int P = p.B * p.K;
  const int pair = hb % P;
  const int gq = hb / P;
  const int b = pair / p.K;
  const int kvh = pair % p.K;
  const int h = kvh * p.G + gq;

  const int i_q = qt * kBM + wave * 32 + n;  // this lane's query (index into T)
  const bool valid_q = i_q < p.T;
  const int64_t qpos = p.offset + i_q;
  const int64_t S = p.offset + p.T;

  // ---- Q: load, fused RMSNorm + RoPE, one rounding, kept as MFMA B operands.
  V8 qreg[KSTEPS];
  {
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
        for (int e = 0; e < 8; ++e) {
          qf[s][e] *= rs;
          if (p.qw) qf[s][e] *= p.qw[16 * s + 8 * hi + e];
        }
    }
    if ((p.flags & FORGE_ROPE) && valid_q) {
      const float* cr = p.cos + (int64_t)i_q * p.cst;
      const float* sr = p.sin + (int64_t)i_q * p.cst;
#pragma unroll
      for (int s = 0; s < KSTEPS / 2; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int x = 16 * s + 8 * hi + e;  // first-half channel; partner x + D/2
          const float a = qf[s][e], z = qf[s + KSTEPS / 2][e];
          qf[s][e] = a * cr[x] - z * sr[x];
          qf[s + KSTEPS / 2][e] = z * cr[x + D / 2] + a * sr[x + D / 2];
        }
    }
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qreg[s][e] = from_f32<T>(qf[s][e]);
  }

  // ---- key tiles this block needs
  const int64_t q_first = p.offset + (int64_t)qt * kBM;
  const int64_t q_last_idx = (int64_t)qt * kBM + kBM - 1 < p.T - 1 ? (int64_t)qt * kBM + kBM - 1 : p.T - 1;
  const int64_t blk_kmax = p.offset + q_last_idx;
  int64_t blk_kmin = p.window > 0 ? q_first - p.window + 1 : 0;
  if (blk_kmin < 0) blk_kmin = 0;
  const int kt_begin = (int)(blk_kmin / kBN);
  const int kt_end = (int)(blk_kmax / kBN);

  // this wave's query span (for tile skipping and the mask-free fast path)
  const int w_first = qt * kBM + wave * 32;
  const int w_last = w_first + 31 < p.T - 1 ? w_first + 31 : p.T - 1;
  const bool wave_any = w_first < p.T;
  const int64_t wq_lo = p.offset + w_first, wq_hi = p.offset + w_last;

  const T* kg = static_cast<const T*>(p.k) + b * p.skb + kvh * p.skh;
  const T* vg = static_cast<const T*>(p.v) + b * p.skb + kvh * p.skh;

  uint4 kpre[KLOADS];
  uint4 vpre[VQUADS][4];
  auto prefetch = [&](int kt) {
    const int64_t key0 = (int64_t)kt * kBN;
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / KCH, ch = idx % KCH;
      const int64_t key = key0 + r;
      kpre[i] = (idx < KTOTAL && key < S) ? load16(kg + key * p.sks + ch * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VQUADS; ++i) {
      const int idx = tid + i * 256;
      const int kq = idx / KCH, ho = idx % KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t key = key0 + kq * 4 + r;
        vpre[i][r] = (idx < VTOTAL && key < S) ? load16(vg + key * p.sks + ho * 8)
                                               : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int idx = tid + i * 256;
      if (KTOTAL % 256 && idx >= KTOTAL) break;
      const int r = idx / KCH, ch = idx % KCH;
      store16(&sK[r][ch * 8], kpre[i]);
    }
#pragma unroll
    for (int i = 0; i < VQUADS; ++i) {
      const int idx = tid + i * 256;
      if (VTOTAL % 256 && idx >= VTOTAL) break;
      const int kq = idx / KCH, ho = idx % KCH;
      const int col = vt_col(kq * 4);
      const unsigned short* e0 = reinterpret_cast<const unsigned short*>(&vpre[i][0]);
      const unsigned short* e1 = reinterpret_cast<const unsigned short*>(&vpre[i][1]);
      const unsigned short* e2 = reinterpret_cast<const unsigned short*>(&vpre[i][2]);
      const unsigned short* e3 = reinterpret_cast<const unsigned short*>(&vpre[i][3]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint2 w;
        w.x = (unsigned)e0[e] | ((unsigned)e1[e] << 16);
        w.y = (unsigned)e2[e] | ((unsigned)e3[e] << 16);
        *reinterpret_cast<uint2*>(&sVt[ho * 8 + e][col]) = w;
      }
    }
  };

  floatx16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int x = 0; x < 16; ++x) oacc[d][x] = 0.0f;
  float m_run = kNegInf, l_run = 0.0f;

  if (kt_begin <= kt_end) prefetch(kt_begin);
  for (int kt = kt_begin; kt <= kt_end; ++kt) {
    __syncthreads();
    commit();
    __syncthreads();
    if (kt + 1 <= kt_end) prefetch(kt + 1);

    const int64_t key0 = (int64_t)kt * kBN;
    // Does this tile hold any key visible to this wave? (wave-uniform)
    const bool wave_needs = wave_any && key0 <= wq_hi &&
                            (p.window <= 0 || key0 + kBN - 1 > wq_lo - p.window);
    if (!wave_needs) continue;
    const bool full = key0 + kBN - 1 <= wq_lo && key0 + kBN - 1 < S &&
                      (p.window <= 0 || wq_hi - key0 < p.window) && w_last - w_first == 31;

    floatx16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int x = 0; x < 16; ++x) sacc[kb][x] = 0.0f;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const V8 a = *reinterpret_cast<const V8*>(&sK[kb * 32 + n][16 * s + 8 * hi]);
        sacc[kb] = Mfma<T>::run(a, qreg[s], sacc[kb]);
      }
    }

    float mx = kNegInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        float v = sacc[kb][x] * p.scale_log2;
        if (!full) {
          const int64_t key = key0 + kb * 32 + 8 * (x >> 2) + 4 * hi + (x & 3);
          const bool ok = valid_q && key <= qpos && key < S &&
                          (p.window <= 0 || qpos - key < p.window);
          if (!ok) v = kNegInf;
        }
        sacc[kb][x] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = rescale(m_run, m_new);
    float rsum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const float pv = exp2_masked(sacc[kb][x], m_new);
        sacc[kb][x] = pv;
        rsum += pv;
      }
    rsum += __shfl_xor(rsum, 32, kWave);
    l_run = l_run * alpha + rsum;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int x = 0; x < 16; ++x) oacc[d][x] *= alpha;

#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        V8 pb;
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[e] = from_f32<T>(sacc[kb][8 * half + e]);
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const V8 a =
              *reinterpret_cast<const V8*>(&sVt[d * 32 + n][kb * 32 + half * 16 + hi * 8]);
          oacc[d] = Mfma<T>::run(a, pb, oacc[d]);
        }
      }
  }

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

template <typename T>
static int launch_prefill(const PrefillParams& p, int D, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.nqt * p.H * p.B));
  switch (D) {
    case 64: hipLaunchKernelGGL((prefill_kernel<T, 64>), grid, dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<T, 128>), grid, dim3(256), 0, s, p); break;
    case 256: hipLaunchKernelGGL((prefill_kernel<T, 256>), grid, dim3(256), 0, s, p); break;
    default: return set_error("forge_attn_prefill: head dim must be 64, 128 or 256");
  }
  return check_launch();
}

}  // namespace forge

using namespace forge;

extern "C" int forge_attn_prefill(int dtype, int B, int T, int H, int K, int D, const void* q,
                                  int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                                  float eps, int flags, const float* cos, const float* sin,
                                  int64_t s_cos_t, const void* k, const void* v, int64_t skb,
                                  int64_t skh, int64_t sks, int64_t offset, int window,
                                  float scale, void* out, int64_t sob, int64_t sot, int64_t soh,
                                  void* stream) {
  clear_error();
  if (dtype != FORGE_BF16 && dtype != FORGE_F16)
    return set_error("forge_attn_prefill: dtype must be bf16 or fp16 (use forge_attn_decode)");
  if (D != 64 && D != 128 && D != 256)
    return set_error("forge_attn_prefill: head dim must be 64, 128 or 256");
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
  p.nqt = (T + kBM - 1) / kBM;
  p.window = window;
  p.scale_log2 = scale * kLog2e;
  p.out = out;
  p.sob = sob;
  p.sot = sot;
  p.soh = soh;
  if ((int64_t)p.nqt * H * B > 0x7fffffff) return set_error("grid too large");
  hipStream_t s = (hipStream_t)stream;
  return dtype == FORGE_BF16 ? launch_prefill<bf16>(p, D, s) : launch_prefill<f16>(p, D, s);
}
