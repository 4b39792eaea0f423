// Per-row head RMSNorm + NEOX RoPE, and the K/V cache append.
//
// One group of GW lanes owns one (b, head, t) row of D values. Lane i holds the VEC
// values starting at i*VEC of the first half and the VEC values at D/2 + i*VEC of the
// second half, so the RoPE pair (c, c + D/2) (rope.py:41-55) is in one lane and only
// the RMS sum needs a cross-lane reduction. Math is fp32 with a single rounding to the
// output dtype, as fused_ops._head_kernel (fused_ops.py:53-85).
#include "common.h"
#include "forge_internal.h"

namespace forge {

struct RowTensor {
  const void* src;
  int64_t sb, sh, st;
  void* dst;
  int64_t db, dh, dt;
  const float* w;  // gain or nullptr
  int heads;
  int norm;
  int rope;
  int at_pos;  // 0: dst row t; 1: dst row base_b + t (cache write)
};

struct RowParams {
  RowTensor t[2];
  int ntensors;
  int B, T, D;
  float eps;
  const float* cos;
  const float* sin;
  int64_t csb, cst;
  const int32_t* row_pos;
  const int64_t* pos_dev;
  int64_t pos0;
  int64_t dst_len;
};

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
  if constexpr (VEC * sizeof(T) == 16) {
    unpack16<T>(load16(p), out);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = to_f32<T>(p[i]);
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const float* in) {
  if constexpr (VEC * sizeof(T) == 16) {
    store16(p, pack16<T>(in));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = from_f32<T>(in[i]);
  }
}

// A lane group handles RPL rows: RPL consecutive heads of one (b, t). They share the
// token's RoPE row and the gain, so those are loaded once per group rather than once per
// row, and the group has all RPL rows' loads in flight together.
template <typename T, int VEC, int GW, int RPL>
__global__ __launch_bounds__(256) void row_norm_rope_kernel(RowParams p) {
  // No implicit contraction (fmas are written out, and a product is not folded into its
  // rounding to fp16): forge_attn_decode_append makes the same rows with the same
  // operations in its own lane layout and must produce the same bits.
#pragma clang fp contract(off)
  constexpr int GROUPS = 256 / GW;  // lane groups per block
  const int li = threadIdx.x % GW;
  const int64_t grp = (int64_t)blockIdx.x * GROUPS + threadIdx.x / GW;
  const int64_t groups0 = (int64_t)p.B * p.t[0].heads * p.T / RPL;
  const int64_t groups1 = p.ntensors > 1 ? (int64_t)p.B * p.t[1].heads * p.T / RPL : 0;
  if (grp >= groups0 + groups1) return;  // whole group leaves together
  const bool second = grp >= groups0;
  const RowTensor& rt = second ? p.t[1] : p.t[0];
  // rows are ordered (b, t, head) with the head fastest (the groups of a wave read
  // neighbouring heads of the projection and share one token's RoPE row); the host makes
  // RPL divide the head count, so a group's rows are heads h0 .. h0 + RPL - 1 of one token
  const int64_t r0 = (second ? grp - groups0 : grp) * RPL;
  const int h0 = (int)(r0 % rt.heads);
  const int t = (int)((r0 / rt.heads) % p.T);
  const int b = (int)(r0 / ((int64_t)p.T * rt.heads));

  const int half = p.D / 2;
  const int c0 = li * VEC;
  const bool active = c0 < half;

  int64_t drow = t;
  if (rt.at_pos) {
    drow = row_base(p.row_pos, p.pos_dev, p.pos0, b) + t;
    if (drow < 0 || drow >= p.dst_len) return;  // never write past the cache
  }

  const T* src = static_cast<const T*>(rt.src) + b * rt.sb + h0 * rt.sh + t * rt.st;
  float a[RPL][VEC], z[RPL][VEC];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    if (active) {
      load_vec<T, VEC>(src + j * rt.sh + c0, a[j]);
      load_vec<T, VEC>(src + j * rt.sh + half + c0, z[j]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) a[j][i] = z[j][i] = 0.0f;
    }
  }
  if (rt.norm) {
    float wa[VEC], wz[VEC];
    const bool gain = rt.w && active;
    if (gain) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        wa[i] = rt.w[c0 + i];
        wz[i] = rt.w[half + c0 + i];
      }
    }
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss += fmaf(a[j][i], a[j][i], z[j][i] * z[j][i]);
      ss = group_sum<GW>(ss);
      const float rs = rsqrtf(fmaf(ss, 1.0f / (float)p.D, p.eps));
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        a[j][i] *= rs;
        z[j][i] *= rs;
      }
      if (gain) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          a[j][i] *= wa[i];
          z[j][i] *= wz[i];
        }
      }
    }
  }
  if (!active) return;
  if (rt.rope) {
    const float* cr = p.cos + b * p.csb + t * p.cst;
    const float* sr = p.sin + b * p.csb + t * p.cst;
    float ca[VEC], sa[VEC], cz[VEC], sz[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      ca[i] = cr[c0 + i];
      sa[i] = sr[c0 + i];
      cz[i] = cr[half + c0 + i];
      sz[i] = sr[half + c0 + i];
    }
#pragma unroll
    for (int j = 0; j < RPL; ++j)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float na = fmaf(a[j][i], ca[i], -(z[j][i] * sa[i]));
        const float nz = fmaf(z[j][i], cz[i], a[j][i] * sz[i]);
        a[j][i] = na;
        z[j][i] = nz;
      }
  }
  T* dst = static_cast<T*>(rt.dst) + b * rt.db + h0 * rt.dh + drow * rt.dt;
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    if constexpr (sizeof(T) < 4) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        a[j][i] = fp32_result(a[j][i]);
        z[j][i] = fp32_result(z[j][i]);
      }
    }
    store_vec<T, VEC>(dst + j * rt.dh + c0, a[j]);
    store_vec<T, VEC>(dst + j * rt.dh + half + c0, z[j]);
  }
}

template <typename T, int VEC, int RPL>
static int launch_rows_rpl(const RowParams& p, int gw, hipStream_t s) {
  const int64_t rows =
      (int64_t)p.B * p.T * (p.t[0].heads + (p.ntensors > 1 ? p.t[1].heads : 0));
  if (rows == 0) return 0;
  const int64_t gpb = 256 / gw;
  const int64_t groups = rows / RPL;
  const dim3 grid((unsigned)((groups + gpb - 1) / gpb));
  switch (gw) {
#define FORGE_GW(W) \
  case W: hipLaunchKernelGGL((row_norm_rope_kernel<T, VEC, W, RPL>), grid, dim3(256), 0, s, p); break;
    FORGE_GW(1) FORGE_GW(2) FORGE_GW(4) FORGE_GW(8) FORGE_GW(16) FORGE_GW(32) FORGE_GW(64)
#undef FORGE_GW
    default: return set_error("row kernel: unsupported group width");
  }
  return check_launch();
}

// Rows per lane group: 4 (or 2) consecutive heads when every tensor's head count allows.
template <typename T, int VEC>
static int launch_rows_vec(const RowParams& p, int gw, hipStream_t s) {
  auto divides = [&](int r) {
    return p.t[0].heads % r == 0 && (p.ntensors < 2 || p.t[1].heads % r == 0);
  };
  if (divides(4)) return launch_rows_rpl<T, VEC, 4>(p, gw, s);
  if (divides(2)) return launch_rows_rpl<T, VEC, 2>(p, gw, s);
  return launch_rows_rpl<T, VEC, 1>(p, gw, s);
}

template <typename T>
static int launch_rows(const RowParams& p, hipStream_t s) {
  const int half = p.D / 2;
  constexpr int V16 = 16 / sizeof(T);
  int vec = 1;
  if (half % V16 == 0) vec = V16;
  else if (half % 2 == 0) vec = 2;
  const int lanes = (half + vec - 1) / vec;
  int gw = 1;
  while (gw < lanes) gw <<= 1;
  if (gw > 64) return set_error("head dim too large for the row kernel (max 64 lanes per row)");
  if (vec == V16) return launch_rows_vec<T, V16>(p, gw, s);
  if (vec == 2) return launch_rows_vec<T, 2>(p, gw, s);
  return launch_rows_vec<T, 1>(p, gw, s);
}

static int dispatch_rows(int dtype, const RowParams& p, hipStream_t s) {
  switch (dtype) {
    case FORGE_F32: return launch_rows<float>(p, s);
    case FORGE_BF16: return launch_rows<bf16>(p, s);
    case FORGE_F16: return launch_rows<f16>(p, s);
    default: return set_error("unknown dtype code");
  }
}

}  // namespace forge

using namespace forge;

extern "C" int forge_head_norm_rope(int dtype, const void* x, void* y, int B, int H, int T,
                                    int D, int64_t sxb, int64_t sxh, int64_t sxt, int64_t syb,
                                    int64_t syh, int64_t syt, const float* weight, float eps,
                                    int norm, const float* cos, const float* sin,
                                    int64_t s_cos_b, int64_t s_cos_t, void* stream) {
  clear_error();
  if (B < 0 || H < 0 || T < 0) return set_error("negative size");
  if (D <= 0 || D % 2) return set_error("head dim must be even and positive");
  if (!x || !y) return set_error("null tensor pointer");
  if ((cos == nullptr) != (sin == nullptr)) return set_error("cos and sin must both be given");
  RowParams p{};
  p.t[0] = RowTensor{x, sxb, sxh, sxt, y, syb, syh, syt, weight, H, norm ? 1 : 0,
                     cos ? 1 : 0, 0};
  p.ntensors = 1;
  p.B = B;
  p.T = T;
  p.D = D;
  p.eps = eps;
  p.cos = cos;
  p.sin = sin;
  p.csb = s_cos_b;
  p.cst = s_cos_t;
  return dispatch_rows(dtype, p, (hipStream_t)stream);
}

extern "C" int forge_kv_append(int dtype, int B, int T, int K, int D, const void* k,
                               int64_t skb, int64_t skh, int64_t skt, const void* v,
                               int64_t svb, int64_t svh, int64_t svt, void* k_dst, void* v_dst,
                               int64_t sdb, int64_t sdh, int64_t sds, int64_t dst_len,
                               const int32_t* row_pos, const int64_t* pos_dev, int64_t pos0,
                               const float* k_weight, float eps, int flags, const float* cos,
                               const float* sin, int64_t s_cos_b, int64_t s_cos_t,
                               void* stream) {
  clear_error();
  if (B < 0 || K <= 0 || T < 0) return set_error("bad sizes");
  if (D <= 0 || D % 2) return set_error("head dim must be even and positive");
  if (!k || !v || !k_dst || !v_dst) return set_error("null tensor pointer");
  const bool rope = flags & FORGE_ROPE;
  if (rope && (!cos || !sin)) return set_error("FORGE_ROPE needs cos and sin");
  if (!row_pos && !pos_dev && (pos0 < 0 || pos0 + T > dst_len))
    return set_error("KV cache full: pos + T exceeds the cache length");
  RowParams p{};
  p.t[0] = RowTensor{k, skb, skh, skt, k_dst, sdb, sdh, sds, k_weight, K,
                     (flags & FORGE_NORM_QK) ? 1 : 0, rope ? 1 : 0, 1};
  p.t[1] = RowTensor{v, svb, svh, svt, v_dst, sdb, sdh, sds, nullptr, K,
                     (flags & FORGE_NORM_V) ? 1 : 0, 0, 1};
  p.ntensors = 2;
  p.B = B;
  p.T = T;
  p.D = D;
  p.eps = eps;
  p.cos = cos;
  p.sin = sin;
  p.csb = s_cos_b;
  p.cst = s_cos_t;
  p.row_pos = row_pos;
  p.pos_dev = pos_dev;
  p.pos0 = pos0;
  p.dst_len = dst_len;
  return dispatch_rows(dtype, p, (hipStream_t)stream);
}
