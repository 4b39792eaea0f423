// Device helpers shared by the FORGE attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace forge {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

typedef __bf16 bf16;
typedef _Float16 f16;

// ---------------------------------------------------------------- element conversion
template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

// 16 bytes of T unpacked to fp32 (VEC = 16 / sizeof(T) values).
template <typename T> struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
};

template <typename T>
__device__ __forceinline__ void unpack16(const uint4& raw, float* out) {
  const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
  for (int i = 0; i < Vec16<T>::N; ++i) out[i] = to_f32<T>(e[i]);
}

template <typename T>
__device__ __forceinline__ uint4 pack16(const float* in) {
  uint4 raw;
  T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
  for (int i = 0; i < Vec16<T>::N; ++i) e[i] = from_f32<T>(in[i]);
  return raw;
}

// Marks x as computed: the compiler may then not fold the fp32 operation that produced it
// into the rounding to a 16-bit type (a v_fma_mix*_f16 rounds once, where the reference's
// fp32 math followed by .to(dtype) rounds twice).
__device__ __forceinline__ float fp32_result(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// 8 consecutive fp32 values from a 16-byte aligned address, as two 16-byte loads.
__device__ __forceinline__ void load_f32x8(const float* p, float* out) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

__device__ __forceinline__ void store16(void* p, const uint4& v) {
  *reinterpret_cast<uint4*>(p) = v;
}

// ---------------------------------------------------------------- cross-lane sums
// DPP lane permutations (GCN/CDNA dpp_ctrl encodings).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7-i within each 8
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15-i within each 16

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Partner value across lane distance 2^k of an aligned group, for the butterfly steps
// below. Steps 1 and 2 swap within quads, steps 4 and 8 mirror the 8- and 16-lane
// halves (after the earlier steps all lanes of a quad / 8 hold the same value, so a
// mirror pairs each lane with the other half exactly like an xor would).
template <int STEP>
__device__ __forceinline__ float butterfly_partner(float v) {
  if constexpr (STEP == 1) return dpp<kDppQuadXor1>(v);
  else if constexpr (STEP == 2) return dpp<kDppQuadXor2>(v);
  else if constexpr (STEP == 4) return dpp<kDppRowHalfMirror>(v);
  else if constexpr (STEP == 8) return dpp<kDppRowMirror>(v);
  else return __shfl_xor(v, STEP, kWave);
}

// All-reduce over aligned groups of W lanes (W a power of two <= 64): every lane of
// the group ends with the same value, since each butterfly step adds the same two
// operands on both partner lanes (a + b == b + a in IEEE arithmetic).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W >= 2) v += butterfly_partner<1>(v);
  if constexpr (W >= 4) v += butterfly_partner<2>(v);
  if constexpr (W >= 8) v += butterfly_partner<4>(v);
  if constexpr (W >= 16) v += butterfly_partner<8>(v);
  if constexpr (W >= 32) v += butterfly_partner<16>(v);
  if constexpr (W >= 64) v += butterfly_partner<32>(v);
  return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (W >= 2) v = fmaxf(v, butterfly_partner<1>(v));
  if constexpr (W >= 4) v = fmaxf(v, butterfly_partner<2>(v));
  if constexpr (W >= 8) v = fmaxf(v, butterfly_partner<4>(v));
  if constexpr (W >= 16) v = fmaxf(v, butterfly_partner<8>(v));
  if constexpr (W >= 32) v = fmaxf(v, butterfly_partner<16>(v));
  if constexpr (W >= 64) v = fmaxf(v, butterfly_partner<32>(v));
  return v;
}

// exp2 that maps -inf to exactly 0 and never sees (-inf) - (-inf).
__device__ __forceinline__ float exp2_masked(float s, float m) {
  return s == kNegInf ? 0.0f : exp2f(s - m);
}

// Rescale factor of a running (max, sum) pair when the max moves from m_old to m_new.
__device__ __forceinline__ float rescale(float m_old, float m_new) {
  return m_old == kNegInf ? 0.0f : exp2f(m_old - m_new);
}

// ---------------------------------------------------------------- LDS direct loads
typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ unsigned lds_offset(const void* ptr) {
  return (unsigned)(uintptr_t)(const lds_char*)ptr;
}
// global_load_lds_dwordx4 (lane i's 16 bytes from gbase + voff land at LDS address
// lds + 16 i) from inline asm: the compiler then does not make later LDS reads wait for
// it, so the kernel waits for these loads itself (s_waitcnt vmcnt). M0 carries the LDS
// address and is restored.
__device__ __forceinline__ void lds_dma16(const void* gbase, unsigned voff, unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(gbase), "s"(lds)
      : "memory");
}

// max over lanes l and l ^ 32 with gfx950's v_permlane32_swap (VALU, no LDS round trip):
// swapping x with itself returns the lower half's and the upper half's value of the pair.
// (The pair is read by value: __builtin_bit_cast of a vector element reads element 0.)
__device__ __forceinline__ float max_xor32(float x) {
  const unsigned u = __float_as_uint(x);
  const auto c = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned c0 = c[0], c1 = c[1];
  return fmaxf(__uint_as_float(c0), __uint_as_float(c1));
}

// Base position of batch row b (see include/forge_attn.h).
__device__ __forceinline__ int64_t row_base(const int32_t* row_pos, const int64_t* pos_dev,
                                            int64_t pos0, int b) {
  if (row_pos) return (int64_t)row_pos[b];
  if (pos_dev) return *pos_dev;
  return pos0;
}

}  // namespace forge
