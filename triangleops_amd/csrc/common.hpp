// Shared device helpers for the gfx950 (CDNA4) kernels of triangleops_amd.
//
// MFMA lane layouts used throughout (checked on MI355X by a lane-layout probe):
//   v_mfma_f32_32x32x16_{bf16,f16}:  A (32 x 16): lane l holds A[l%32][8*(l/32) + e], e = 0..7
//                                    B (16 x 32): lane l holds B[8*(l/32) + e][l%32]
//                                    D (32 x 32): lane l, slot v holds D[8*(v/4) + 4*(l/32) + v%4][l%32]
//   v_mfma_f32_16x16x32_{bf16,f16}:  A (16 x 32): lane l holds A[l%16][8*(l/16) + e]
//                                    B (32 x 16): lane l holds B[8*(l/16) + e][l%16]
//                                    D (16 x 16): lane l, slot v holds D[4*(l/16) + v][l%16]
// Only the pairing of A and B along k matters for a product, so any k-permutation applied
// identically to both operands gives the same result; the kernels use that freedom to feed
// one MFMA's D registers straight into the next MFMA's A/B operand without shuffles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tops {

template <typename T, int N>
using vec = T __attribute__((ext_vector_type(N)));

using f32x4 = vec<float, 4>;
using f32x16 = vec<float, 16>;

constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct Mma;

template <>
struct Mma<__bf16> {
  __device__ static inline f32x16 m32(vec<__bf16, 8> a, vec<__bf16, 8> b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4 m16(vec<__bf16, 8> a, vec<__bf16, 8> b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // c + a.x * b.x + a.y * b.y with fp32 products and sum (v_dot2c_f32_bf16)
  __device__ static inline float dot2(vec<__bf16, 2> a, vec<__bf16, 2> b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
  static constexpr float kMaxP = 18446744073709551616.0f;  // 2^64: bf16 keeps fp32's range
};

template <>
struct Mma<_Float16> {
  __device__ static inline f32x16 m32(vec<_Float16, 8> a, vec<_Float16, 8> b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4 m16(vec<_Float16, 8> a, vec<_Float16, 8> b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline float dot2(vec<_Float16, 2> a, vec<_Float16, 2> b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
  static constexpr float kMaxP = 32768.0f;  // 2^15: below fp16's largest finite value 65504
};

// acc + the sum of the 8 elements of `a`, in fp32 (4 packed-pair dot products against 1.0).
template <typename T>
__device__ inline float sum8(vec<T, 8> a, float acc) {
  const vec<T, 2> one = {(T)1.0f, (T)1.0f};
#pragma unroll
  for (int e = 0; e < 8; e += 2) acc = Mma<T>::dot2(vec<T, 2>{a[e], a[e + 1]}, one, acc);
  return acc;
}

// Division by a runtime constant d >= 1 of 32-bit unsigned n (Granlund-Montgomery): a multiply-
// high, an add and a shift, all scalar when n is wave-uniform.
struct FastDiv {
  uint32_t d, m, s;
  __host__ __device__ FastDiv() : d(1), m(1), s(0) {}
  __host__ explicit FastDiv(uint32_t div) : d(div), m(0), s(0) {
    while ((1ull << s) < div) ++s;
    m = (uint32_t)(((1ull << 32) * ((1ull << s) - div)) / div + 1);
  }
  __host__ __device__ uint32_t div(uint32_t n) const {
#ifdef __HIP_DEVICE_COMPILE__
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
    return (uint32_t)(((uint64_t)hi + n) >> s);
  }
};

// Pins `v` in registers at this point of the program: the compiler must compute it here and
// may not sink its computation into a later branch.
template <typename V>
__device__ inline void pin(V& v) {
  asm volatile("" : "+v"(v));
}

template <typename V>
__device__ inline V ldg(const void* p) {
  return *reinterpret_cast<const V*>(p);
}

template <typename V>
__device__ inline void stg(void* p, V v) {
  *reinterpret_cast<V*>(p) = v;
}

// Waits until at most N vector-memory operations of this wave are outstanding (s_waitcnt with
// the expcnt / lgkmcnt fields at their maxima, i.e. not waited on).  gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
template <int N>
__device__ inline void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// LDS chunk swizzle of a token row of the pre-pass and gate tiles: 16 rows read together (one
// per lane of a 16-lane group) hit 16 distinct 16-byte bank groups.  A 256-byte row (C = 128)
// spans all 64 banks: chunk ^ (t & 15).  A 128-byte row (C = 64) spans half of them, the row
// parity picks the half: chunk ^ ((t >> 1) & 7).
template <int C>
__device__ inline int row_key(int t) {
  static_assert(C == 128 || C == 64, "row width");
  return C == 128 ? (t & 15) : ((t >> 1) & 7);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)); saturates cleanly to 0 / 1.
__device__ inline float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-x * kLog2e)); }

// Lane permutation through DPP (a VALU operand modifier, no LDS traffic).
template <int CTRL>
__device__ inline float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of `W` adjacent lanes (W = 1, 2, 4, 8, 16), result in every lane of
// the group: quad permutations (xor 1, xor 2), then half-row and row mirrors, which pair each
// lane with one in the other half of its 8- / 16-lane group.
template <int W>
__device__ inline float group_sum(float v) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16, "group width");
  if constexpr (W >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp<0x141>(v);  // row_half_mirror
  if constexpr (W >= 16) v += dpp<0x140>(v); // row_mirror
  return v;
}

// max / sum of the values held by lanes l and l ^ 32, returned in both lanes.
// v_permlane32_swap exchanges the upper half of its first operand with the lower half of
// its second; with both operands = v the two results hold (lo, lo) and (hi, hi).
__device__ inline float halves_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float halves_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace tops
