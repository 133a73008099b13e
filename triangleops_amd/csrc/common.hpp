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
};

template <>
struct Mma<_Float16> {
  __device__ static inline f32x16 m32(vec<_Float16, 8> a, vec<_Float16, 8> b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4 m16(vec<_Float16, 8> a, vec<_Float16, 8> b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <typename V>
__device__ inline V ldg(const void* p) {
  return *reinterpret_cast<const V*>(p);
}

template <typename V>
__device__ inline void stg(void* p, V v) {
  *reinterpret_cast<V*>(p) = v;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)); saturates cleanly to 0 / 1.
__device__ inline float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-x * kLog2e)); }

// Sum over groups of `W` adjacent lanes (W = 2, 4, 8, ...) via xor shuffles.
template <int W>
__device__ inline float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < W; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// max / sum of the values held by lanes l and l ^ 32, returned in both lanes.
__device__ inline float halves_max(float v) { return fmaxf(v, __shfl_xor(v, 32)); }
__device__ inline float halves_sum(float v) { return v + __shfl_xor(v, 32); }

}  // namespace tops
