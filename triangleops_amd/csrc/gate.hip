// Gate + output projection, shared by triangle_attention and attention_pair_bias:
//   out[t] = ((o[t] * sigmoid(g_in[t] . Wg^T + bg)) -> io) . Wo^T + bo,   C = 128,
// where g_in = LN(x) (triangle attention: the gate reads LN(x), recomputed here from x so the
// normalized tensor is never written to HBM) or the raw input (attention_pair_bias).
//
// Reference: triangle_attn/kernel.py:387-470 (`fused_gate_kernel`, o gathered at native
// strides) and attn_pair_bias/module.py:69-70 (gate on raw X with biases, then Wo).
// Both weights are read in their (out, in) nn.Linear layout: no per-call transposes.
//
// 64-token tiles, 4 waves; wave w owns features [32w, 32w + 32) of both GEMMs with its weight
// rows in registers.  The gate input and the gated activations go through token-major LDS
// tiles (XOR-swizzled 16-byte chunks) so each GEMM reads all 128 channels of a token as k.
#include "capi.hpp"
#include "common.hpp"

namespace tops {

template <typename T>
__global__ __launch_bounds__(256) void gate_out_kernel(const T* __restrict__ o, int64_t so0, int64_t so1,
                                                      const T* __restrict__ gin, int64_t sg0, int64_t sg1,
                                                      const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                      float ln_eps, int apply_ln, const T* __restrict__ Wg,
                                                      const T* __restrict__ bg, const T* __restrict__ Wo,
                                                      const T* __restrict__ bo, T* __restrict__ out, int64_t M2,
                                                      int64_t M, int64_t ntiles) {
  constexpr int C = 128, ROW = C * 2, KS = C / 16;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;
  __shared__ __attribute__((aligned(16))) char gs[64 * ROW];
  __shared__ __attribute__((aligned(16))) char ts[64 * ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;

  V8 wg[KS], wo[KS];
  {
    const int64_t frow = (int64_t)(wave * 32 + col) * C;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      wg[s] = ldg<V8>(Wg + frow + 16 * s + 8 * hl);
      wo[s] = ldg<V8>(Wo + frow + 16 * s + 8 * hl);
    }
  }
  float cbg[16], cbo[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int f = wave * 32 + 8 * (v / 4) + 4 * hl + (v % 4);
    cbg[v] = bg ? (float)bg[f] : 0.f;
    cbo[v] = bo ? (float)bo[f] : 0.f;
  }
  const int ltok = tid >> 2, part = tid & 3;  // gate-input loader: 4 threads per token

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t t0 = tile * 64;
    // ---- gate input tile (LN applied if asked) -> LDS ----
    {
      const int64_t m = t0 + ltok;
      float v[32];
      if (m < M) {
        const T* src = gin + (m / M2) * sg0 + (m % M2) * sg1 + 32 * part;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const V8 a = ldg<V8>(src + 8 * e);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[8 * e + j] = (float)a[j];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 32; ++e) v[e] = 0.f;
      }
      if (apply_ln) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) s += v[e];
        const float mean = group_sum<4>(s) * (1.0f / C);
        float q = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) q += (v[e] - mean) * (v[e] - mean);
        const float rstd = rsqrtf(group_sum<4>(q) * (1.0f / C) + ln_eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const V8 w8 = ldg<V8>(w_ln + 32 * part + 8 * e);
          const V8 b8 = b_ln ? ldg<V8>(b_ln + 32 * part + 8 * e) : V8{};
#pragma unroll
          for (int j = 0; j < 8; ++j) v[8 * e + j] = (v[8 * e + j] - mean) * rstd * (float)w8[j] + (float)b8[j];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        V8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (T)v[8 * e + j];
        const int chunk = 4 * part + e;
        *reinterpret_cast<V8*>(&gs[ltok * ROW + ((chunk ^ (ltok & 7)) << 4)]) = r;
      }
    }
    __syncthreads();
    // ---- gate GEMM, sigmoid, multiply by o -> LDS ----
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int t = sub * 32 + col;
      int64_t tok = t0 + t;
      tok = tok < M ? tok : M - 1;
      f32x16 acc = {};
#pragma unroll
      for (int k = 0; k < KS; ++k)
        acc = Mma<T>::m32(wg[k], *reinterpret_cast<const V8*>(&gs[t * ROW + (((2 * k + hl) ^ (t & 7)) << 4)]), acc);
      const T* orow = o + (tok / M2) * so0 + (tok % M2) * so1 + wave * 32 + 4 * hl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const V4 ov = ldg<V4>(orow + 8 * g);
        V4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (T)((float)ov[e] * sigmoid(acc[4 * g + e] + cbg[4 * g + e]));
        const int chunk = wave * 4 + g;  // features [8 chunk, 8 chunk + 8)
        *reinterpret_cast<V4*>(&ts[t * ROW + ((chunk ^ (t & 7)) << 4) + 8 * hl]) = r;
      }
    }
    __syncthreads();
    // ---- output GEMM ----
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int t = sub * 32 + col;
      f32x16 acc = {};
#pragma unroll
      for (int k = 0; k < KS; ++k)
        acc = Mma<T>::m32(wo[k], *reinterpret_cast<const V8*>(&ts[t * ROW + (((2 * k + hl) ^ (t & 7)) << 4)]), acc);
      const int64_t tok = t0 + t;
      if (tok < M) {
        T* dst = out + tok * C + wave * 32 + 4 * hl;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          V4 r;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = (T)(acc[4 * g + e] + cbo[4 * g + e]);
          stg<V4>(dst + 8 * g, r);
        }
      }
    }
    __syncthreads();
  }
}

template <typename T>
static int gate_out_t(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                      const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg, const void* bg,
                      const void* Wo, const void* bo, void* out, int64_t M1, int64_t M2, hipStream_t st) {
  const int64_t M = M1 * M2;
  const int64_t ntiles = (M + 63) / 64;
  if (ntiles == 0) return TOPS_OK;
  const int64_t grid = ntiles < 8LL * num_cus() ? ntiles : 8LL * num_cus();
  hipLaunchKernelGGL((gate_out_kernel<T>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)o, so0, so1,
                     (const T*)gin, sg0, sg1, (const T*)w_ln, (const T*)b_ln, ln_eps, apply_ln, (const T*)Wg,
                     (const T*)bg, (const T*)Wo, (const T*)bo, (T*)out, M2, M, ntiles);
  return launched("tops_gate_out");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_gate_out(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                             const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg,
                             const void* bg, const void* Wo, const void* bo, void* out, int64_t M1, int64_t M2,
                             int64_t C, int dtype, void* stream) {
  TOPS_REQUIRE(o && gin && Wg && Wo && out, "tops_gate_out: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_gate_out: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(C == 128, "tops_gate_out: C must be 128 (got %lld)", (long long)C);
  TOPS_REQUIRE(M1 >= 0 && M2 >= 0, "tops_gate_out: bad sizes");
  TOPS_REQUIRE(so0 % 4 == 0 && so1 % 4 == 0, "tops_gate_out: o token strides must be multiples of 4");
  TOPS_REQUIRE(sg0 % 8 == 0 && sg1 % 8 == 0, "tops_gate_out: gate-input token strides must be multiples of 8");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return gate_out_t<__bf16>(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, out, M1, M2,
                              st);
  if (dtype == TOPS_DTYPE_F16)
    return gate_out_t<_Float16>(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, out, M1,
                                M2, st);
  return fail(TOPS_EUNSUPPORTED, "tops_gate_out: unsupported dtype code %d", dtype);
}
