// Gate + output projection, shared by triangle_attention and attention_pair_bias:
//   out[t] = ((o[t] * sigmoid(g_in[t] . Wg^T + bg)) -> io) . Wo^T + bo,   C = C_in = H*D = C_out,
// C = 128 or 64,
// where g_in = LN(x) (triangle attention: the gate reads LN(x), recomputed here from x so the
// normalized tensor is never written to HBM) or the raw input (attention_pair_bias).
//
// Reference: triangle_attn/kernel.py:387-470 (`fused_gate_kernel`, o gathered at native
// strides) and attn_pair_bias/module.py:69-70 (gate on raw X with biases, then Wo).
// Both weights are read in their (out, in) nn.Linear layout: no per-call transposes.
//
// Tiles of 8192 / C tokens (64 at C = 128, 128 at C = 64: 16 KB of each input), 8 waves.  Waves
// 0-3 fetch the gate-input tile two tiles ahead (two register stages; C / 8 lanes per token row)
// and stage it in LDS, normalised; waves 4-7 fetch and stage the o tile the same way and write
// the results (splitting the loads between the two roles balances them: the loaders' LayerNorm
// had kept every other wave waiting at the first barrier; 3 % faster at N = 1024).  All waves compute: wave w owns features [32 (w % (C / 32)), +32) of both GEMMs
// for tokens [32 (w / (C / 32)), +32), weight rows in registers (permuted so each lane ends up
// with 16 consecutive features of one token; Wg's rows times -log2(e), rounded to the I/O type,
// and -log2(e) bg as one more MFMA k-step, so the first GEMM's accumulator is the gate's exp2
// argument: 3-5 % faster than an fp32 multiply-add per output, results within a bf16 step; bo
// enters the second GEMM the same way instead of an add per output, 2-4 % faster).  The
// gated activations overwrite the o tile in LDS and are the second GEMM's operand; the output
// goes through a token-major LDS tile so each store instruction writes whole token rows.
#include "capi.hpp"
#include "common.hpp"

namespace tops {

// RES: out[m1, m2] = res[m1, m2] + result, both at their own token strides (the residual add of
// a Pairformer block fused into the store; the sum is rounded once, as a separate add would be).
template <typename T, bool LN, bool RES, int C>
__global__ __launch_bounds__(512) void gate_out_kernel(const T* __restrict__ o, int64_t so0, int64_t so1,
                                                      const T* __restrict__ gin, int64_t sg0, int64_t sg1,
                                                      const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                      float ln_eps, const T* __restrict__ Wg,
                                                      const T* __restrict__ bg, const T* __restrict__ Wo,
                                                      const T* __restrict__ bo, const T* __restrict__ res,
                                                      int64_t sr0, int64_t sr1, T* __restrict__ out, int64_t sd0,
                                                      int64_t sd1, FastDiv M2, uint32_t M, uint32_t ntiles) {
  static_assert(C == 128 || C == 64, "feature width");
  constexpr int ROW = C * 2, KS = C / 16;
  constexpr int TOK = 8192 / C;  // tokens per tile
  constexpr int LPT = C / 8;     // loader lanes (16-byte chunks) per token row
  constexpr int FS = C / 32;     // feature groups of 32: wave w = feature group w % FS, tokens w / FS
  constexpr int NL = 256;        // loader threads (waves 0-3); writers are waves 4-7
  constexpr int PD = 2;          // register stages in flight
  using V8 = vec<T, 8>;
  using V2 = vec<T, 2>;

  // one staging buffer suffices: the next tile is staged only after the third barrier, when
  // every wave has finished reading this one
  __shared__ __attribute__((aligned(16))) char gs[TOK * ROW];   // gate input (normalised)
  __shared__ __attribute__((aligned(16))) char ots[TOK * ROW];  // o, then the gated values
  __shared__ __attribute__((aligned(16))) T os[TOK * C];          // output tile, token-major

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int fset = wave % FS, sub = wave / FS;

  // A operand row r = col holds feature 32 fset + prow: D slot v of lane half hl is then
  // feature 32 fset + 16 hl + v
  const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);
  // G's rows times -log2(e) and its bias -log2(e) bg as one more MFMA k-step (A: the row's bias
  // as two 16-bit parts at k = 0, 1; B: 1 there for every token), so the accumulator is the
  // gate's exp2 argument: no multiply-add per output
  V8 wg[KS], wo[KS], gb_a, one_b, ob_a;
  {
    const int64_t frow = (int64_t)(32 * fset + prow) * C;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const V8 g = ldg<V8>(Wg + frow + 16 * s + 8 * hl);
#pragma unroll
      for (int e = 0; e < 8; ++e) wg[s][e] = (T)((float)g[e] * -kLog2e);
      wo[s] = ldg<V8>(Wo + frow + 16 * s + 8 * hl);
    }
    // (clamped: exp2 saturates long before, and the 16-bit parts of a larger value could overflow)
    const float cb = fminf(fmaxf(bg ? -kLog2e * (float)bg[32 * fset + prow] : 0.f, -3e4f), 3e4f);
    const T bhi = (T)cb, blo = (T)(cb - (float)bhi);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gb_a[e] = hl == 0 && e == 0 ? bhi : (hl == 0 && e == 1 ? blo : (T)0.f);
      one_b[e] = (T)((hl == 0 && e < 2) ? 1.f : 0.f);
      ob_a[e] = hl == 0 && e == 0 && bo ? bo[32 * fset + prow] : (T)0.f;  // bo (16-bit) as W_o's bias k-step
    }
  }

  auto swz = [](int t, int chunk) { return (chunk ^ row_key<C>(t)) << 4; };
  const int f0 = 32 * fset + 16 * hl;
  // GEMM 1, sigmoid gate, o * gate -> in place over the o tile (all waves)
  auto compute1 = [&]() {
    const int tok = 32 * sub + col;
    const char* grow = &gs[tok * ROW];
    char* orow = &ots[tok * ROW];
    f32x16 acc = Mma<T>::m32(gb_a, one_b, f32x16{});
#pragma unroll
    for (int k = 0; k < KS; ++k)
      acc = Mma<T>::m32(wg[k], *reinterpret_cast<const V8*>(grow + swz(tok, 2 * k + hl)), acc);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = f0 / 8 + h;
      V8* p = reinterpret_cast<V8*>(orow + swz(tok, c));
      const V8 ov = *p;
      V8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float gate = __builtin_amdgcn_rcpf(1.0f + fast_exp2(acc[8 * h + e]));
        r[e] = (T)((float)ov[e] * gate);
      }
      *p = r;
    }
  };
  // GEMM 2 on the gated tile -> token-major output tile (all waves)
  auto compute2 = [&]() {
    const int tok = 32 * sub + col;
    const char* trow = &ots[tok * ROW];
    f32x16 acc = Mma<T>::m32(ob_a, one_b, f32x16{});
#pragma unroll
    for (int k = 0; k < KS; ++k)
      acc = Mma<T>::m32(wo[k], *reinterpret_cast<const V8*>(trow + swz(tok, 2 * k + hl)), acc);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      V8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = (T)acc[8 * h + e];
      const int c = f0 / 8 + h;
      *reinterpret_cast<V8*>(&os[tok * C + ((c ^ row_key<C>(tok)) << 3)]) = r;
    }
  };

  const uint32_t G = gridDim.x;
  uint32_t t = blockIdx.x;
  if (wave < 4) {
    // ================= loaders =================
    const int ch = tid % LPT;  // this thread's 16-byte chunk of every token row it loads
    V8 lnw = {}, lnb = {};
    if constexpr (LN) {
      lnw = ldg<V8>(w_ln + 8 * ch);
      if (b_ln) lnb = ldg<V8>(b_ln + 8 * ch);
    }
    struct Stage {
      V8 g[4];
    };
    // same loads on every call (past the end: the last tile; tokens >= M read token M - 1)
    auto fetch = [&](uint32_t tt, Stage& sg) {
      tt = tt < ntiles ? tt : ntiles - 1;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t m = tt * TOK + (k * NL + tid) / LPT;
        m = m < M ? m : M - 1;
        const uint32_t m1 = M2.div(m), m2 = m - m1 * M2.d;
        sg.g[k] = ldg<V8>(gin + m1 * sg0 + m2 * sg1 + 8 * ch);
      }
    };
    auto step = [&](uint32_t tt, Stage& sg) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int tk = (k * NL + tid) / LPT;
        V8 g = sg.g[k];
        if constexpr (LN) {  // LayerNorm over the token's LPT lanes (sum and sum of squares in fp32)
          float s1 = 0.f, s2 = 0.f;
          const V2 one = {(T)1.f, (T)1.f};
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const V2 pr = {g[e], g[e + 1]};
            s1 = Mma<T>::dot2(pr, one, s1);
            s2 = Mma<T>::dot2(pr, pr, s2);
          }
          const float mean = group_sum<LPT>(s1) * (1.0f / C);
          const float var = fmaxf(group_sum<LPT>(s2) * (1.0f / C) - mean * mean, 0.f);
          const float rstd = rsqrtf(var + ln_eps);
#pragma unroll
          for (int e = 0; e < 8; ++e) g[e] = (T)(((float)g[e] - mean) * rstd * (float)lnw[e] + (float)lnb[e]);
        }
        *reinterpret_cast<V8*>(&gs[tk * ROW + swz(tk, ch)]) = g;
      }
      __syncthreads();
      fetch(tt + PD * G, sg);  // refill this stage
      __builtin_amdgcn_sched_barrier(0);
      compute1();
      __syncthreads();
      compute2();
      __syncthreads();
    };
    Stage s0, s1;
    fetch(t, s0);
    __builtin_amdgcn_sched_barrier(0);  // keep the stages' loads in issue order
    fetch(t + G, s1);
    __builtin_amdgcn_sched_barrier(0);
    // block-uniform trip count (barriers match the writers'); the odd last tile runs after the
    // loop so that the back edge is the only way to the loop head (a break out of the unrolled
    // body would merge into the latch and make the compiler wait for every load)
    uint32_t n = t < ntiles ? (ntiles - t + G - 1) / G : 0;
    for (; n >= 2; n -= 2, t += 2 * G) {
      step(t, s0);
      step(t + G, s1);
    }
    if (n > 0) step(t, s0);
  } else {
    // ================= writers: also fetch o two tiles ahead and stage it =================
    const int wt = tid - NL;
    const int wch = wt % LPT;
    struct OStage {
      V8 o[4];
    };
    auto ofetch = [&](uint32_t tt, OStage& sg) {
      tt = tt < ntiles ? tt : ntiles - 1;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t m = tt * TOK + (k * NL + wt) / LPT;
        m = m < M ? m : M - 1;
        const uint32_t m1 = M2.div(m), m2 = m - m1 * M2.d;
        sg.o[k] = ldg<V8>(o + m1 * so0 + m2 * so1 + 8 * wch);
      }
    };
    auto wstore = [&](uint32_t tt) {
#pragma unroll
      for (int k = 0; k < TOK * C / 8 / NL; ++k) {
        const int ci = k * NL + wt;  // token ci / LPT, chunk ci % LPT
        const int tk = ci / LPT, c = ci % LPT;
        const uint32_t m = tt * TOK + tk;
        if (m >= M) continue;
        V8 v = *reinterpret_cast<const V8*>(&os[tk * C + ((c ^ row_key<C>(tk)) << 3)]);
        if constexpr (RES) {
          const uint32_t m1 = M2.div(m), m2 = m - m1 * M2.d;
          const V8 r = ldg<V8>(res + m1 * sr0 + m2 * sr1 + 8 * c);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (T)((float)r[e] + (float)v[e]);
          stg<V8>(out + m1 * sd0 + m2 * sd1 + 8 * c, v);
        } else {
          stg<V8>(out + (int64_t)m * C + 8 * c, v);
        }
      }
    };
    auto wstep = [&](uint32_t tt, OStage& sg) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int tk = (k * NL + wt) / LPT;
        *reinterpret_cast<V8*>(&ots[tk * ROW + swz(tk, wch)]) = sg.o[k];
      }
      __syncthreads();  // tile staged
      ofetch(tt + PD * G, sg);  // refill this stage
      __builtin_amdgcn_sched_barrier(0);
      compute1();
      __syncthreads();  // gated tile complete
      compute2();
      __syncthreads();  // output tile complete
      wstore(tt);
    };
    OStage o0, o1;
    ofetch(t, o0);
    __builtin_amdgcn_sched_barrier(0);
    ofetch(t + G, o1);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t n = t < ntiles ? (ntiles - t + G - 1) / G : 0;
    for (; n >= 2; n -= 2, t += 2 * G) {
      wstep(t, o0);
      wstep(t + G, o1);
    }
    if (n > 0) wstep(t, o0);
  }
}

template <typename T, int C>
static int gate_out_t(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                      const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg, const void* bg,
                      const void* Wo, const void* bo, const void* res, int64_t sr0, int64_t sr1, void* out,
                      int64_t sd0, int64_t sd1, int64_t M1, int64_t M2, hipStream_t st) {
  constexpr int64_t TOK = 8192 / C;
  const int64_t M = M1 * M2;
  const int64_t ntiles = (M + TOK - 1) / TOK;
  if (ntiles == 0) return TOPS_OK;
  const int64_t grid = ntiles < (int64_t)num_cus() ? ntiles : (int64_t)num_cus();
  auto kern = apply_ln ? (res ? gate_out_kernel<T, true, true, C> : gate_out_kernel<T, true, false, C>)
                       : (res ? gate_out_kernel<T, false, true, C> : gate_out_kernel<T, false, false, C>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(512), 0, st, (const T*)o, so0, so1, (const T*)gin, sg0, sg1,
                     (const T*)w_ln, (const T*)b_ln, ln_eps, (const T*)Wg, (const T*)bg, (const T*)Wo,
                     (const T*)bo, (const T*)res, sr0, sr1, (T*)out, sd0, sd1, FastDiv((uint32_t)M2), (uint32_t)M,
                     (uint32_t)ntiles);
  return launched(res ? "tops_gate_out_residual" : "tops_gate_out");
}

template <typename T, typename... A>
static int gate_out_c(int64_t C, A... a) {
  return C == 128 ? gate_out_t<T, 128>(a...) : gate_out_t<T, 64>(a...);
}

}  // namespace tops

using namespace tops;

extern "C" int tops_gate_out(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                             const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg,
                             const void* bg, const void* Wo, const void* bo, void* out, int64_t M1, int64_t M2,
                             int64_t C, int dtype, void* stream) {
  TOPS_REQUIRE(o && gin && Wg && Wo && out, "tops_gate_out: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_gate_out: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(C == 128 || C == 64, "tops_gate_out: C must be 128 or 64 (got %lld)", (long long)C);
  TOPS_REQUIRE(M1 >= 0 && M2 >= 0 && M1 * M2 < (1LL << 31), "tops_gate_out: bad sizes");
  TOPS_REQUIRE(so0 % 8 == 0 && so1 % 8 == 0 && sg0 % 8 == 0 && sg1 % 8 == 0,
               "tops_gate_out: token strides must be multiples of 8 elements");
  TOPS_REQUIRE((uintptr_t)o % 16 == 0 && (uintptr_t)gin % 16 == 0 && (uintptr_t)out % 16 == 0,
               "tops_gate_out: o, gin and out must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return gate_out_c<__bf16>(C, o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, nullptr, 0, 0,
                              out, 0, 0, M1, M2, st);
  if (dtype == TOPS_DTYPE_F16)
    return gate_out_c<_Float16>(C, o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, nullptr, 0,
                                0, out, 0, 0, M1, M2, st);
  return fail(TOPS_EUNSUPPORTED, "tops_gate_out: unsupported dtype code %d", dtype);
}

extern "C" int tops_gate_out_residual(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0,
                                      int64_t sg1, const void* w_ln, const void* b_ln, float ln_eps, int apply_ln,
                                      const void* Wg, const void* bg, const void* Wo, const void* bo, const void* res,
                                      int64_t sr0, int64_t sr1, void* out, int64_t sd0, int64_t sd1, int64_t M1,
                                      int64_t M2, int64_t C, int dtype, void* stream) {
  TOPS_REQUIRE(o && gin && Wg && Wo && res && out, "tops_gate_out_residual: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_gate_out_residual: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(C == 128 || C == 64, "tops_gate_out_residual: C must be 128 or 64 (got %lld)", (long long)C);
  TOPS_REQUIRE(M1 >= 0 && M2 >= 0 && M1 * M2 < (1LL << 31), "tops_gate_out_residual: bad sizes");
  TOPS_REQUIRE(so0 % 8 == 0 && so1 % 8 == 0 && sg0 % 8 == 0 && sg1 % 8 == 0 && sr0 % 8 == 0 && sr1 % 8 == 0 &&
                   sd0 % 8 == 0 && sd1 % 8 == 0,
               "tops_gate_out_residual: token strides must be multiples of 8 elements");
  TOPS_REQUIRE((uintptr_t)o % 16 == 0 && (uintptr_t)gin % 16 == 0 && (uintptr_t)res % 16 == 0 &&
                   (uintptr_t)out % 16 == 0,
               "tops_gate_out_residual: o, gin, res and out must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return gate_out_c<__bf16>(C, o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, res, sr0, sr1,
                              out, sd0, sd1, M1, M2, st);
  if (dtype == TOPS_DTYPE_F16)
    return gate_out_c<_Float16>(C, o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, res, sr0,
                                sr1, out, sd0, sd1, M1, M2, st);
  return fail(TOPS_EUNSUPPORTED, "tops_gate_out_residual: unsupported dtype code %d", dtype);
}
