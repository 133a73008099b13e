// triangle_multiplicative_update on gfx950: three launches.
//
//   tmu_in_kernel    LN_in + gated projection (P, G) + pair mask, written channel-major
//                    ("D-major") so every channel is an L x L matrix for the einsum.
//                    Incoming writes the token grid transposed, so the einsum is always
//                    y = A . B^T with k contiguous in both operands.
//   tmu_einsum       batched bf16/f16 MFMA GEMM, one slab per channel: y = A . B^T
//                    (256 x 256 tiles for L > 384, persistent when L % 256 == 0; 128 x 128
//                    tiles below).
//   tmu_out_kernel   LN_out(y) . Wp^T gated by sigmoid(LN_in(x) . Wg^T), token-major output.
//
// Reference: triangle_mul/kernel.py:54-162 (fused LN + gated projection), :235-326 (phase
// launchers) and triangle_mul/module.py:80-84 (einsum).  The LayerNorm affines are folded
// into the weights at precompute time exactly as in _common/ln_absorption.py:28-44:
//   LN(x) . W^T = rstd * (x . Wc^T - mean * sum(Wc)) + W . beta.
#include <type_traits>

#include "capi.hpp"
#include "common.hpp"
#include "generic.hpp"

namespace tops {

// scheduling-group masks of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100, kSchedDsWrite = 0x200;

// Token tiles: 64 consecutive positions c of one row r of the (B, L, ld) store grid.
struct GridTile {
  int64_t b, r, c0;
};

__device__ inline GridTile grid_tile(int64_t t, int64_t L, int tiles_per_row) {
  GridTile g;
  g.c0 = (t % tiles_per_row) * 64;
  int64_t rr = t / tiles_per_row;
  g.r = rr % L;
  g.b = rr / L;
  return g;
}

// LayerNorm statistics of a C-element token held as 8 elements by each of 16 consecutive lanes.
// bf16: one pass of packed dot products (sum and sum of squares, fp32 products and sums; 8 instead
// of 16 converts + 24 fp32 ops per lane), variance clamped at 0.  The output phase's loaders use it
// (measured 2 % faster there, and faster than fp32 sums); the input phase, which converts x to fp32
// anyway, takes the same one-pass statistics from fp32 sums (faster there than both).  For
// bf16 (8 significant bits) the fp32 cancellation in E[x^2] - mean^2 has relative error about
// (mean / std)^2 * 2^-22 in the variance, at most 2^-6 where a token's mean exceeds its deviation by
// 2^8, the ratio at which bf16 already quantises the deviation to about one step.  fp16 resolves
// deviations down to mean / std ~ 2^11, where that error would reach 100 %: fp16 takes two passes
// (mean, then the sum of squared deviations), as the reference does (triangle_mul/kernel.py:111-113).
template <typename T, int C>
__device__ inline void ln_stats16(const vec<T, 8>& x, float eps, float& mean, float& rstd) {
  if constexpr (std::is_same<T, _Float16>::value) {
    float v[8], s = 0.f, q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (float)x[e];
      s += v[e];
    }
    mean = group_sum<16>(s) * (1.0f / C);
#pragma unroll
    for (int e = 0; e < 8; ++e) q = fmaf(v[e] - mean, v[e] - mean, q);
    rstd = rsqrtf(group_sum<16>(q) * (1.0f / C) + eps);
  } else {
    const vec<T, 2> one = {(T)1.f, (T)1.f};
    float s = 0.f, q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const vec<T, 2> pr = {x[e], x[e + 1]};
      s = Mma<T>::dot2(pr, one, s);
      q = Mma<T>::dot2(pr, pr, q);
    }
    mean = group_sum<16>(s) * (1.0f / C);
    rstd = rsqrtf(fmaxf(group_sum<16>(q) * (1.0f / C) - mean * mean, 0.f) + eps);
  }
}

// Tile coordinates with scalar divisions (tile indices are wave-uniform).
__device__ inline GridTile grid_tile_fast(uint32_t t, const FastDiv& tpr, const FastDiv& Ld) {
  GridTile g;
  const uint32_t rr = tpr.div(t);
  g.c0 = (int64_t)(t - rr * tpr.d) * 64;
  const uint32_t b = Ld.div(rr);
  g.r = rr - b * Ld.d;
  g.b = b;
  return g;
}

// ---------------------------------------------------------------------------------------------
// Input phase.  64-token tiles (64 consecutive positions c of one row r of the (B, L, ld)
// store grid), 8 waves in two roles:
//   waves 0-3 (loaders) fetch x four tiles ahead (16 lanes per 256-byte token row; positions
//   c >= L reload position L - 1 and get mask 0, so every fetch issues the same loads), take
//   each token's LayerNorm statistics (fp32; one pass of sum and sum of squares for bf16, two
//   passes for fp16, as in ln_stats16) and stage the normalised tile and the mask in LDS
//   (double-buffered);
//   waves 4 .. 4 + NWR - 1 (writers, NWR = C_out / 32) each own 32 output features: P and G weight rows in
//   registers as the MFMA B operand (G's scaled by -log2(e)), D = x . W^T with the A operand read in
//   a permuted token order so each lane ends up with 16 consecutive tokens of one feature (each
//   bias added by one more MFMA k-step, so G's accumulator is the gate's exp2 argument), the gate
//   and mask in the epilogue, and a private feature-major LDS tile
//   that the same wave stores with whole 128-byte rows (8 features x 64 tokens per store
//   instruction).
// No wave has loads and stores in flight together; one barrier per tile, and the loaders'
// LayerNorm of tile n + 1 overlaps the writers' GEMM of tile n.  The LN affine is folded into
// the weights, so the GEMM of the normalised x gives LN(x) . W^T directly.  The loaders also
// publish per tile whether every token is masked (the writers then store zeros without the
// GEMM: padded rows / columns) or every token is valid (no mask multiply); the kernel is
// bound by the writers' vector work (two transcendentals per output for the gate).
// ---------------------------------------------------------------------------------------------
template <typename T, int NWR>
__global__ __launch_bounds__(64 * (4 + NWR)) void tmu_in_kernel(const T* __restrict__ x, const int8_t* __restrict__ mask,
                                                    const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                    const float* __restrict__ Bp, const float* __restrict__ Bg,
                                                    T* __restrict__ ab, int64_t L, int64_t ld, int64_t fstride,
                                                    int transpose, float eps, uint32_t ntiles, FastDiv tpr,
                                                    FastDiv Ld) {
  constexpr int C = 128, ROW = C * 2, KS = C / 16, FW = 32;
  constexpr int PD = 4;  // loader register stages in flight
  using V8 = vec<T, 8>;

  __shared__ __attribute__((aligned(16))) char xs[2][64 * ROW];  // normalised x tiles
  __shared__ __attribute__((aligned(16))) float smask[2][64];
  // per tile and loader wave: bit 0 = some token of the wave's quarter masked, bit 1 = some valid
  __shared__ __attribute__((aligned(16))) int tstate[2][4];
  __shared__ __attribute__((aligned(16))) T os[NWR][FW * 64];   // per writer wave: [feature][token]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // LDS chunk swizzle of a 256-byte token row: distinct for the 16 rows a fragment read touches
  // (the permuted order below visits rows {0-3, 16-19, 4-7, 20-23} + 8 per lane half)
  auto key = [](int t) { return (t & 7) | ((t >> 1) & 8); };
  const uint32_t G = gridDim.x;
  uint32_t t = blockIdx.x;

  if (wave < 4) {
    // ================= loaders =================
    const int ch = tid & 15, tq = tid >> 4;  // 16-byte chunk ch of tokens 16 k + tq, k < 4
    struct Stage {
      V8 x[4];
      int mb[4];  // raw mask bytes, converted when the stage is consumed
    };
    // token of position c0 + d of a tile: tok0 + d * sc (sc = L when incoming, 1 when outgoing);
    // the tile's base is wave-uniform, the lane parts are 32-bit offsets from 24-bit products
    // (d < 64, L * 2C < 2^24: the launcher admits L < 2^15) (no mask: the dummy byte read is x's
    // first)
    const uint32_t sc = transpose ? (uint32_t)L : 1u, msc = mask ? sc : 0u, xsc = sc * (uint32_t)(C * sizeof(T));
    auto fetch = [&](uint32_t tt, Stage& sg) {
      tt = tt < ntiles ? tt : ntiles - 1;
      const GridTile g = grid_tile_fast(tt, tpr, Ld);
      const int64_t tok0 = transpose ? (g.b * L + g.c0) * L + g.r : (g.b * L + g.r) * L + g.c0;
      const char* xb = reinterpret_cast<const char*>(x + tok0 * C);
      const int8_t* mbase = mask ? mask + tok0 : reinterpret_cast<const int8_t*>(x);
      const int lim = (int)(L - 1 - g.c0);  // positions >= L reload position L - 1
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t d = (uint32_t)min(16 * k + tq, lim);
        sg.x[k] = ldg<V8>(xb + (__umul24(d, xsc) + 16u * ch));
        sg.mb[k] = mbase[__umul24(d, msc)];
      }
    };
    auto step = [&](uint32_t tt, int bb, Stage& sg) {
      const GridTile g = grid_tile_fast(tt, tpr, Ld);
      uint64_t zero = 0, valid = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int tk = 16 * k + tq;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)sg.x[k][e];
        float mean, rstd;
        if constexpr (std::is_same<T, _Float16>::value) {  // two passes (see ln_stats16)
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) s += v[e];
          mean = group_sum<16>(s) * (1.0f / C);
          float q = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) q = fmaf(v[e] - mean, v[e] - mean, q);
          rstd = rsqrtf(group_sum<16>(q) * (1.0f / C) + eps);
        } else {  // one pass of fp32 sums (two independent lane reductions)
          float s = 0.f, q = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            s += v[e];
            q = fmaf(v[e], v[e], q);
          }
          s = group_sum<16>(s);
          q = group_sum<16>(q);
          mean = s * (1.0f / C);
          rstd = rsqrtf(fmaxf(q * (1.0f / C) - mean * mean, 0.f) + eps);
        }
        const float nb = -mean * rstd;
        V8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (T)fmaf(v[e], rstd, nb);
        *reinterpret_cast<V8*>(&xs[bb][tk * ROW + ((ch ^ key(tk)) << 4)]) = o;
        // every lane of the token stores the same value: no divergent branch in the loop
        const float mv = g.c0 + tk < L ? (mask ? (float)(sg.mb[k] != 0) : 1.f) : 0.f;
        smask[bb][tk] = mv;
        zero |= __ballot(mv == 0.f);
        valid |= __ballot(mv != 0.f);
      }
      if (lane == 0) tstate[bb][wave] = (zero ? 1 : 0) | (valid ? 2 : 0);
      __syncthreads();  // tile tt staged; the writers are done with the tile before tt - 1
      __builtin_amdgcn_s_setprio(2);
      fetch(tt + PD * G, sg);  // refill this stage
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    };
    const int bb = 0;
    Stage s0, s1, s2, s3;
    fetch(t, s0);
    __builtin_amdgcn_sched_barrier(0);  // keep the stages' loads in issue order
    fetch(t + G, s1);
    __builtin_amdgcn_sched_barrier(0);
    fetch(t + 2 * G, s2);
    __builtin_amdgcn_sched_barrier(0);
    fetch(t + 3 * G, s3);
    __builtin_amdgcn_sched_barrier(0);
    // block-uniform trip count (barriers match the writers'); the remainder runs after the
    // loop so that its back edge is the only way to the loop head (a break out of the
    // unrolled body would merge into the latch and make the compiler wait for every load)
    uint32_t n = t < ntiles ? (ntiles - t + G - 1) / G : 0;
    for (; n >= 4; n -= 4, t += 4 * G) {
      step(t, bb, s0);
      step(t + G, bb ^ 1, s1);
      step(t + 2 * G, bb, s2);
      step(t + 3 * G, bb ^ 1, s3);
    }
    if (n > 0) step(t, bb, s0);
    if (n > 1) step(t + G, bb ^ 1, s1);
    if (n > 2) step(t + 2 * G, bb, s2);
  } else {
    // ================= writers: wave 4 + w owns features [32 w, 32 w + 32) =================
    const int w = wave - 4, hl = lane >> 5, col = lane & 31;
    const int f0 = w * FW;
    V8 wp[KS], wg[KS];
    const int f = f0 + col;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      wp[s] = ldg<V8>(Wp + (int64_t)f * C + 16 * s + 8 * hl);
      // G's rows times -log2(e) (one more 16-bit rounding of the weight), so the accumulator is
      // the gate's exp2 argument: no multiply-add per output (3 % faster, outputs within a bf16
      // step)
      const V8 g = ldg<V8>(Wg + (int64_t)f * C + 16 * s + 8 * hl);
#pragma unroll
      for (int e = 0; e < 8; ++e) wg[s][e] = (T)((float)g[e] * -kLog2e);
    }
    const float cbg2 = -kLog2e * Bg[f];  // gate in the exp2 domain
    // P's bias and G's (-log2(e) Bg) enter through one more MFMA k-step each: A = 1 at k = 0, 1
    // for every token, B = the feature's fp32 bias as two 16-bit parts (hi + lo equal to it
    // within ~2^-16 relative)
    V8 one_a, bias_b, biasg_b;
    {
      const float cbp = Bp[f];
      const T bhi = (T)cbp, blo = (T)(cbp - (float)bhi);
      // (clamped: exp2 saturates long before, and the 16-bit parts of a larger value could overflow)
      const float cg = fminf(fmaxf(cbg2, -3e4f), 3e4f);
      const T ghi = (T)cg, glo = (T)(cg - (float)ghi);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        one_a[e] = (T)((hl == 0 && e < 2) ? 1.f : 0.f);
        bias_b[e] = hl == 0 && e == 0 ? bhi : (hl == 0 && e == 1 ? blo : (T)0.f);
        biasg_b[e] = hl == 0 && e == 0 ? ghi : (hl == 0 && e == 1 ? glo : (T)0.f);
      }
    }
    // token of MFMA row r: 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3), so D slot v of lane
    // half hl is token 16 hl + v of the 32-token sub-tile
    const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);
    T* ow = os[w];
    int bb = 0;
    // the writers issue ahead of the loaders (whose LayerNorm then fills the writers' idle issue
    // slots instead of stretching their first sub-tile: 3-7 % faster, same bits); the loaders'
    // refill fetch goes ahead of both
    __builtin_amdgcn_s_setprio(1);
    for (; t < ntiles; t += G) {
      __syncthreads();  // tile t staged
      // the second writer on each SIMD (waves 8-11 share SIMDs with waves 4-7) starts ~384 cycles
      // later, so one wave's MFMA phase meets the other's gate arithmetic instead of its MFMAs
      // (measured 7-9 % faster at L = 1024, 2-4 % at 2048; a store-phase offset did not help)
      if (w >= 4) __builtin_amdgcn_s_sleep(6);
      // tile state from the loader waves: every token masked (the outputs are exact zeros, no
      // GEMM needed), every token valid (no mask multiply) or mixed
      const int4 ts = *reinterpret_cast<const int4*>(&tstate[bb][0]);
      const int st = ts.x | ts.y | ts.z | ts.w;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int tok = sub * 32 + prow;
        const int tb = sub * 32 + 16 * hl;  // first of this lane's 16 tokens
        {
          V8 o[2];
          if (st == 1) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[0][e] = o[1][e] = (T)0.0f;
          } else {
            f32x16 accP = Mma<T>::m32(one_a, bias_b, f32x16{}), accG = Mma<T>::m32(one_a, biasg_b, f32x16{});
#pragma unroll
            for (int k = 0; k < KS; ++k) {
              const V8 xa = *reinterpret_cast<const V8*>(&xs[bb][tok * ROW + (((2 * k + hl) ^ key(tok)) << 4)]);
              accP = Mma<T>::m32(xa, wp[k], accP);
              accG = Mma<T>::m32(xa, wg[k], accG);
            }
            if (st == 2) {
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const float gate = __builtin_amdgcn_rcpf(1.0f + fast_exp2(accG[v]));
                o[v / 8][v % 8] = (T)(accP[v] * gate);
              }
            } else {
#pragma unroll
              for (int gq = 0; gq < 4; ++gq) {
                const f32x4 rm = *reinterpret_cast<const f32x4*>(&smask[bb][tb + 4 * gq]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  const int v = 4 * gq + j;
                  const float gate = __builtin_amdgcn_rcpf(1.0f + fast_exp2(accG[v]));
                  o[v / 8][v % 8] = (T)(accP[v] * gate * rm[j]);
                }
              }
            }
          }
          // 16-byte chunks c = tb / 8 + {0, 1} of local feature row ff, XOR-swizzled by (ff >> 1) & 7
          const int ff = col;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int c = tb / 8 + h;
            *reinterpret_cast<V8*>(&ow[ff * 64 + ((c ^ ((ff >> 1) & 7)) << 3)]) = o[h];
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // one sub-tile's accumulators live at a time
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const GridTile g = grid_tile_fast(t, tpr, Ld);
      const int64_t rowoff = (g.b * L + g.r) * ld + g.c0;
#pragma unroll
      for (int q = 0; q < FW / 8; ++q) {
        const int ci = q * 64 + lane;  // chunk index: local feature ci / 8, chunk ci % 8
        const int ff = ci >> 3, c = ci & 7;
        const V8 v = *reinterpret_cast<const V8*>(&ow[ff * 64 + ((c ^ ((ff >> 1) & 7)) << 3)]);
        // non-temporal: the 2 C L^2 ab bytes go to HBM now instead of sitting dirty in L2 and the
        // memory-side cache, whose write-back otherwise competes with the einsum's reads of ab
        // (einsum 0.291 -> 0.274 ms after this kernel at L = 1024, this kernel unchanged)
        __builtin_nontemporal_store(v, reinterpret_cast<V8*>(ab + (int64_t)(f0 + ff) * fstride + rowoff + 8 * c));
      }
      bb ^= 1;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Einsum: per slab s, Y = A . B^T with A, B (L x ld) row-major (k contiguous), ld % 64 == 0.
// Block tile BM (i) x BN (j), k-tile 64, NW waves in a 2 x (NW / 2) arrangement (two waves per
// SIMD with NW = 8, so one wave's MFMAs cover the other's LDS reads), double-buffered LDS with
// one barrier per k-tile: the next k-tile goes from registers into the other buffer while the
// last k-steps of this one run.  The MFMA computes D = B_tile . A_tile^T (rows j, columns i)
// with the B-tile rows read in a permuted order, so each lane ends up with 16 consecutive j of
// one row i of Y and writes them as two 16-byte stores.  LDS rows (128 bytes = 8 chunks of
// 16 bytes) are XOR-swizzled by (row >> 1) & 7: 16 consecutive rows read at one chunk column
// hit all 64 banks once.
// ---------------------------------------------------------------------------------------------
template <typename T, int BM, int BN, int NW>
__global__ __launch_bounds__(NW * 64) void tmu_einsum_kernel(const T* __restrict__ A, const T* __restrict__ Bmat,
                                                            T* __restrict__ Y, int64_t L, int64_t ld, int64_t ldy,
                                                            int64_t nslab, int tiles_m, int tiles_n) {
  constexpr int NT = NW * 64;
  constexpr int BK = 64;
  constexpr int WM = BM / 2, WN = BN / (NW / 2);
  constexpr int MI = WM / 32, NJ = WN / 32;
  constexpr int RPP = NT / 8;                   // rows per load pass (8 threads per 128-byte row)
  constexpr int ACH = BM / RPP, BCH = BN / RPP;  // 16-byte chunks per thread per k-tile
  static_assert(ACH * RPP == BM && BCH * RPP == BN, "tile / block shape");
  using V8 = vec<T, 8>;

  __shared__ __attribute__((aligned(16))) T As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) T Bs[2][BN * BK];

  // XCD-aware order: hardware round-robins blocks over the 8 XCDs; give each XCD a
  // contiguous run of logical tiles so the slabs it works on stay in its own L2.
  const int64_t total = nslab * tiles_m * tiles_n;
  int64_t id = blockIdx.x;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  const int64_t slab = id / (tiles_m * tiles_n);
  const int rem = (int)(id % (tiles_m * tiles_n));
  const int tm = rem / tiles_n, tn = rem % tiles_n;

  const int64_t slab_ab = L * ld;
  const T* Ab = A + slab * slab_ab;
  const T* Bb = Bmat + slab * slab_ab;
  T* Yb = Y + slab * L * ldy;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int wm = wave % 2, wn = wave / 2;
  // B-tile row read by MFMA row r = col: D slot v of lane half hl is then j = 16 hl + v
  const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);

  auto swz = [](int row, int chunk) { return (chunk ^ ((row >> 1) & 7)) << 3; };
  const int lc = tid & 7, lr = tid >> 3;  // loader: chunk within the 128-byte row, base row
  V8 ra[ACH], rb[BCH];
  auto gload = [&](int kt) {
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
      int64_t row = (int64_t)tm * BM + lr + RPP * j;
      row = row < L ? row : L - 1;
      ra[j] = ldg<V8>(Ab + row * ld + kt * BK + lc * 8);
    }
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
      int64_t row = (int64_t)tn * BN + lr + RPP * j;
      row = row < L ? row : L - 1;
      rb[j] = ldg<V8>(Bb + row * ld + kt * BK + lc * 8);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
      const int row = lr + RPP * j;
      *reinterpret_cast<V8*>(&As[buf][row * BK + swz(row, lc)]) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
      const int row = lr + RPP * j;
      *reinterpret_cast<V8*>(&Bs[buf][row * BK + swz(row, lc)]) = rb[j];
    }
  };

  f32x16 acc[NJ][MI];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[j][i] = f32x16{};

  auto frags = [&](int buf, int ks, V8* fa, V8* fb) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int row = wm * WM + i * 32 + col;
      fa[i] = *reinterpret_cast<const V8*>(&As[buf][row * BK + swz(row, 2 * ks + hl)]);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int row = wn * WN + j * 32 + prow;
      fb[j] = *reinterpret_cast<const V8*>(&Bs[buf][row * BK + swz(row, 2 * ks + hl)]);
    }
  };

  // Branch-free k-tile body (the last k-tile reloads itself into the unused buffer), scheduled
  // explicitly: fragments of k-step ks + 1 are read from LDS before the MFMAs of ks issue.
  const int nk = (int)((L + BK - 1) / BK);  // k-tiles holding a k < L (the rest of the row is zero)
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    gload(kt + 1 < nk ? kt + 1 : kt);
    V8 fa[2][MI], fb[2][NJ];
    frags(buf, 0, fa[0], fb[0]);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      if (ks + 1 < BK / 16) frags(buf, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i) acc[j][i] = Mma<T>::m32(fb[ks & 1][j], fa[ks & 1][i], acc[j][i]);
      if (ks == BK / 16 - 2) sstore(buf ^ 1);  // that buffer was last read before the barrier
    }
    // schedule: global loads, fragments of step 0, then per step [next fragments | MFMAs]
    __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, ACH + BCH, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, MI + NJ, 0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      if (ks + 1 < BK / 16) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, MI + NJ, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, MI * NJ, 0);
      if (ks == BK / 16 - 2) __builtin_amdgcn_sched_group_barrier(kSchedDsWrite, ACH + BCH, 0);
    }
    __syncthreads();
  }

  // ---- Y[i][j0 .. j0 + 15] per lane: two 16-byte stores (columns [L, ldy) get finite filler) ----
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int64_t ii = (int64_t)tm * BM + wm * WM + i * 32 + col;
    if (ii < L) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t j0 = (int64_t)tn * BN + wn * WN + j * 32 + 16 * hl;
        if (j0 >= ldy) continue;  // ldy % 64 == 0: j0 < ldy implies j0 + 16 <= ldy
        V8 o0, o1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o0[e] = (T)acc[j][i][e];
          o1[e] = (T)acc[j][i][8 + e];
        }
        stg<V8>(Yb + ii * ldy + j0, o0);
        stg<V8>(Yb + ii * ldy + j0 + 8, o1);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Einsum, large L (L > 384; the persistent variant below runs the same pipeline when L % 256 == 0):
// 256 x 256 block tile, 8 waves of 128 x 64 (2 x 4; accumulators in VGPRs, 214 registers, so two
// waves share each SIMD and one issues MFMAs while the other waits), k-tile 64,
// operands copied from HBM / L2 straight into LDS with global_load_lds (no staging registers, no
// LDS store instructions), double-buffered.  One load instruction fills 1 KB of LDS in lane order
// and covers 8 rows x 128 bytes, i.e. 8 whole cache lines: a footprint of half lines (k-tile 32)
// halves the rate at which L2 feeds LDS and leaves the loop load-bound.  Each lane fetches the
// 16-byte chunk that belongs at its LDS position under the fragment reads' XOR swizzle.
// Per k-tile kt (stage kt % 2): k-steps 0-2 run with the next k-step's fragments read alongside;
// then each wave waits for its loads of tile kt + 1 and for its fragment reads, and the block meets
// at one barrier; after it the loads of tile kt + 2 go into the stage just drained, and k-step 3
// runs with tile kt + 1's first fragments read alongside.  The waits and the barrier are written
// out explicitly (the compiler's fence before a barrier would wait for every load in flight), and
// the loads are inline asm, so the compiler adds no waits of its own for them.
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(512) void tmu_einsum_large_kernel(const T* __restrict__ A, const T* __restrict__ Bmat,
                                                         T* __restrict__ Y, int64_t L, int64_t ld, int64_t ldy,
                                                         int64_t nslab, int tiles) {
  constexpr int BM = 256, BK = 64, MI = 4, NJ = 2;
  constexpr int TILE = BM * BK;  // elements of one operand's k-tile (32 KB)
  using V8 = vec<T, 8>;

  // one LDS object per stage and operand (static stage indices: the k-loop is unrolled by two)
  __shared__ __attribute__((aligned(16))) T As0[TILE], As1[TILE];
  __shared__ __attribute__((aligned(16))) T Bs0[TILE], Bs1[TILE];
  auto abuf = [&](auto S) -> T* { return decltype(S)::value == 0 ? As0 : As1; };
  auto bbuf = [&](auto S) -> T* { return decltype(S)::value == 0 ? Bs0 : Bs1; };

  const int64_t total = nslab * tiles * tiles;
  int64_t id = blockIdx.x;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  const int64_t slab = id / (tiles * tiles);
  const int rem = (int)(id % (tiles * tiles));
  const int tm = rem / tiles, tn = rem % tiles;

  const T* Ab = A + slab * L * ld;
  const T* Bb = Bmat + slab * L * ld;
  T* Yb = Y + slab * L * ldy;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, col = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);

  // LDS rows are 128 bytes (8 chunks of 16); physical chunk = logical chunk ^ swz(row).  A fragment
  // reads cover 16 consecutive rows per 16 lanes, B fragment reads the rows prow() picks: both
  // swizzles put the 16 lanes of each group on 16 distinct 16-byte bank groups.
  auto swa = [](int row) { return (row >> 1) & 7; };
  auto swb = [](int row) { return ((row >> 1) & 3) | ((row >> 2) & 4); };

  // loads: wave w < 8, instruction j < 4 fills LDS bytes [(4 w + j) KB, +1 KB) of an operand's
  // tile, lane i writing 16 bytes at m0 + 16 i: row r = 8 (4 w + j) + lane / 8, physical chunk
  // lane % 8 <- logical chunk (lane % 8) ^ swz(r).  Rows past L reload row L - 1 (their products
  // are never stored).
  const int nk = (int)((L + BK - 1) / BK);  // k-tiles holding a k < L (the rest of the row is zero)
  const char* abase = reinterpret_cast<const char*>(Ab + (int64_t)tm * BM * ld);
  const char* bbase = reinterpret_cast<const char*>(Bb + (int64_t)tn * BM * ld);
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 8 * (4 * wave + j) + (lane >> 3), cp = lane & 7;
    const int ra = (int64_t)tm * BM + r < L ? r : (int)(L - 1 - (int64_t)tm * BM);
    const int rb = (int64_t)tn * BM + r < L ? r : (int)(L - 1 - (int64_t)tn * BM);
    aoff[j] = (uint32_t)((ra * ld + 8 * (cp ^ swa(r))) * (int64_t)sizeof(T));
    boff[j] = (uint32_t)((rb * ld + 8 * (cp ^ swb(r))) * (int64_t)sizeof(T));
  }
  auto gload = [&](int kt, auto S) {
    const char* ak = abase + (int64_t)kt * BK * sizeof(T);
    const char* bk = bbase + (int64_t)kt * BK * sizeof(T);
    const uint32_t as = (uint32_t)reinterpret_cast<uintptr_t>(abuf(S)) + (uint32_t)(wave * 4 * 1024);
    const uint32_t bs = (uint32_t)reinterpret_cast<uintptr_t>(bbuf(S)) + (uint32_t)(wave * 4 * 1024);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t va = aoff[j], vb = boff[j], ma = as + 1024 * j, mb = bs + 1024 * j;
      asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(va), "s"(ak), "{m0}"(ma) : "memory");
      asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(vb), "s"(bk), "{m0}"(mb) : "memory");
    }
  };
  struct Frags {
    V8 a[MI], b[NJ];
  };
  // fragment i (j) of k-step ks: row wm 128 + 32 i + col (wn 64 + 32 j + prow); neither swizzle
  // sees the 32 i / 32 j part of the row, so one address per k-step and operand serves all its
  // fragments (four of A, two of B), which sit 4 KiB apart (immediate offsets)
  auto frags = [&](auto S, int ks, Frags& f) {
    const T* as = abuf(S) + (wm * 128 + col) * BK + (((2 * ks + hl) ^ swa(col)) << 3);
    const T* bs = bbuf(S) + (wn * 64 + prow) * BK + (((2 * ks + hl) ^ swb(prow)) << 3);
#pragma unroll
    for (int i = 0; i < MI; ++i) f.a[i] = *reinterpret_cast<const V8*>(as + 32 * i * BK);
#pragma unroll
    for (int j = 0; j < NJ; ++j) f.b[j] = *reinterpret_cast<const V8*>(bs + 32 * j * BK);
  };

  f32x16 acc[NJ][MI];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[j][i] = f32x16{};
  auto mfmas = [&](const Frags& f) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < MI; ++i) acc[j][i] = Mma<T>::m32(f.b[j], f.a[i], acc[j][i]);
  };
  auto interleave = [] {
#pragma unroll
    for (int m = 0; m < 6; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  Frags fa, fb;
  auto tile = [&](int kt, auto S) {
    using N = std::integral_constant<int, 1 - decltype(S)::value>;
    mfmas(fa);
    frags(S, 1, fb);
    interleave();
    mfmas(fb);
    frags(S, 2, fa);
    interleave();
    mfmas(fa);
    frags(S, 3, fb);
    interleave();
    // tile kt + 1 complete for this wave, this wave's reads of stage S done; then the block barrier
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kt + 2 < nk) gload(kt + 2, S);
    mfmas(fb);
    frags(N{}, 0, fa);  // past the last tile: reads stage N's stale contents, never used
    interleave();
  };

  gload(0, std::integral_constant<int, 0>{});
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // tile 0 in LDS
  if (1 < nk) gload(1, std::integral_constant<int, 1>{});
  frags(std::integral_constant<int, 0>{}, 0, fa);
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    tile(kt, std::integral_constant<int, 0>{});
    tile(kt + 1, std::integral_constant<int, 1>{});
  }
  if (kt < nk) tile(kt, std::integral_constant<int, 0>{});

  // ---- Y[i][j0 .. j0 + 15] per lane: two 16-byte stores (columns [L, ldy) get finite filler) ----
  // (lane coordinates recomputed from an opaque copy of the thread index, so they are not kept
  // live across the k-loop)
  unsigned t2 = threadIdx.x;
  asm volatile("" : "+v"(t2));
  const int ecol = (int)(t2 & 31), ehl = (int)((t2 >> 5) & 1);
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int64_t ii = (int64_t)tm * BM + wm * 128 + i * 32 + ecol;
    if (ii < L) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t j0 = (int64_t)tn * BM + wn * 64 + j * 32 + 16 * ehl;
        if (j0 >= ldy) continue;  // ldy % 64 == 0: j0 < ldy implies j0 + 16 <= ldy
        V8 o0, o1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o0[e] = (T)acc[j][i][e];
          o1[e] = (T)acc[j][i][8 + e];
        }
        stg<V8>(Yb + ii * ldy + j0, o0);
        stg<V8>(Yb + ii * ldy + j0 + 8, o1);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Einsum, large L, persistent: the k-tile pipeline of tmu_einsum_large_kernel (the same LDS
// layout, loads and fragment swizzles) with 8 waves of 128 x 64 (2 x 4; accumulators in VGPRs,
// 218 registers, so two waves share each SIMD and one issues MFMAs while the other waits on its
// fragment reads or loads), run by one block per CU over the block tiles blockIdx.x,
// blockIdx.x + gridDim.x, ... without draining between tiles: the last two k-tiles of a tile load
// the next tile's first two, and the tile's output stores are issued while those loads are in
// flight, so neither the next tile's first load nor a block launch is waited for (each cost
// ~2.4 / ~0.6 us per 256 x 256 tile, against ~32 us of k-loop at L = 1024).  The first k-step of
// a tile starts from zero accumulators.  Requires L % 256 == 0 (no row of a block tile lies past
// L) and an even k-tile count (two static stages per tile); with gridDim.x a multiple of 8 block
// tile t stays on XCD t % 8 under the XCD-major tile order.  A k-tile's copy is issued in two
// halves, the A operand right after the barrier and the B operand after the k-step that follows
// (one burst of all eight copy instructions per wave measured 2 % / 6 % slower at L = 1024 / 2048;
// quarters spread further, into the next k-tile, leave the late ones too little time).
// Staggered k order: block tile (tm, tn) takes k-tile kt ^ r at step kt, r = (tm + tn) & (P - 1)
// (P: the largest power of two <= tiles that divides the k-tile count).  The blocks of one slab run
// in step, so in the natural order the P blocks that read one A or B k-slice all miss in L2 on it
// together; with r distinct over those readers (a Latin square over the slab's tiles) they visit the
// slice at distinct steps of one aligned group of P steps, so all but the first find it in L2, and
// no reader comes back to a slice long after the others (a cyclic shift by r instead took as long
// but re-fetched the r slices that wrap around, 1.19x the operand bytes at L = 1024 against 1.007x
// here).  0.266 -> 0.251 ms at L = 1024, 1.806 -> 1.760 at 2048.  The k order is the only change:
// the sum over k is associated per k-tile in this order.
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(512) void tmu_einsum_persist_kernel(const T* __restrict__ A, const T* __restrict__ Bmat,
                                                                T* __restrict__ Y, int64_t L, int64_t ld, int64_t ldy,
                                                                int64_t nslab, int tiles) {
  constexpr int BM = 256, BK = 64, MI = 4, NJ = 2;
  constexpr int TILE = BM * BK;
  using V8 = vec<T, 8>;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  __shared__ __attribute__((aligned(16))) T As0[TILE], As1[TILE];
  __shared__ __attribute__((aligned(16))) T Bs0[TILE], Bs1[TILE];
  // per wave: 32 rows x 64 columns of its output slice on the way to HBM (the rest of the 160 KiB)
  __shared__ __attribute__((aligned(16))) T Os[8][32 * 64];
  auto abuf = [&](auto S) -> T* { return decltype(S)::value == 0 ? As0 : As1; };
  auto bbuf = [&](auto S) -> T* { return decltype(S)::value == 0 ? Bs0 : Bs1; };

  // tile counts fit 32 bits (checked by the launcher): 32-bit index arithmetic
  const uint32_t total = (uint32_t)(nslab * tiles * tiles);
  const uint32_t tt = (uint32_t)tiles * (uint32_t)tiles;
  // block tile t -> (slab, tm, tn), XCD-major (tiles of one XCD contiguous)
  auto coords = [&](uint32_t t, int64_t& slab, int& tm, int& tn) {
    uint32_t id = t;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    slab = (int64_t)(id / tt);
    const uint32_t rem = id % tt;
    tm = (int)(rem / (uint32_t)tiles);
    tn = (int)(rem % (uint32_t)tiles);
  };

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, col = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;  // 8 waves: 2 x 4 of 128 x 64
  const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);
  auto swa = [](int row) { return (row >> 1) & 7; };
  auto swb = [](int row) { return ((row >> 1) & 3) | ((row >> 2) & 4); };

  const int nk = (int)((L + BK - 1) / BK);  // k-tiles holding a k < L (the rest of the row is zero)
  // loads: wave w < 8, instruction j < 4 fills LDS bytes [(4 w + j) KB, +1 KB) of an operand's
  // tile, lane i writing 16 bytes at m0 + 16 i: row r = 8 (4 w + j) + i / 8, physical chunk i % 8
  // <- logical chunk (i % 8) ^ swz(r).  L % 256 == 0, so every block tile's rows lie inside its
  // slab: the lane offsets are the same for every tile, only the scalar bases change.
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 8 * (4 * wave + j) + (lane >> 3), cp = lane & 7;
    aoff[j] = (uint32_t)((r * ld + 8 * (cp ^ swa(r))) * (int64_t)sizeof(T));
    boff[j] = (uint32_t)((r * ld + 8 * (cp ^ swb(r))) * (int64_t)sizeof(T));
  }
  const char* abase;
  const char* bbase;
  int rot = 0;  // k order of the block tile being loaded: k-tile kt ^ rot at step kt
  int rmask = 0;  // P - 1
  while (2 * (rmask + 1) <= tiles && nk % (2 * (rmask + 1)) == 0) rmask = 2 * rmask + 1;
  auto setup = [&](uint32_t t) {
    int64_t slab;
    int tm, tn;
    coords(t, slab, tm, tn);
    abase = reinterpret_cast<const char*>(A + (slab * L + (int64_t)tm * BM) * ld);
    bbase = reinterpret_cast<const char*>(Bmat + (slab * L + (int64_t)tn * BM) * ld);
    rot = (tm + tn) & rmask;
  };
  // operand part: 0 = A, 1 = B, 2 = both
  auto gload = [&](int kt, auto S, int part = 2) {
    const int pk = kt ^ rot;  // < nk: rmask + 1 divides nk
    const char* ak = abase + (int64_t)pk * BK * sizeof(T);
    const char* bk = bbase + (int64_t)pk * BK * sizeof(T);
    const uint32_t as = (uint32_t)reinterpret_cast<uintptr_t>(abuf(S)) + (uint32_t)(wave * 4 * 1024);
    const uint32_t bs = (uint32_t)reinterpret_cast<uintptr_t>(bbuf(S)) + (uint32_t)(wave * 4 * 1024);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t va = aoff[j], vb = boff[j], ma = as + 1024 * j, mb = bs + 1024 * j;
      if (part != 1) asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(va), "s"(ak), "{m0}"(ma) : "memory");
      if (part != 0) asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(vb), "s"(bk), "{m0}"(mb) : "memory");
    }
  };
  struct Frags {
    V8 a[MI], b[NJ];
  };
  // fragment i (j) of k-step ks: row wm 128 + 32 i + col (wn 64 + 32 j + prow); neither swizzle
  // sees the 32 i / 32 j part of the row, so one address per k-step and operand serves all its
  // fragments (four of A, two of B), which sit 4 KiB apart (immediate offsets)
  auto frags = [&](auto S, int ks, Frags& f) {
    const T* as = abuf(S) + (wm * 128 + col) * BK + (((2 * ks + hl) ^ swa(col)) << 3);
    const T* bs = bbuf(S) + (wn * 64 + prow) * BK + (((2 * ks + hl) ^ swb(prow)) << 3);
#pragma unroll
    for (int i = 0; i < MI; ++i) f.a[i] = *reinterpret_cast<const V8*>(as + 32 * i * BK);
#pragma unroll
    for (int j = 0; j < NJ; ++j) f.b[j] = *reinterpret_cast<const V8*>(bs + 32 * j * BK);
  };

  f32x16 acc[NJ][MI];
  auto mfmas = [&](const Frags& f, auto first) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < MI; ++i)
        acc[j][i] = Mma<T>::m32(f.b[j], f.a[i], decltype(first)::value ? f32x16{} : acc[j][i]);
  };
  auto interleave = [] {
#pragma unroll
    for (int m = 0; m < 6; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  const uint32_t G = gridDim.x;
  Frags fa, fb;
  uint32_t t = blockIdx.x;
  bool has_next = false;
  // stores_out: the previous block tile's 16 output stores per wave were issued after this k-tile's
  // loads; vector memory operations count down in issue order (the compiler's own waits assume the
  // same), so vmcnt(16) waits for the loads alone and the stores drain during this k-tile
  // (0.263 -> 0.261 ms at L = 1024, same bits)
  auto ktile = [&](int kt, auto S, auto first, bool stores_out = false) {
    using N = std::integral_constant<int, 1 - decltype(S)::value>;
    using NO = std::false_type;
    mfmas(fa, first);
    frags(S, 1, fb);
    interleave();
    mfmas(fb, NO{});
    frags(S, 2, fa);
    interleave();
    mfmas(fa, NO{});
    frags(S, 3, fb);
    interleave();
    if (stores_out)
      asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // the copy of k-tile kt + 2 into the stage just drained: A now, B after this k-step's MFMAs
    int lk = -1;
    if (kt + 2 < nk) {
      lk = kt + 2;
    } else if (has_next) {  // the next block tile's k-tiles 0 and 1
      if (kt + 2 == nk) setup(t + G);
      lk = kt + 2 - nk;
    }
    if (lk >= 0) gload(lk, S, 0);
    mfmas(fb, NO{});
    frags(N{}, 0, fa);  // after the block's last k-tile: stale contents, never used
    interleave();
    if (lk >= 0) gload(lk, S, 1);
  };

  setup(t);
  gload(0, S0{});
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if (1 < nk) gload(1, S1{});
  frags(S0{}, 0, fa);
  for (; t < total; t += G) {
    has_next = t + G < total;
    ktile(0, S0{}, std::true_type{}, t != blockIdx.x);
    ktile(1, S1{}, std::false_type{});
    for (int kt = 2; kt < nk; kt += 2) {
      ktile(kt, S0{}, std::false_type{});
      ktile(kt + 1, S1{}, std::false_type{});
    }
    // ---- the wave's 128 x 64 slice of Y through its LDS buffer, 32 rows at a time: lane (c, h)
    // ---- writes its 16 columns of row c of each 32-row group (chunks 4 j + 2 h, + 1 of the row's
    // ---- 8, XOR-swizzled by (row >> 1) & 7: conflict-free), then each group of 8 lanes reads one
    // ---- whole 128-byte row segment back and stores it (L % 256 == 0: every row and column of
    // ---- the block tile lies inside Y) ----
    int64_t slab;
    int tm, tn;
    coords(t, slab, tm, tn);
    T* Yw = Y + slab * L * ldy + (int64_t)(tm * BM + wm * 128) * ldy + tn * BM + wn * 64;
    T* ob = Os[wave];
    unsigned t2 = threadIdx.x;
    asm volatile("" : "+v"(t2));
    const int ecol = (int)(t2 & 31), ehl = (int)((t2 >> 5) & 1);
    const int rrow = (int)((t2 & 63) >> 3), rch = (int)(t2 & 7);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        V8 o0, o1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o0[e] = (T)acc[j][i][e];
          o1[e] = (T)acc[j][i][8 + e];
        }
        const int c0 = 4 * j + 2 * ehl, sw = (ecol >> 1) & 7;
        *reinterpret_cast<V8*>(&ob[ecol * 64 + ((c0 ^ sw) << 3)]) = o0;
        *reinterpret_cast<V8*>(&ob[ecol * 64 + (((c0 + 1) ^ sw) << 3)]) = o1;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 8 * q + rrow;
        const V8 v = *reinterpret_cast<const V8*>(&ob[r * 64 + ((rch ^ ((r >> 1) & 7)) << 3)]);
        // non-temporal: Y is read back only by the output phase (0.257 -> 0.253 ms at L = 1024)
        __builtin_nontemporal_store(v, reinterpret_cast<V8*>(Yw + (int64_t)(i * 32 + r) * ldy + 8 * rch));
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Einsum in fp32 (fp32 I/O): the same Y = A . B^T per slab on the fp32 MFMA
// (v_mfma_f32_32x32x2_f32: fp32 products, fp32 sums).  128 x 128 block tile, 4 waves of 64 x 64
// (2 x 2 MFMA tiles), k-tiles of 32 register-staged into double-buffered LDS, one barrier per
// k-tile.  Within a k-tile, MFMA k-step s (of 16) pairs k = s in lane half 0 with k = s + 16 in
// lane half 1 (any k order applied to both operands gives the same product), so each lane's
// operand values of a tile are 16 consecutive floats of one row: four 16-byte LDS reads per
// fragment.  LDS rows are padded to 36 floats (the 32 rows of a fragment read spread over the
// banks).  Rows >= L read as zeros; k < round_up(L, 64) is read (the columns [L, ld) are zeros).
// ---------------------------------------------------------------------------------------------
constexpr int kF32Row = 36;  // LDS floats per 32-float k-tile row

__global__ __launch_bounds__(256, 2) void tmu_einsum_f32_kernel(const float* __restrict__ A,
                                                               const float* __restrict__ Bm, float* __restrict__ Y,
                                                               int64_t L, int64_t ld, int64_t ldy, int tiles) {
  constexpr int TM = 128, TK = 32;
  __shared__ __attribute__((aligned(16))) float as[2][TM * kF32Row];
  __shared__ __attribute__((aligned(16))) float bs[2][TM * kF32Row];
  const int64_t slab = blockIdx.x / ((int64_t)tiles * tiles);
  const int rem = (int)(blockIdx.x % ((int64_t)tiles * tiles));
  const int tm = rem / tiles, tn = rem % tiles;
  const float* Ab = A + slab * L * ld;
  const float* Bb = Bm + slab * L * ld;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, hl = lane >> 5, col = lane & 31;
  const int nkt = (int)((L + 63) / 64 * 64 / TK);

  // global -> registers: thread t moves the 16-byte chunks c = t + 256 i (i < 4) of each operand
  // tile, row c / 8, floats 4 (c % 8) .. + 3: eight lanes per 128-byte row
  f32x4 ra[4], rb[4];
  auto gload = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, r = c >> 3, p = c & 7;
      const int64_t ia = (int64_t)tm * TM + r, ib = (int64_t)tn * TM + r;
      ra[i] = ia < L ? ldg<f32x4>(Ab + ia * ld + (int64_t)kt * TK + 4 * p) : f32x4{};
      rb[i] = ib < L ? ldg<f32x4>(Bb + ib * ld + (int64_t)kt * TK + 4 * p) : f32x4{};
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, r = c >> 3, p = c & 7;
      *reinterpret_cast<f32x4*>(&as[buf][r * kF32Row + 4 * p]) = ra[i];
      *reinterpret_cast<f32x4*>(&bs[buf][r * kF32Row + 4 * p]) = rb[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x16{};
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt) gload(kt + 1);
    f32x4 fa[2][4], fb[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        fa[mi][q] = *reinterpret_cast<const f32x4*>(&as[buf][(wm * 64 + 32 * mi + col) * kF32Row + 16 * hl + 4 * q]);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        fb[ni][q] = *reinterpret_cast<const f32x4*>(&bs[buf][(wn * 64 + 32 * ni + col) * kF32Row + 16 * hl + 4 * q]);
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          acc[mi][ni] =
              __builtin_amdgcn_mfma_f32_32x32x2f32(fa[mi][s / 4][s % 4], fb[ni][s / 4][s % 4], acc[mi][ni], 0, 0, 0);
    if (kt + 1 < nkt) lstore(buf ^ 1);  // buf ^ 1 was last read before the previous barrier
    __syncthreads();
  }

  // D slot v of lane (col, hl): row 8 (v / 4) + 4 hl + v % 4, column col of its 32 x 32 tile
  float* Yb = Y + slab * L * ldy;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int64_t j = (int64_t)tn * TM + wn * 64 + 32 * ni + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t i = (int64_t)tm * TM + wm * 64 + 32 * mi + 8 * (v / 4) + 4 * hl + v % 4;
        if (i < L && j < L) Yb[i * ldy + j] = acc[mi][ni][v];
      }
    }
}

// ---------------------------------------------------------------------------------------------
// Output phase (C = C_out = 128).  64-token tiles, 12 waves in two roles:
//   waves 0-3 (loaders) fetch y and x three tiles ahead and stage them in LDS (double-buffered):
//   y (channel-major in HBM) is read 8 lanes per 128-byte channel row and transposed in
//   registers (4 channels x 8 tokens per thread) into a token-major tile, and each loader wave
//   sums y and y^2 of every token over its 32 channels (fp32, reduced across the 8 lanes of a
//   token group with lane swaps); x (token-major) is normalised on the way in (16 lanes per
//   token, `ln_stats16`: one pass for bf16, two for fp16);
//   waves 4-11 (writers) compute features [32 (w & 3), +32) for the 32 tokens [32 (w >> 2), +32)
//   (w = wave - 4) with their Wp / Wg rows in registers (rows permuted so each lane ends up with
//   16 consecutive features of one token), add the loaders' four partial sums of y into its LN
//   statistics and apply them in the epilogue (once per token instead of once per writer wave),
//   and write a token-major output tile (double-buffered); tile n is stored,
//   whole 256-byte rows per 16 lanes, after the barrier of tile n + 1, when every writer has
//   finished it.  One barrier per tile.
// ---------------------------------------------------------------------------------------------
// RES: out = res + result (res in out's layout; the Pairformer residual add fused into the store,
// the sum rounded once, as a separate add would be).
template <typename T, bool RES>
__global__ __launch_bounds__(768) void tmu_out_kernel(const T* __restrict__ y, const T* __restrict__ x,
                                                     const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                     const float* __restrict__ sWp, const float* __restrict__ Bp,
                                                     const float* __restrict__ Bg, const T* __restrict__ res,
                                                     T* __restrict__ out, int64_t L,
                                                     int64_t ldy, int64_t cstride, float eps, uint32_t ntiles,
                                                     FastDiv tpr, FastDiv Ld) {
  constexpr int C = 128, COUT = 128;
  constexpr int ROW = C * 2;  // LDS bytes per token row (16 chunks of 16 bytes)
  constexpr int KS = C / 16;
  constexpr int NL = 256;  // loader threads (waves 0-3); the writers are the other 512
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;

  __shared__ __attribute__((aligned(16))) char ys[2][64 * ROW];  // raw y, token-major
  __shared__ __attribute__((aligned(16))) char xs[2][64 * ROW];  // normalised x
  __shared__ __attribute__((aligned(16))) T os[2][64 * COUT];    // gated output, token-major
  __shared__ __attribute__((aligned(16))) float cst[2][COUT];    // sum(Wp_c), Bp
  // LN statistics of y per token and loader wave: (sum, sum of squares) over the wave's 32 channels
  __shared__ __attribute__((aligned(16))) float2 ystat[2][64][4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < COUT; i += 768) {
    cst[0][i] = sWp[i];
    cst[1][i] = Bp[i];
  }
  __syncthreads();  // cst

  // 16-byte chunk swizzle of a ys row (16 chunks): distinct over any 16 consecutive tokens of an
  // aligned group of 16 (the writers' operand and statistics reads), and distinct in its top three
  // bits over the tokens 8 g + e, g < 8 (the loaders' 8-byte transposed stores, 32 lanes at a
  // time), so neither access pattern puts two lanes of a group on one LDS bank.  (A 3-bit swizzle
  // gave both patterns 2-way conflicts.)
  auto yswz = [](int t) { return (t & 15) ^ ((t >> 3) & 14); };
  const uint32_t G = gridDim.x;
  uint32_t t = blockIdx.x;
  if (wave < 4) {
    // ================= loaders =================
    const int cq = tid >> 3, tg = tid & 7;  // y: channels 4 cq .. 4 cq + 3, tokens 8 tg .. 8 tg + 7
    struct Stage {
      V8 y[4], x[4];
    };
    // same loads on every call (past the end: the last tile; tokens >= L read token L - 1).  Lane
    // parts of the addresses are loop-invariant (y: one 64-bit pointer per channel row; x: token
    // (16 k + tid / 16) of the tile, chunk tid % 16, as 32-bit offsets from the tile's first token)
    const T* yl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) yl[r] = y + (int64_t)(4 * cq + r) * cstride + 8 * tg;
    auto fetch = [&](uint32_t tt, Stage& sg) {
      tt = tt < ntiles ? tt : ntiles - 1;
      const GridTile g = grid_tile_fast(tt, tpr, Ld);
      const int64_t rowbase = g.b * L + g.r;
      const int64_t yoff = rowbase * ldy + g.c0;
#pragma unroll
      for (int r = 0; r < 4; ++r)  // y is read once: non-temporal, so it does not displace x in the caches
        sg.y[r] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(yl[r] + yoff));
      const char* xb = reinterpret_cast<const char*>(x + (rowbase * L + g.c0) * C);
      const int lim = (int)(L - 1 - g.c0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t d = (uint32_t)min(16 * k + (tid >> 4), lim);
        sg.x[k] = ldg<V8>(xb + (d * (uint32_t)(C * sizeof(T)) + 16u * (tid & 15)));
      }
    };
    auto step = [&](int bb, Stage& sg, uint32_t tnext) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // x: LayerNorm (16 lanes per token) -> LDS
        const int ci = k * NL + tid, xt = ci >> 4, ch = ci & 15;
        float mean, rstd;
        ln_stats16<T, C>(sg.x[k], eps, mean, rstd);
        const float nb = -mean * rstd;
        V8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (T)fmaf((float)sg.x[k][e], rstd, nb);
        *reinterpret_cast<V8*>(&xs[bb][xt * ROW + ((ch ^ (xt & 15)) << 4)]) = h;
      }
      float st16[16];  // (sum, sum of squares) of this lane's 4 channels of token 8 tg + e at 2 e, 2 e + 1
#pragma unroll
      for (int e = 0; e < 8; ++e) {  // y: 4 x 8 register transpose -> token-major rows
        const int tk = 8 * tg + e;
        const V4 q4 = {sg.y[0][e], sg.y[1][e], sg.y[2][e], sg.y[3][e]};
        *reinterpret_cast<V4*>(&ys[bb][tk * ROW + (((cq >> 1) ^ yswz(tk)) << 4) + ((cq & 1) << 3)]) = q4;
        float a[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = (float)q4[r];
        st16[2 * e] = (a[0] + a[1]) + (a[2] + a[3]);
        st16[2 * e + 1] = fmaf(a[0], a[0], fmaf(a[1], a[1], fmaf(a[2], a[2], a[3] * a[3])));
      }
      // sum over the 8 lanes that hold token group tg (lane bits 3-5, this wave's 32 channels):
      // each swap-and-add step halves what a lane keeps, so lane bits (5, 4, 3) end with token
      // 4 b5 + 2 b4 + b3 of the group (v_permlane32 / 16_swap exchange the upper half / odd rows of
      // the first operand with the lower half / even rows of the second; DPP row_ror:8 reads l ^ 8)
      float st8[8], st4[4], st2[2];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(st16[i]), __float_as_uint(st16[i + 8]), false, false);
        st8[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(st8[i]), __float_as_uint(st8[i + 4]), false, false);
        st4[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
      const bool b3 = (lane >> 3) & 1;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float keep = b3 ? st4[i + 2] : st4[i], send = b3 ? st4[i] : st4[i + 2];
        st2[i] = keep + dpp<0x128>(send);
      }
      ystat[bb][8 * tg + ((lane >> 3) & 7)][wave] = make_float2(st2[0], st2[1]);
      __syncthreads();  // tile staged
      fetch(tnext, sg);  // refill this stage
      __builtin_amdgcn_sched_barrier(0);
    };
    const int bb = 0;
    Stage s0, s1, s2;
    fetch(t, s0);
    __builtin_amdgcn_sched_barrier(0);  // keep the stages' loads in issue order
    fetch(t + G, s1);
    __builtin_amdgcn_sched_barrier(0);
    fetch(t + 2 * G, s2);
    __builtin_amdgcn_sched_barrier(0);
    // block-uniform trip count (barriers match the writers'); step k uses stage k % 3 and
    // buffer k % 2, so the loop runs rounds of six steps and the remainder follows it (the back
    // edge stays the only way to the loop head)
    uint32_t n = t < ntiles ? (ntiles - t + G - 1) / G : 0;
    for (; n >= 6; n -= 6, t += 6 * G) {
      step(bb, s0, t + 3 * G);
      step(bb ^ 1, s1, t + 4 * G);
      step(bb, s2, t + 5 * G);
      step(bb ^ 1, s0, t + 6 * G);
      step(bb, s1, t + 7 * G);
      step(bb ^ 1, s2, t + 8 * G);
    }
    if (n > 0) step(bb, s0, t + 3 * G);
    if (n > 1) step(bb ^ 1, s1, t + 4 * G);
    if (n > 2) step(bb, s2, t + 5 * G);
    if (n > 3) step(bb ^ 1, s0, t + 6 * G);
    if (n > 4) step(bb, s1, t + 7 * G);
    __syncthreads();  // the writers' final store waits for this
  } else {
    // ================= writers =================
    const int w = wave - 4, hl = lane >> 5, col = lane & 31;
    const int fset = w & 3, sub = w >> 2;
    // A operand row r = col holds feature 32 fset + prow: D slot v of lane half hl is then
    // feature 32 fset + 16 hl + v
    const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);
    // G's rows times -log2(e) and its bias -log2(e) Bg as one more MFMA k-step (A: the row's bias
    // as two 16-bit parts at k = 0, 1; B: 1 there for every token), so the accumulator is the
    // gate's exp2 argument: no multiply-add per output (0.159 -> 0.149 ms at L = 1024, outputs
    // within a bf16 step)
    V8 wp[KS], wg[KS], gb_a, one_b;
    {
      const int64_t frow = (int64_t)(32 * fset + prow) * C;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        wp[s] = ldg<V8>(Wp + frow + 16 * s + 8 * hl);
        const V8 g = ldg<V8>(Wg + frow + 16 * s + 8 * hl);
#pragma unroll
        for (int e = 0; e < 8; ++e) wg[s][e] = (T)((float)g[e] * -kLog2e);
      }
      const float cb = fminf(fmaxf(-kLog2e * Bg[32 * fset + prow], -3e4f), 3e4f);  // as in the input phase
      const T bhi = (T)cb, blo = (T)(cb - (float)bhi);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gb_a[e] = hl == 0 && e == 0 ? bhi : (hl == 0 && e == 1 ? blo : (T)0.f);
        one_b[e] = (T)((hl == 0 && e < 2) ? 1.f : 0.f);
      }
    }
    const int wt = tid - NL;  // store role: 16-byte chunks wt and 512 + wt of the output tile
    auto store = [&](uint32_t tt, int ob) {
      const GridTile g = grid_tile_fast(tt, tpr, Ld);
      const int64_t tok0 = (g.b * L + g.r) * L + g.c0;
#pragma unroll(RES ? 1 : 2)
      for (int k = 0; k < 2; ++k) {
        const int ci = k * 512 + wt;  // token ci / 16, chunk ci % 16
        const int tk = ci >> 4, c = ci & 15;
        if (g.c0 + tk < L) {
          V8 v = *reinterpret_cast<const V8*>(&os[ob][tk * COUT + ((c ^ (tk & 15)) << 3)]);
          if constexpr (RES) {
            const V8 r = ldg<V8>(res + (tok0 + tk) * COUT + 8 * c);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (T)((float)r[e] + (float)v[e]);
          }
          // non-temporal: 2 C L^2 output bytes, beyond what the caches would keep for the next op
          // (0.1594 -> 0.1574 ms in the tmu call sequence at L = 1024)
          __builtin_nontemporal_store(v, reinterpret_cast<V8*>(out + (tok0 + tk) * COUT + 8 * c));
        }
      }
    };
    int bb = 0;
    for (; t < ntiles; t += G) {
      __syncthreads();  // tile t staged; every writer has finished tile t - G
      const int tok = 32 * sub + col;
      const char* yrow = &ys[bb][tok * ROW];
      const char* xrow = &xs[bb][tok * ROW];
      // the gate's GEMM first, then the P GEMM's MFMAs interleaved with the gate's exponentials and
      // reciprocals (which need only accG), so the matrix core and the VALU of this wave work
      // together (3 % faster than the two chains interleaved at L = 1024 and 2048, same results)
      f32x16 accP = {}, accG = Mma<T>::m32(gb_a, one_b, f32x16{});
#pragma unroll
      for (int k = 0; k < KS; ++k)
        accG = Mma<T>::m32(wg[k], *reinterpret_cast<const V8*>(xrow + (((2 * k + hl) ^ (tok & 15)) << 4)), accG);
      __builtin_amdgcn_sched_barrier(0);
      const int f0 = 32 * fset + 16 * hl;
      float gate[16];
#pragma unroll
      for (int k = 0; k < KS; ++k)
        accP = Mma<T>::m32(wp[k], *reinterpret_cast<const V8*>(yrow + (((2 * k + hl) ^ yswz(tok)) << 4)), accP);
#pragma unroll
      for (int v = 0; v < 16; ++v) gate[v] = __builtin_amdgcn_rcpf(1.0f + fast_exp2(accG[v]));
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedValu, 6, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // LN statistics of y for this token: the loader waves' partial sums over 32 channels each
      const float4 p01 = *reinterpret_cast<const float4*>(&ystat[bb][tok][0]);
      const float4 p23 = *reinterpret_cast<const float4*>(&ystat[bb][tok][2]);
      const float mean = ((p01.x + p01.z) + (p23.x + p23.z)) * (1.0f / C);
      const float var = fmaxf(((p01.y + p01.w) + (p23.y + p23.w)) * (1.0f / C) - mean * mean, 0.f);
      const float ra = rsqrtf(var + eps), rb = -mean * ra;
      V8 o[2];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 cs = *reinterpret_cast<const f32x4*>(&cst[0][f0 + 4 * q]);
        const f32x4 cb = *reinterpret_cast<const f32x4*>(&cst[1][f0 + 4 * q]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int v = 4 * q + j;
          const float P = fmaf(accP[v], ra, fmaf(rb, cs[j], cb[j]));
          o[v / 8][v % 8] = (T)(P * gate[v]);
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = f0 / 8 + h;
        *reinterpret_cast<V8*>(&os[bb][tok * COUT + ((c ^ (tok & 15)) << 3)]) = o[h];
      }
      if (t >= (uint32_t)blockIdx.x + G) store(t - G, bb ^ 1);  // previous tile, complete since the barrier
      bb ^= 1;
    }
    __syncthreads();  // the last tile is complete
    if (t >= (uint32_t)blockIdx.x + G) store(t - G, bb ^ 1);
  }
}

template <typename T>
static int tmu_input_phase_t(const void* x, const void* mask, const void* Wp, const void* Wg, const float* Bp,
                             const float* Bg, void* ab, int64_t B, int64_t L, int64_t C_out, int64_t ld, int transpose,
                             float eps, hipStream_t st) {
  const int64_t tpr = ld / 64;
  const int64_t ntiles = B * L * tpr;
  if (ntiles == 0) return TOPS_OK;
  const int64_t fstride = B * L * ld;
  const int64_t grid = ntiles < (int64_t)num_cus() ? ntiles : (int64_t)num_cus();
  const FastDiv tdiv((uint32_t)tpr), ldiv((uint32_t)L);
  if (C_out == 256)
    hipLaunchKernelGGL((tmu_in_kernel<T, 8>), dim3((unsigned)grid), dim3(768), 0, st, (const T*)x,
                       (const int8_t*)mask, (const T*)Wp, (const T*)Wg, Bp, Bg, (T*)ab, L, ld, fstride, transpose, eps,
                       (uint32_t)ntiles, tdiv, ldiv);
  else
    hipLaunchKernelGGL((tmu_in_kernel<T, 4>), dim3((unsigned)grid), dim3(512), 0, st, (const T*)x,
                       (const int8_t*)mask, (const T*)Wp, (const T*)Wg, Bp, Bg, (T*)ab, L, ld, fstride, transpose, eps,
                       (uint32_t)ntiles, tdiv, ldiv);
  return launched("tops_tmu_input_phase");
}

template <typename T>
static int tmu_einsum_t(const void* ab, void* y, int64_t nslab, int64_t L, int64_t ld, int64_t ldy, hipStream_t st) {
  const T* A = (const T*)ab;
  const T* Bm = A + nslab * L * ld;
  if (L > 384) {
    const int t = (int)((L + 255) / 256);
    const int64_t grid = nslab * t * t;
    const int64_t cus = num_cus() / 8 * 8;
    if (L % 256 == 0 && (L / 64) % 2 == 0 && grid < (1LL << 31) && cus >= 8) {
      // persistent: one 8-wave block per CU (a multiple of 8 blocks, so each block stays on one
      // XCD's tiles)
      const int64_t pg = grid < cus ? grid : cus;
      hipLaunchKernelGGL((tmu_einsum_persist_kernel<T>), dim3((unsigned)pg), dim3(512), 0, st, A, Bm, (T*)y, L, ld,
                         ldy, nslab, t);
    } else {
      hipLaunchKernelGGL((tmu_einsum_large_kernel<T>), dim3((unsigned)grid), dim3(512), 0, st, A, Bm, (T*)y, L, ld,
                         ldy, nslab, t);
    }
  } else {
    const int t = (int)((L + 127) / 128);
    const int64_t grid = nslab * t * t;
    hipLaunchKernelGGL((tmu_einsum_kernel<T, 128, 128, 4>), dim3((unsigned)grid), dim3(256), 0, st, A, Bm, (T*)y, L,
                       ld, ldy, nslab, t, t);
  }
  return launched("tops_tmu_einsum");
}

template <typename T>
static int tmu_output_phase_t(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                              const float* Bp, const float* Bg, const void* res, void* out, int64_t B, int64_t L,
                              int64_t ldy, float eps, hipStream_t st) {
  const int64_t tpr = (L + 63) / 64;
  const int64_t ntiles = B * L * tpr;
  if (ntiles == 0) return TOPS_OK;
  const int64_t cstride = B * L * ldy;
  const int64_t grid = ntiles < (int64_t)num_cus() ? ntiles : (int64_t)num_cus();
  const FastDiv tdiv((uint32_t)tpr), ldiv((uint32_t)L);
  if (res)
    hipLaunchKernelGGL((tmu_out_kernel<T, true>), dim3((unsigned)grid), dim3(768), 0, st, (const T*)y, (const T*)x,
                       (const T*)Wp, (const T*)Wg, sWp, Bp, Bg, (const T*)res, (T*)out, L, ldy, cstride, eps,
                       (uint32_t)ntiles, tdiv, ldiv);
  else
    hipLaunchKernelGGL((tmu_out_kernel<T, false>), dim3((unsigned)grid), dim3(768), 0, st, (const T*)y, (const T*)x,
                       (const T*)Wp, (const T*)Wg, sWp, Bp, Bg, (const T*)nullptr, (T*)out, L, ldy, cstride, eps,
                       (uint32_t)ntiles, tdiv, ldiv);
  return launched(res ? "tops_tmu_output_phase_residual" : "tops_tmu_output_phase");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_tmu_input_phase(const void* x, const void* mask, const void* Wp, const void* Wg, const float* sWp,
                                    const float* sWg, const float* Bp, const float* Bg, void* ab, int64_t B, int64_t L,
                                    int64_t C, int64_t C_out, int64_t ld, int transpose, float eps, int dtype,
                                    void* stream) {
  TOPS_REQUIRE(x && Wp && Wg && sWp && sWg && Bp && Bg && ab, "tops_tmu_input_phase: null pointer argument");
  TOPS_REQUIRE(B >= 0 && L >= 0 && ld >= L && ld % 64 == 0,
               "tops_tmu_input_phase: bad sizes B=%lld L=%lld ld=%lld (ld must be a multiple of 64)", (long long)B,
               (long long)L, (long long)ld);
  TOPS_REQUIRE(B * L * (ld / 64) < (1LL << 31), "tops_tmu_input_phase: too many tokens");
  // any-shape kernels (and L >= 2^15, where the tuned kernel's 24-bit lane offsets would not hold)
  if (C != 128 || (C_out != 128 && C_out != 256) || dtype == TOPS_DTYPE_F32 || L >= (1 << 15))
    return tmu_generic_input_phase(x, mask, Wp, Wg, Bp, Bg, ab, B, L, C, C_out, ld, transpose, eps, dtype,
                                   (hipStream_t)stream);
  (void)sWp;  // the kernel normalises x before the GEMM: the column sums of the folded weights
  (void)sWg;  // are part of the ABI (reference layout) but not needed
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tmu_input_phase_t<__bf16>(x, mask, Wp, Wg, Bp, Bg, ab, B, L, C_out, ld, transpose, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return tmu_input_phase_t<_Float16>(x, mask, Wp, Wg, Bp, Bg, ab, B, L, C_out, ld, transpose, eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tmu_input_phase: unsupported dtype code %d", dtype);
}

extern "C" int tops_tmu_einsum(const void* ab, void* y, int64_t nslab, int64_t L, int64_t ld, int64_t ldy, int dtype,
                               void* stream) {
  TOPS_REQUIRE(ab && y, "tops_tmu_einsum: null pointer argument");
  TOPS_REQUIRE(ld % 64 == 0 && ldy % 64 == 0 && ld >= L && ldy >= L && L >= 0 && nslab >= 0,
               "tops_tmu_einsum: bad sizes nslab=%lld L=%lld ld=%lld ldy=%lld (ld, ldy must be multiples of 64)",
               (long long)nslab, (long long)L, (long long)ld, (long long)ldy);
  if (L == 0 || nslab == 0) return TOPS_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_F32) {
    const int t = (int)((L + 127) / 128);
    const int64_t grid = nslab * t * t;
    TOPS_REQUIRE(grid < (1LL << 31), "tops_tmu_einsum: too many tiles");
    const float* A = (const float*)ab;
    hipLaunchKernelGGL(tmu_einsum_f32_kernel, dim3((unsigned)grid), dim3(256), 0, st, A, A + nslab * L * ld, (float*)y,
                       L, ld, ldy, t);
    return launched("tops_tmu_einsum");
  }
  if (dtype == TOPS_DTYPE_BF16) return tmu_einsum_t<__bf16>(ab, y, nslab, L, ld, ldy, st);
  if (dtype == TOPS_DTYPE_F16) return tmu_einsum_t<_Float16>(ab, y, nslab, L, ld, ldy, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tmu_einsum: unsupported dtype code %d", dtype);
}

static int tmu_output_phase_any(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                                const float* sWg, const float* Bp, const float* Bg, const void* res, void* out,
                                int64_t B, int64_t L, int64_t C, int64_t C_out, int64_t ldy, float eps, int dtype,
                                void* stream) {
  TOPS_REQUIRE(y && x && Wp && Wg && sWp && sWg && Bp && Bg && out, "tops_tmu_output_phase: null pointer argument");
  TOPS_REQUIRE(B >= 0 && L >= 0 && ldy >= L && ldy % 64 == 0,
               "tops_tmu_output_phase: bad sizes B=%lld L=%lld ldy=%lld (ldy must be a multiple of 64)",
               (long long)B, (long long)L, (long long)ldy);
  TOPS_REQUIRE(B * L * ((L + 63) / 64) < (1LL << 31), "tops_tmu_output_phase: too many tokens");
  if (C != 128 || C_out != 128 || dtype == TOPS_DTYPE_F32)  // any-shape kernels
    return tmu_generic_output_phase(y, x, Wp, Wg, Bp, Bg, res, out, B, L, C, C_out, ldy, eps, dtype,
                                    (hipStream_t)stream);
  (void)sWg;  // x is normalised before its GEMM: the column sums of Wg_c are not needed
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tmu_output_phase_t<__bf16>(y, x, Wp, Wg, sWp, Bp, Bg, res, out, B, L, ldy, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return tmu_output_phase_t<_Float16>(y, x, Wp, Wg, sWp, Bp, Bg, res, out, B, L, ldy, eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tmu_output_phase: unsupported dtype code %d", dtype);
}

extern "C" int tops_tmu_output_phase(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                                     const float* sWg, const float* Bp, const float* Bg, void* out, int64_t B,
                                     int64_t L, int64_t C, int64_t C_out, int64_t ldy, float eps, int dtype,
                                     void* stream) {
  return tmu_output_phase_any(y, x, Wp, Wg, sWp, sWg, Bp, Bg, nullptr, out, B, L, C, C_out, ldy, eps, dtype, stream);
}

extern "C" int tops_tmu_output_phase_residual(const void* y, const void* x, const void* Wp, const void* Wg,
                                              const float* sWp, const float* sWg, const float* Bp, const float* Bg,
                                              const void* res, void* out, int64_t B, int64_t L, int64_t C,
                                              int64_t C_out, int64_t ldy, float eps, int dtype, void* stream) {
  TOPS_REQUIRE(res, "tops_tmu_output_phase_residual: null residual");
  TOPS_REQUIRE((uintptr_t)res % 16 == 0 || C != 128, "tops_tmu_output_phase_residual: res must be 16-byte aligned");
  return tmu_output_phase_any(y, x, Wp, Wg, sWp, sWg, Bp, Bg, res, out, B, L, C, C_out, ldy, eps, dtype, stream);
}
