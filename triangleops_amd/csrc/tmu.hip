// triangle_multiplicative_update on gfx950: three launches.
//
//   tmu_in_kernel    LN_in + gated projection (P, G) + pair mask, written channel-major
//                    ("D-major") so every channel is an L x L matrix for the einsum.
//                    Incoming writes the token grid transposed, so the einsum is always
//                    y = A . B^T with k contiguous in both operands.
//   tmu_einsum       batched bf16/f16 MFMA GEMM, one slab per channel: y = A . B^T.
//   tmu_out_kernel   LN_out(y) . Wp^T gated by sigmoid(LN_in(x) . Wg^T), token-major output.
//
// Reference: triangle_mul/kernel.py:54-162 (fused LN + gated projection), :235-326 (phase
// launchers) and triangle_mul/module.py:80-84 (einsum).  The LayerNorm affines are folded
// into the weights at precompute time exactly as in _common/ln_absorption.py:28-44:
//   LN(x) . W^T = rstd * (x . Wc^T - mean * sum(Wc)) + W . beta.
#include "capi.hpp"
#include "common.hpp"

namespace tops {

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
// Input phase.  NW waves; wave w owns output features f = 32w + lane%32 of both P and G, with
// its weight rows in registers as the MFMA B operand.  A block walks 64-token tiles in a
// grid-stride loop, with two roles: waves [0, NW/2) fetch x (three tiles ahead, in a ring of
// register stages) and waves [NW/2, NW) write the results, so neither role ever has loads and
// stores outstanding together and the in-order memory counter waits only for the stage being
// consumed.  The loaders normalise each token with its LayerNorm statistics (one pass, fp32,
// packed dot products) on the way into LDS, so the GEMM yields LN(x) . Wc^T directly and the
// epilogue is a bias add and the gate.  The A operand reads tokens in a permuted order so
// that D = x . W^T leaves 16 consecutive tokens of one feature in each lane; the gated result
// goes through a feature-major LDS tile and every store instruction writes whole 128-byte
// rows (8 features x 64 tokens) of the channel-major output.
// ---------------------------------------------------------------------------------------------
template <typename T, int C, int NW>
__global__ __launch_bounds__(NW * 64) void tmu_in_kernel(const T* __restrict__ x, const int8_t* __restrict__ mask,
                                                        const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                        const float* __restrict__ Bp, const float* __restrict__ Bg,
                                                        T* __restrict__ ab, int64_t L, int64_t ld, int64_t fstride,
                                                        int transpose, float eps, uint32_t ntiles, FastDiv tpr,
                                                        FastDiv Ld) {
  constexpr int NT = NW * 64;
  constexpr int NL = NT / 2;          // loader threads
  constexpr int TPT = NL / 64;        // loader threads per token
  constexpr int CPT = (C / 8) / TPT;  // 16-byte chunks per loader thread
  constexpr int ROW = C * 2;          // LDS bytes per token row
  constexpr int KS = C / 16;          // MFMA k-steps
  constexpr int PD = 3;               // register stages in flight
  static_assert(CPT * TPT * 8 == C, "channel split");
  using V8 = vec<T, 8>;
  using V2 = vec<T, 2>;

  __shared__ __attribute__((aligned(16))) char xs[2][64 * ROW];  // normalised x tile
  __shared__ __attribute__((aligned(16))) float smask[2][64];
  __shared__ __attribute__((aligned(16))) T os[NW * 32 * 64];  // gated tile, [feature][token]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int f = wave * 32 + col;

  V8 wp[KS], wg[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    wp[s] = ldg<V8>(Wp + (int64_t)f * C + 16 * s + 8 * hl);
    wg[s] = ldg<V8>(Wg + (int64_t)f * C + 16 * s + 8 * hl);
  }
  const float cbp = Bp[f], cbg2 = -kLog2e * Bg[f];  // gate in the exp2 domain

  // token of MFMA row r: 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3), so D slot v of lane
  // half hl is token 16 hl + v of the 32-token sub-tile
  const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);
  // GEMMs + gate of one staged tile -> feature-major LDS tile (all waves)
  auto compute = [&](int buf) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int tok = sub * 32 + prow;
      f32x16 accP = {}, accG = {};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const V8 xa = *reinterpret_cast<const V8*>(&xs[buf][tok * ROW + (((2 * k + hl) ^ (tok & 7)) << 4)]);
        accP = Mma<T>::m32(xa, wp[k], accP);
        accG = Mma<T>::m32(xa, wg[k], accG);
      }
      const int tb = sub * 32 + 16 * hl;  // first of this lane's 16 tokens
      V8 o[2];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4 rm = *reinterpret_cast<const f32x4*>(&smask[buf][tb + 4 * gq]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int v = 4 * gq + j;
          const float P = accP[v] + cbp;
          const float gate = __builtin_amdgcn_rcpf(1.0f + fast_exp2(fmaf(accG[v], -kLog2e, cbg2)));
          o[v / 8][v % 8] = (T)(P * gate * rm[j]);
        }
      }
      // 16-byte chunks c = tb / 8 + {0, 1} of feature row f, XOR-swizzled by (f >> 1) & 7
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = tb / 8 + h;
        *reinterpret_cast<V8*>(&os[f * 64 + ((c ^ ((f >> 1) & 7)) << 3)]) = o[h];
      }
    }
  };

  const uint32_t G = gridDim.x;
  uint32_t t = blockIdx.x;
  if (wave < NW / 2) {
    // ================= loaders =================
    const int my_tok = tid / TPT, my_part = tid % TPT;
    struct Stage {
      V8 x[CPT];
      int mb;   // raw mask byte and position flag, combined when the stage is consumed so
      bool ok;  // the fetch itself never waits for its loads
    };
    // Every fetch issues the same loads (past the end it reloads the last tile; positions
    // c >= L read token L - 1 and get mask 0), keeping the memory-counter accounting exact.
    auto fetch = [&](uint32_t tt, Stage& sg) {
      tt = tt < ntiles ? tt : ntiles - 1;
      const GridTile g = grid_tile_fast(tt, tpr, Ld);
      int64_t c = g.c0 + my_tok;
      const bool ok = c < L;
      c = ok ? c : L - 1;
      const int64_t i = transpose ? c : g.r, j = transpose ? g.r : c;
      const int64_t tok = (g.b * L + i) * L + j;
      const T* src = x + tok * C + my_part * CPT * 8;
#pragma unroll
      for (int e = 0; e < CPT; ++e) sg.x[e] = ldg<V8>(src + 8 * e);
      sg.mb = *(mask ? mask + tok : reinterpret_cast<const int8_t*>(x));
      sg.ok = ok;
    };
    auto step = [&](uint32_t tt, int buf, Stage& sg) {
      // LayerNorm of this thread's token (sum and sum of squares in fp32) -> LDS
      float s1 = 0.f, s2 = 0.f;
      const V2 one = {(T)1.f, (T)1.f};
#pragma unroll
      for (int e = 0; e < CPT; ++e)
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
          const V2 pr = {sg.x[e][k], sg.x[e][k + 1]};
          s1 = Mma<T>::dot2(pr, one, s1);
          s2 = Mma<T>::dot2(pr, pr, s2);
        }
      const float mean = group_sum<TPT>(s1) * (1.0f / C);
      const float var = fmaxf(group_sum<TPT>(s2) * (1.0f / C) - mean * mean, 0.f);
      const float rstd = rsqrtf(var + eps), shift = -mean * rstd;
#pragma unroll
      for (int e = 0; e < CPT; ++e) {
        V8 h;
#pragma unroll
        for (int k = 0; k < 8; ++k) h[k] = (T)((float)sg.x[e][k] * rstd + shift);
        const int chunk = my_part * CPT + e;
        *reinterpret_cast<V8*>(&xs[buf][my_tok * ROW + ((chunk ^ (my_tok & 7)) << 4)]) = h;
      }
      // every thread of the token stores the same value: no divergent branch in the loop (it
      // would make the compiler wait for all outstanding loads at the loop head)
      smask[buf][my_tok] = sg.ok ? (mask ? (float)sg.mb : 1.f) : 0.f;
      __syncthreads();
      fetch(tt + PD * G, sg);  // refill this stage
      compute(buf);
      __syncthreads();
    };
    int buf = 0;
    Stage s0, s1, s2;
    fetch(t, s0);
    fetch(t + G, s1);
    fetch(t + 2 * G, s2);
    for (; t < ntiles; t += 3 * G) {  // block-uniform trip count: barriers match the writers
      step(t, buf, s0);
      buf ^= 1;
      if (t + G >= ntiles) break;
      step(t + G, buf, s1);
      buf ^= 1;
      if (t + 2 * G >= ntiles) break;
      step(t + 2 * G, buf, s2);
      buf ^= 1;
    }
  } else {
    // ================= writers =================
    const int wt = tid - NL;
    int buf = 0;
    for (; t < ntiles; t += G) {
      __syncthreads();  // tile staged by the loaders
      compute(buf);
      __syncthreads();  // feature-major tile complete
      const GridTile g = grid_tile_fast(t, tpr, Ld);
      const int64_t rowoff = (g.b * L + g.r) * ld + g.c0;
#pragma unroll
      for (int k = 0; k < NW * 32 * 8 / NL; ++k) {
        const int ci = k * NL + wt;  // chunk index: feature ci / 8, chunk ci % 8
        const int ff = ci >> 3, c = ci & 7;
        const V8 v = *reinterpret_cast<const V8*>(&os[ff * 64 + ((c ^ ((ff >> 1) & 7)) << 3)]);
        stg<V8>(ab + (int64_t)ff * fstride + rowoff + 8 * c, v);
      }
      buf ^= 1;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Einsum: per slab s, Y = A . B^T with A, B (L x ld) row-major (k contiguous), ld % 64 == 0.
// Block tile BM x BN, k-tile 64, 4 waves in a 2 x 2 arrangement, double-buffered LDS with the
// 16-byte chunks of each 128-byte row XOR-swizzled by (row & 7) so the MFMA operand reads
// (8 lanes = 8 rows, same chunk) are bank-conflict free.
// ---------------------------------------------------------------------------------------------
template <typename T, int BM, int BN>
__global__ __launch_bounds__(256) void tmu_einsum_kernel(const T* __restrict__ A, const T* __restrict__ Bmat,
                                                        T* __restrict__ Y, int64_t L, int64_t ld, int64_t ldy,
                                                        int64_t nslab, int tiles_m, int tiles_n) {
  constexpr int BK = 64;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MI = WM / 32, NI = WN / 32;
  constexpr int ACH = BM * 8 / 256, BCH = BN * 8 / 256;  // 16-byte chunks per thread per tile
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
  const int wm = wave >> 1, wn = wave & 1;

  const int lc = tid & 7, lr = tid >> 3;  // loader: chunk within the 128-byte row, base row
  V8 ra[ACH], rb[BCH];
  auto gload = [&](int kt) {
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
      int64_t row = (int64_t)tm * BM + lr + 32 * j;
      row = row < L ? row : L - 1;
      ra[j] = ldg<V8>(Ab + row * ld + kt * BK + lc * 8);
    }
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
      int64_t row = (int64_t)tn * BN + lr + 32 * j;
      row = row < L ? row : L - 1;
      rb[j] = ldg<V8>(Bb + row * ld + kt * BK + lc * 8);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < ACH; ++j) {
      const int row = lr + 32 * j;
      *reinterpret_cast<V8*>(&As[buf][row * BK + ((lc ^ (row & 7)) << 3)]) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < BCH; ++j) {
      const int row = lr + 32 * j;
      *reinterpret_cast<V8*>(&Bs[buf][row * BK + ((lc ^ (row & 7)) << 3)]) = rb[j];
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};

  const int nk = (int)(ld / BK);
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      V8 a[MI], b[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int row = wm * WM + i * 32 + col;
        a[i] = *reinterpret_cast<const V8*>(&As[buf][row * BK + (((2 * ks + hl) ^ (row & 7)) << 3)]);
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int row = wn * WN + j * 32 + col;
        b[j] = *reinterpret_cast<const V8*>(&Bs[buf][row * BK + (((2 * ks + hl) ^ (row & 7)) << 3)]);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = Mma<T>::m32(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int64_t cc = (int64_t)tn * BN + wn * WN + j * 32 + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t rr = (int64_t)tm * BM + wm * WM + i * 32 + 8 * (v / 4) + 4 * hl + (v % 4);
        if (rr < L && cc < L) Yb[rr * ldy + cc] = (T)acc[i][j][v];
      }
    }
}

// ---------------------------------------------------------------------------------------------
// Output phase.  4 waves x 32 output features (C_out = 128).  Per 64-token tile the y tile
// (channel-major in HBM) is transposed into a token-major LDS tile, x is staged beside it,
// LN statistics for both are computed from LDS, then each wave runs the two K = C GEMMs
// (P from y, G from x) with its weight rows in registers.
// ---------------------------------------------------------------------------------------------
template <typename T, int C, int COUT>
__global__ __launch_bounds__(256) void tmu_out_kernel(const T* __restrict__ y, const T* __restrict__ x,
                                                     const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                     const float* __restrict__ sWp, const float* __restrict__ sWg,
                                                     const float* __restrict__ Bp, const float* __restrict__ Bg,
                                                     T* __restrict__ out, int64_t L, int64_t ldy, int64_t cstride,
                                                     float eps, int64_t ntiles, int tiles_per_row) {
  static_assert(C == 128 && COUT == 128, "tmu_out_kernel is specialised for C = C_out = 128");
  constexpr int ROW = C * 2;
  constexpr int KS = C / 16;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;

  __shared__ __attribute__((aligned(16))) char ys[64 * ROW];
  __shared__ __attribute__((aligned(16))) char xs[64 * ROW];
  __shared__ float st[4][64];  // mean_y, rstd_y, mean_x, rstd_x

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;

  V8 wp[KS], wg[KS];
  {
    const int64_t frow = (int64_t)(wave * 32 + col) * C;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      wp[s] = ldg<V8>(Wp + frow + 16 * s + 8 * hl);
      wg[s] = ldg<V8>(Wg + frow + 16 * s + 8 * hl);
    }
  }
  float csp[16], cbp[16], csg[16], cbg[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int f = wave * 32 + 8 * (v / 4) + 4 * hl + (v % 4);
    csp[v] = sWp[f];
    cbp[v] = Bp[f];
    csg[v] = sWg[f];
    cbg[v] = Bg[f];
  }

  const bool vec_y = (ldy % 8) == 0;
  // y loader: channels 4*cq .. 4*cq+3, tokens 8*tg .. 8*tg+7 of the tile
  const int cq = tid & 31, tg = tid >> 5;
  // x loader / stats: token tid/4, channels [32*(tid%4), +32)
  const int xt = tid >> 2, xq = tid & 3;

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const GridTile g = grid_tile(tile, L, tiles_per_row);
    const int64_t rowbase = g.b * L + g.r;  // token row (b, i=r); tokens j = c0 + t
    const int nvalid = (int)((L - g.c0) < 64 ? (L - g.c0) : 64);

    // ---- y tile -> LDS (token-major, swizzled) ----
    {
      T yv[4][8];
      const T* ysrc = y + rowbase * ldy + g.c0 + 8 * tg;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const T* p = ysrc + (int64_t)(4 * cq + r) * cstride;
        if (vec_y && 8 * tg + 8 <= nvalid) {
          const V8 v = ldg<V8>(p);
#pragma unroll
          for (int e = 0; e < 8; ++e) yv[r][e] = v[e];
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) yv[r][e] = (8 * tg + e < nvalid) ? p[e] : (T)0.f;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = 8 * tg + e;
        V4 q4 = {yv[0][e], yv[1][e], yv[2][e], yv[3][e]};
        const int chunk = cq >> 1;
        *reinterpret_cast<V4*>(&ys[t * ROW + ((chunk ^ (t & 7)) << 4) + ((cq & 1) << 3)]) = q4;
      }
    }
    // ---- x tile -> LDS ----
    {
      const int64_t tok = rowbase * L + g.c0 + xt;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        V8 v = V8{};
        if (xt < nvalid) v = ldg<V8>(x + tok * C + 32 * xq + 8 * e);
        const int chunk = 4 * xq + e;
        *reinterpret_cast<V8*>(&xs[xt * ROW + ((chunk ^ (xt & 7)) << 4)]) = v;
      }
    }
    __syncthreads();
    // ---- LN statistics (token xt, 4 threads per token) ----
    {
      float vy[32], vx[32];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int chunk = 4 * xq + e;
        const V8 a = *reinterpret_cast<const V8*>(&ys[xt * ROW + ((chunk ^ (xt & 7)) << 4)]);
        const V8 b = *reinterpret_cast<const V8*>(&xs[xt * ROW + ((chunk ^ (xt & 7)) << 4)]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          vy[8 * e + k] = (float)a[k];
          vx[8 * e + k] = (float)b[k];
        }
      }
      float sy = 0.f, sx = 0.f;
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        sy += vy[k];
        sx += vx[k];
      }
      const float my = group_sum<4>(sy) * (1.0f / C), mx = group_sum<4>(sx) * (1.0f / C);
      float qy = 0.f, qx = 0.f;
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        qy += (vy[k] - my) * (vy[k] - my);
        qx += (vx[k] - mx) * (vx[k] - mx);
      }
      qy = group_sum<4>(qy);
      qx = group_sum<4>(qx);
      if (xq == 0) {
        st[0][xt] = my;
        st[1][xt] = rsqrtf(qy * (1.0f / C) + eps);
        st[2][xt] = mx;
        st[3][xt] = rsqrtf(qx * (1.0f / C) + eps);
      }
    }
    __syncthreads();
    // ---- projections + gate ----
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int t = sub * 32 + col;
      f32x16 accP = {}, accG = {};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const int off = t * ROW + (((2 * k + hl) ^ (t & 7)) << 4);
        accP = Mma<T>::m32(wp[k], *reinterpret_cast<const V8*>(&ys[off]), accP);
        accG = Mma<T>::m32(wg[k], *reinterpret_cast<const V8*>(&xs[off]), accG);
      }
      if (t < nvalid) {
        const float my = st[0][t], ry = st[1][t], mx = st[2][t], rx = st[3][t];
        T* dst = out + (rowbase * L + g.c0 + t) * COUT + wave * 32 + 4 * hl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          V4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = 4 * q + e;
            const float P = ry * (accP[v] - my * csp[v]) + cbp[v];
            const float G = rx * (accG[v] - mx * csg[v]) + cbg[v];
            o[e] = (T)(P * sigmoid(G));
          }
          stg<V4>(dst + 8 * q, o);
        }
      }
    }
    __syncthreads();
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
  if (C_out == 256) {
    hipLaunchKernelGGL((tmu_in_kernel<T, 128, 8>), dim3((unsigned)grid), dim3(512), 0, st, (const T*)x,
                       (const int8_t*)mask, (const T*)Wp, (const T*)Wg, Bp, Bg, (T*)ab, L, ld, fstride, transpose, eps,
                       (uint32_t)ntiles, tdiv, ldiv);
  } else {
    hipLaunchKernelGGL((tmu_in_kernel<T, 128, 4>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)x,
                       (const int8_t*)mask, (const T*)Wp, (const T*)Wg, Bp, Bg, (T*)ab, L, ld, fstride, transpose, eps,
                       (uint32_t)ntiles, tdiv, ldiv);
  }
  return launched("tops_tmu_input_phase");
}

template <typename T>
static int tmu_einsum_t(const void* ab, void* y, int64_t nslab, int64_t L, int64_t ld, int64_t ldy, hipStream_t st) {
  const T* A = (const T*)ab;
  const T* Bm = A + nslab * L * ld;
  if (L > 384) {
    const int t = (int)((L + 255) / 256);
    const int64_t grid = nslab * t * t;
    hipLaunchKernelGGL((tmu_einsum_kernel<T, 256, 256>), dim3((unsigned)grid), dim3(256), 0, st, A, Bm, (T*)y, L, ld,
                       ldy, nslab, t, t);
  } else {
    const int t = (int)((L + 127) / 128);
    const int64_t grid = nslab * t * t;
    hipLaunchKernelGGL((tmu_einsum_kernel<T, 128, 128>), dim3((unsigned)grid), dim3(256), 0, st, A, Bm, (T*)y, L, ld,
                       ldy, nslab, t, t);
  }
  return launched("tops_tmu_einsum");
}

template <typename T>
static int tmu_output_phase_t(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                              const float* sWg, const float* Bp, const float* Bg, void* out, int64_t B, int64_t L,
                              int64_t ldy, float eps, hipStream_t st) {
  const int tpr = (int)((L + 63) / 64);
  const int64_t ntiles = B * L * tpr;
  if (ntiles == 0) return TOPS_OK;
  const int64_t cstride = B * L * ldy;
  const int64_t grid = ntiles < 8LL * num_cus() ? ntiles : 8LL * num_cus();
  hipLaunchKernelGGL((tmu_out_kernel<T, 128, 128>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)y, (const T*)x,
                     (const T*)Wp, (const T*)Wg, sWp, sWg, Bp, Bg, (T*)out, L, ldy, cstride, eps, ntiles, tpr);
  return launched("tops_tmu_output_phase");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_tmu_input_phase(const void* x, const void* mask, const void* Wp, const void* Wg, const float* sWp,
                                    const float* sWg, const float* Bp, const float* Bg, void* ab, int64_t B, int64_t L,
                                    int64_t C, int64_t C_out, int64_t ld, int transpose, float eps, int dtype,
                                    void* stream) {
  TOPS_REQUIRE(x && Wp && Wg && sWp && sWg && Bp && Bg && ab, "tops_tmu_input_phase: null pointer argument");
  TOPS_REQUIRE(C == 128, "tops_tmu_input_phase: C must be 128 (got %lld)", (long long)C);
  TOPS_REQUIRE(C_out == 128 || C_out == 256, "tops_tmu_input_phase: C_out must be 128 or 256 (got %lld)",
               (long long)C_out);
  TOPS_REQUIRE(B >= 0 && L >= 0 && ld >= L && ld % 64 == 0,
               "tops_tmu_input_phase: bad sizes B=%lld L=%lld ld=%lld (ld must be a multiple of 64)", (long long)B,
               (long long)L, (long long)ld);
  TOPS_REQUIRE(B * L * (ld / 64) < (1LL << 31), "tops_tmu_input_phase: too many tokens");
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
  TOPS_REQUIRE(ld % 64 == 0 && ld >= L && ldy >= L && L >= 0 && nslab >= 0,
               "tops_tmu_einsum: bad sizes nslab=%lld L=%lld ld=%lld ldy=%lld (ld must be a multiple of 64)",
               (long long)nslab, (long long)L, (long long)ld, (long long)ldy);
  if (L == 0 || nslab == 0) return TOPS_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16) return tmu_einsum_t<__bf16>(ab, y, nslab, L, ld, ldy, st);
  if (dtype == TOPS_DTYPE_F16) return tmu_einsum_t<_Float16>(ab, y, nslab, L, ld, ldy, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tmu_einsum: unsupported dtype code %d", dtype);
}

extern "C" int tops_tmu_output_phase(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                                     const float* sWg, const float* Bp, const float* Bg, void* out, int64_t B,
                                     int64_t L, int64_t C, int64_t C_out, int64_t ldy, float eps, int dtype,
                                     void* stream) {
  TOPS_REQUIRE(y && x && Wp && Wg && sWp && sWg && Bp && Bg && out, "tops_tmu_output_phase: null pointer argument");
  TOPS_REQUIRE(C == 128 && C_out == 128, "tops_tmu_output_phase: C and C_out must be 128 (got %lld, %lld)",
               (long long)C, (long long)C_out);
  TOPS_REQUIRE(B >= 0 && L >= 0 && ldy >= L, "tops_tmu_output_phase: bad sizes");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tmu_output_phase_t<__bf16>(y, x, Wp, Wg, sWp, sWg, Bp, Bg, out, B, L, ldy, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return tmu_output_phase_t<_Float16>(y, x, Wp, Wg, sWp, sWg, Bp, Bg, out, B, L, ldy, eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tmu_output_phase: unsupported dtype code %d", dtype);
}
