// Any-shape kernels for the triangle-attention op and the gate / output projection: the
// shapes the tuned kernels do not cover (C_in != 128, D != 32, H != 4, C_out != 128, e.g. the
// D = 16, C_in = 64 "Apo" configuration).  Plain fp32 VALU arithmetic (no MFMA), written for
// correctness at small and medium sizes, and the path of fp32 I/O (then every value stays fp32);
// with 16-bit I/O the rounding points follow the tuned path:
//   LN(x) is rounded to the I/O type before the Q / K / V and gate products, Q / K / V and the
//   gated activations are rounded to the I/O type, the pair bias stays fp32.
//
//   tri_generic_prep_kernel   per token: LN(x) (fp32, two-pass), Q / K / V of all heads and
//                             the row-shared pair bias bias[h][a][b] = LN(x[a, b]) . Wz[h] + bz[h]
//   tri_generic_attn_kernel   64 queries of one (row i, head h) per block, keys split over 4 waves
//                             in 32-key chunks staged in LDS: online softmax in fp32, scores
//                             q . k * scale + bias, masked keys get the reference's fp32 "+ (-1e9)"
//   gate_generic_kernel       per token: y = (o * sigmoid(g . Wg^T + bg)) -> io, out = y . Wo^T + bo
//                             with g = LN(gin) or gin
//
//   tmu_generic_in_kernel     triangle_multiplicative_update input phase at any C / C_out:
//                             ab[f] = (xn . Wp[f] + Bp[f]) * sigmoid(xn . Wg[f] + Bg[f]) * mask,
//                             xn = (x - mean) * rstd (the LN affine is folded into Wp / Wg)
//   tmu_generic_out_kernel    output phase: (yn . Wp + Bp) * sigmoid(xn . Wg + Bg), yn = LN_out(y)
//
// Reference: triangle_attn/module.py:57-125 and benchmarks/references.py:174-205 (the op),
// triangle_attn/kernel.py:230-238 (-1e9 pair mask), :282-290 (D = 16 keeps separate K / V
// weights), tests/test_triangle_attn.py:137-192 (the Apo shape).
#include "capi.hpp"
#include "common.hpp"
#include "generic.hpp"

namespace tops {

constexpr int kGenTok = 16;  // tokens per block; 16 lanes per token for the LayerNorm sums
constexpr int kTK = 32;      // k-tile of the weights the tiled kernels stage through LDS

// LayerNorm of kGenTok token rows held in LDS (fp32, row length C, row stride ld): 16
// consecutive lanes per token, two-pass statistics.  Writes normalised rows back in place.
template <typename T>
__device__ void gen_layer_norm(float* rows, int ld, int C, const T* w_ln, const T* b_ln, float eps) {
  const int tid = threadIdx.x, t = tid >> 4, part = tid & 15;
  float* r = rows + t * ld;
  float s = 0.f;
  for (int c = part; c < C; c += 16) s += r[c];
  const float mean = group_sum<16>(s) / (float)C;
  float q = 0.f;
  for (int c = part; c < C; c += 16) q = fmaf(r[c] - mean, r[c] - mean, q);
  const float rstd = rsqrtf(group_sum<16>(q) / (float)C + eps);
  for (int c = part; c < C; c += 16) {
    const float w = w_ln ? (float)w_ln[c] : 1.f, b = b_ln ? (float)b_ln[c] : 0.f;
    r[c] = (r[c] - mean) * rstd * w + b;
  }
}

// ---------------------------------------------------------------------------------------------
// Pre-pass: 256 threads per kGenTok tokens.  xs holds the fp32 rows, LN'd in place.
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void tri_generic_prep_kernel(const T* __restrict__ x, int64_t sx0, int64_t sx1,
                                                              const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                              int apply_ln, const T* __restrict__ wqkv,
                                                              const T* __restrict__ WZ, const float* __restrict__ BZ,
                                                              T* __restrict__ xln, T* __restrict__ qo,
                                                              T* __restrict__ ko, T* __restrict__ vo,
                                                              float* __restrict__ bias, int64_t N, int C, int H, int D,
                                                              float eps) {
  extern __shared__ float xs[];  // [kGenTok][C]
  const int tid = threadIdx.x;
  const int64_t ntok = N * N, tok0 = (int64_t)blockIdx.x * kGenTok;
  for (int e = tid; e < kGenTok * C; e += 256) {
    const int t = e / C, c = e % C;
    const int64_t tok = tok0 + t;
    float v = 0.f;
    if (tok < ntok) v = (float)x[(tok / N) * sx0 + (tok % N) * sx1 + c];
    xs[e] = v;
  }
  __syncthreads();
  if (apply_ln) gen_layer_norm<T>(xs, C, C, w_ln, b_ln, eps);
  __syncthreads();
  const int HD = H * D, F = 3 * HD + H;
  for (int e = tid; e < kGenTok * F; e += 256) {
    const int t = e / F, f = e % F;
    const int64_t tok = tok0 + t;
    if (tok >= ntok) continue;
    const float* r = xs + t * C;
    if (f < 3 * HD) {  // head h, which (0 = Q, 1 = K, 2 = V), d
      const int h = f / (3 * D), which = (f / D) % 3, d = f % D;
      const T* w = wqkv + (int64_t)f * C;  // (H, 3, D, C): row f
      float acc = 0.f;
      for (int c = 0; c < C; ++c) acc = fmaf((float)(T)r[c], (float)w[c], acc);
      T* dst = which == 0 ? qo : which == 1 ? ko : vo;
      dst[tok * HD + h * D + d] = (T)acc;
    } else {
      const int h = f - 3 * HD;
      const T* w = WZ + (int64_t)h * C;
      float acc = 0.f;
      for (int c = 0; c < C; ++c) acc = fmaf(r[c], (float)w[c], acc);
      bias[(int64_t)h * ntok + tok] = acc + (BZ ? BZ[h] : 0.f);
    }
  }
  for (int e = tid; e < kGenTok * C; e += 256) {
    const int64_t tok = tok0 + e / C;
    if (tok < ntok) xln[tok * C + e % C] = (T)xs[e];
  }
}

// ---------------------------------------------------------------------------------------------
// Attention over R rows of N queries and N keys, any H, D <= DM.  A block takes 64 queries of
// one (row i, head h), lane = query; its 4 waves split the keys into 32-key chunks (chunk c to
// wave c % 4).  Per chunk a wave stages the chunk's K and V in LDS (fp32; every lane then reads
// the same element, a broadcast), computes the 32 scores of its queries (q . k * scale + bias;
// masked keys (mask[i*sm0 + k*sm1] == 0) get "+ (-1e9)" in fp32 (triangle attention) or -inf
// (MASK_INF, attention_pair_bias: a row without valid keys gives NaN, as torch's softmax does);
// keys >= N are left out), rescales its running (o, l) once to the chunk's maximum and adds
// exp(s - m) and exp(s - m) v.  The 4 waves' (m, l, o) are merged through LDS at the end.
// ---------------------------------------------------------------------------------------------
constexpr int kGenKC = 32, kGenAW = 4;  // keys per chunk, waves (key splits) per block

template <typename T, int DM, bool MASK_INF>
__global__ __launch_bounds__(256, 2) void tri_generic_attn_kernel(const T* __restrict__ qi_, const T* __restrict__ ki_,
                                                              const T* __restrict__ vi_, const float* __restrict__ bias,
                                                              const int8_t* __restrict__ mask, int64_t sm0, int64_t sm1,
                                                              T* __restrict__ out, int64_t so0, int64_t so1, int64_t R,
                                                              int64_t N, int H, int D, float scale) {
  __shared__ __attribute__((aligned(16))) float kvs[kGenAW][2][kGenKC][DM];  // per wave: K, V of its chunk
  __shared__ float madd[kGenAW][kGenKC];                                     // per key: 0, -1e9, -inf
  __shared__ float mls[kGenAW][64][2];                                       // per wave and query: m, l
  const int64_t nqb = (N + 63) / 64, qb = blockIdx.x % nqb, ih = blockIdx.x / nqb;
  const int h = (int)(ih % H);
  const int64_t i = ih / H;
  (void)R;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t q = qb * 64 + lane, qq = q < N ? q : N - 1;
  const int HD = H * D;
  float qv[DM], o[DM];
  const T* qp = qi_ + (i * N + qq) * HD + h * D;
#pragma unroll
  for (int d = 0; d < DM; ++d) {
    qv[d] = d < D ? (float)qp[d] * scale : 0.f;
    o[d] = 0.f;
  }
  const float* brow = bias + ((int64_t)h * N + qq) * N;
  float m = -INFINITY, l = 0.f;
  const int64_t nch = (N + kGenKC - 1) / kGenKC;
  for (int64_t c = wave; c < nch; c += kGenAW) {
    const int64_t k0 = c * kGenKC;
    for (int e = lane; e < kGenKC * DM; e += 64) {
      const int kk = e / DM, d = e % DM;
      const int64_t key = k0 + kk;
      const bool ok = key < N && d < D;
      const int64_t off = (i * N + key) * HD + h * D + d;
      kvs[wave][0][kk][d] = ok ? (float)ki_[off] : 0.f;
      kvs[wave][1][kk][d] = ok ? (float)vi_[off] : 0.f;
    }
    if (lane < kGenKC) {
      const int64_t key = k0 + lane;
      madd[wave][lane] = key >= N ? -INFINITY
                         : (mask && mask[i * sm0 + key * sm1] == 0) ? (MASK_INF ? -INFINITY : -1e9f)
                                                                     : 0.f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 8-key sub-chunks, each with its own maximum and one rescale of (o, l)
#pragma unroll 1
    for (int k8 = 0; k8 < kGenKC; k8 += 8) {
      float sc[8] = {};
      // q . k for the 8 keys, 4 channels per step; at most 32 K values live (the pins end a step's
      // products, the empty asm with a memory clobber keeps the next step's LDS reads after them)
#pragma unroll
      for (int d0 = 0; d0 < DM; d0 += 4) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const f32x4 kq = *reinterpret_cast<const f32x4*>(&kvs[wave][0][k8 + kk][d0]);
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[kk] = fmaf(qv[d0 + e], kq[e], sc[kk]);
        }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) pin(sc[kk]);  // this step's products are done here
        asm volatile("" ::: "memory");                 // and the next step's reads follow
      }
      float cm = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float a = sc[kk];
        const float ma = madd[wave][k8 + kk];
        const int64_t key = k0 + k8 + kk;
        const float sk = a + (key < N ? brow[key] : 0.f);
        sc[kk] = ma == 0.f ? sk : (ma == -INFINITY ? -INFINITY : sk + ma);
        cm = fmaxf(cm, sc[kk]);
      }
      const float mn = fmaxf(m, cm);
      // while every key so far is left out, m = mn = -inf: shift by 0 instead, so those keys get
      // p = 0 and the state stays (m, l, o) = (-inf, 0, 0) instead of NaN
      const float sh = mn == -INFINITY ? 0.f : mn;
      const float corr = __expf(m - sh);
      l *= corr;
#pragma unroll
      for (int d = 0; d < DM; ++d) o[d] *= corr;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float p = __expf(sc[kk] - sh);
        l += p;
#pragma unroll
        for (int d = 0; d < DM; d += 4) {
          const f32x4 vq = *reinterpret_cast<const f32x4*>(&kvs[wave][1][k8 + kk][d]);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[d + e] = fmaf(p, vq[e], o[d + e]);
        }
#pragma unroll
        for (int d = 0; d < DM; ++d) pin(o[d]);
        asm volatile("" ::: "memory");
      }
      m = mn;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // the chunk's K / V are read before the next chunk overwrites them
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // ---- merge the 4 waves' partial states (o goes through the K / V staging area) ----
  __syncthreads();
  float* ob = &kvs[0][0][0][0];  // [kGenAW][64][DM]
#pragma unroll
  for (int d = 0; d < DM; ++d) ob[(wave * 64 + lane) * DM + d] = o[d];
  mls[wave][lane][0] = m;
  mls[wave][lane][1] = l;
  __syncthreads();
  float mw[kGenAW], mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kGenAW; ++w) {
    mw[w] = mls[w][lane][0];
    mx = fmaxf(mx, mw[w]);
  }
  const float sh = mx == -INFINITY ? 0.f : mx;
  float sw[kGenAW], lt = 0.f;
#pragma unroll
  for (int w = 0; w < kGenAW; ++w) {
    sw[w] = __expf(mw[w] - sh);
    lt += sw[w] * mls[w][lane][1];
  }
  const float inv = 1.f / lt;
  if (q < N) {
    T* dst = out + i * so0 + q * so1 + h * D;
    for (int d = wave; d < D; d += kGenAW) {  // each wave writes every 4th element of the row
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kGenAW; ++w) acc += sw[w] * ob[(w * 64 + lane) * DM + d];
      dst[d] = (T)(acc * inv);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Gate + output projection, any (C_in, HD, C_out): 256 threads per kGenTok tokens.
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gate_generic_kernel(const T* __restrict__ o, int64_t so0, int64_t so1,
                                                          const T* __restrict__ gin, int64_t sg0, int64_t sg1,
                                                          const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                          float eps, int apply_ln, const T* __restrict__ Wg,
                                                          const T* __restrict__ bg, const T* __restrict__ Wo,
                                                          const T* __restrict__ bo, const T* __restrict__ res,
                                                          int64_t sr0, int64_t sr1, T* __restrict__ out, int64_t sd0,
                                                          int64_t sd1, int64_t M1, int64_t M2, int Cin, int HD,
                                                          int Cout) {
  extern __shared__ float sm[];
  float* gs = sm;                   // [kGenTok][Cin]  gate input (normalised)
  float* ys = sm + kGenTok * Cin;   // [kGenTok][HD]   o, then the gated activations
  const int tid = threadIdx.x;
  const int64_t M = M1 * M2, tok0 = (int64_t)blockIdx.x * kGenTok;
  for (int e = tid; e < kGenTok * Cin; e += 256) {
    const int64_t tok = tok0 + e / Cin;
    float v = 0.f;
    if (tok < M) v = (float)gin[(tok / M2) * sg0 + (tok % M2) * sg1 + e % Cin];
    gs[e] = v;
  }
  for (int e = tid; e < kGenTok * HD; e += 256) {
    const int64_t tok = tok0 + e / HD;
    float v = 0.f;
    if (tok < M) v = (float)o[(tok / M2) * so0 + (tok % M2) * so1 + e % HD];
    ys[e] = v;
  }
  __syncthreads();
  if (apply_ln) gen_layer_norm<T>(gs, Cin, Cin, w_ln, b_ln, eps);
  __syncthreads();
  for (int e = tid; e < kGenTok * HD; e += 256) {
    const int t = e / HD, j = e % HD;
    const float* g = gs + t * Cin;
    const T* w = Wg + (int64_t)j * Cin;
    float acc = bg ? (float)bg[j] : 0.f;
    for (int c = 0; c < Cin; ++c) acc = fmaf((float)(T)g[c], (float)w[c], acc);
    ys[e] = (float)(T)(ys[e] * sigmoid(acc));
  }
  __syncthreads();
  for (int e = tid; e < kGenTok * Cout; e += 256) {
    const int t = e / Cout, c = e % Cout;
    const int64_t tok = tok0 + t;
    if (tok >= M) continue;
    const float* y = ys + t * HD;
    const T* w = Wo + (int64_t)c * HD;
    float acc = bo ? (float)bo[c] : 0.f;
    for (int j = 0; j < HD; ++j) acc = fmaf(y[j], (float)w[j], acc);
    const int64_t m1 = tok / M2, m2 = tok % M2;
    // with a residual: out = res + result, the result rounded first as a separate add would see it
    out[m1 * sd0 + m2 * sd1 + c] = res ? (T)((float)res[m1 * sr0 + m2 * sr1 + c] + (float)(T)acc) : (T)acc;
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled pre-pass and gate for C_in <= 256 (and H * D <= 256 for the gate): 64 tokens per block,
// 256 threads.  Activations go to LDS k-major ([channel][token], fp32); every product is a block
// GEMM over that tile (tiled_gemm64: weights of 64 output features at a time staged k-major
// through LDS in 32-deep k-tiles, 4 tokens x 4 features per thread in registers).  Rounding
// points are those of the per-token kernels above.
// ---------------------------------------------------------------------------------------------
constexpr int kGT = 64, kGRow = kGT + 4;  // tokens per tile, LDS row of the k-major tiles

// out[t][f] = sum_k a[k][t] * W[f][k] (a: k-major LDS tile of kGT tokens, K valid rows of CK;
// W: F x K row-major in global memory), handed to epi(t, f, value) for t < ntok, f < F.  With
// ROUND the activations are rounded to T as the products' operand.  The (64-feature chunk,
// 32-deep k-tile) steps run as one sequence; each step's weights go k-major into LDS (ws: NBUF x
// kTK x kGRow floats) from registers loaded during the previous step, so the loads' latency
// overlaps the products.  One block barrier per step with two buffers, two with one (which
// leaves more LDS for the caller's tiles and more blocks per CU).
template <typename T, bool ROUND, int NBUF = 2, typename Epi>
__device__ __attribute__((always_inline)) inline void tiled_gemm64(const float* a, int K, int CK,
                                                                   const T* __restrict__ W, int F, float* ws,
                                                                   int ntok, Epi epi) {
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int nk = CK / kTK, nsteps = ((F + 63) / 64) * nk;
  // staging: thread tid moves weights (f, k) = (e / kTK, e % kTK), e = tid + 256 i, i < 8
  float wr[8];
  auto wload = [&](int step) __attribute__((always_inline)) {
    const int f0 = (step / nk) * 64, k0 = (step % nk) * kTK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = tid + 256 * i, ff = f0 + e / kTK, kk = k0 + e % kTK;
      wr[i] = ff < F && kk < K ? (float)W[(int64_t)ff * K + kk] : 0.f;
    }
  };
  auto wstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = tid + 256 * i;
      ws[(buf * kTK + e % kTK) * kGRow + e / kTK] = wr[i];
    }
  };
  __syncthreads();  // the caller's tile is complete; ws is free
  wload(0);
  wstore(0);
  float acc[4][4] = {};
  for (int step = 0; step < nsteps; ++step) {
    if constexpr (NBUF == 1) {
      if (step > 0) {
        __syncthreads();  // every thread is done with the previous step's weights
        wstore(0);
      }
    }
    __syncthreads();  // this step's buffer is filled (two buffers: the other one is no longer read)
    if (step + 1 < nsteps) wload(step + 1);
    const int k0 = (step % nk) * kTK;
    const float* wb = ws + (NBUF == 1 ? 0 : (step & 1)) * kTK * kGRow;
#pragma unroll 8
    for (int k = 0; k < kTK; ++k) {
      f32x4 x = *reinterpret_cast<const f32x4*>(&a[(k0 + k) * kGRow + 4 * ty]);
      if constexpr (ROUND) {
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = (float)(T)x[u];
      }
      const f32x4 w = *reinterpret_cast<const f32x4*>(&wb[k * kGRow + 4 * tx]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] = fmaf(x[u], w[v], acc[u][v]);
    }
    if constexpr (NBUF == 2) {
      if (step + 1 < nsteps) wstore((step + 1) & 1);
    }
    if (step % nk == nk - 1) {  // the chunk's last k-tile: epilogue, fresh accumulators
      const int f0 = (step / nk) * 64;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 4 * ty + u, f = f0 + 4 * tx + v;
          if (t < ntok && f < F) epi(t, f, acc[u][v]);
          acc[u][v] = 0.f;
        }
    }
  }
  __syncthreads();  // ws and the caller's tile may be reused after return
}

// LayerNorm (optionally with the affine w, b) of the kGT token columns of a k-major tile, in place
// (fp32, two-pass, 4 threads per token); rows [C, CK) are set to zero.
template <typename T>
__device__ __attribute__((always_inline)) inline void tiled_ln_affine(float* xs, int C, int CK, const T* __restrict__ w, const T* __restrict__ b,
                                       float eps) {
  const int t = threadIdx.x >> 2, part = threadIdx.x & 3;
  float s = 0.f;
  for (int k = part; k < C; k += 4) s += xs[k * kGRow + t];
  const float mean = group_sum<4>(s) / (float)C;
  float q = 0.f;
  for (int k = part; k < C; k += 4) {
    const float d = xs[k * kGRow + t] - mean;
    q = fmaf(d, d, q);
  }
  const float rstd = rsqrtf(group_sum<4>(q) / (float)C + eps);
  for (int k = part; k < CK; k += 4) {
    float v = 0.f;
    if (k < C) {
      v = (xs[k * kGRow + t] - mean) * rstd;
      if (w) v = v * (float)w[k] + (b ? (float)b[k] : 0.f);
    }
    xs[k * kGRow + t] = v;
  }
}

// Loads the rows of kGT tokens into a k-major tile dst[c][t] (c < C; rows [C, CK) and tokens
// t >= ntok are zeros; CK <= 256): wave w takes tokens w, w + 4, ..., its lanes consecutive
// channels, and row(t) gives the element offset of token t's row (once per token, wave-uniform).
// Four tokens' loads are issued before their LDS stores, so their latencies overlap.
template <typename T, typename Row>
__device__ __attribute__((always_inline)) inline void tiled_load_rows(float* dst, const T* __restrict__ src, int C,
                                                                      int CK, int ntok, Row row) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int t0 = wave; t0 < kGT; t0 += 16) {
    float v[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int t = t0 + 4 * a;
      const bool ok = t < ntok;
      const int64_t r0 = ok ? row(t) : 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int c = lane + 64 * b;
        v[a][b] = ok && c < C ? (float)src[r0 + c] : 0.f;
      }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int c = lane + 64 * b;
        if (c < CK) dst[c * kGRow + t0 + 4 * a] = v[a][b];
      }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void tri_gen_prep_tiled_kernel(const T* __restrict__ x, int64_t sx0, int64_t sx1,
                                                                const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                                int apply_ln, const T* __restrict__ wqkv,
                                                                const T* __restrict__ WZ, const float* __restrict__ BZ,
                                                                T* __restrict__ xln, T* __restrict__ qo,
                                                                T* __restrict__ ko, T* __restrict__ vo,
                                                                float* __restrict__ bias, int64_t N, int C, int H, int D,
                                                                float eps) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int CK = (C + kTK - 1) / kTK * kTK;
  float* xs = sm;                  // [CK][kGRow]  (LN(x)), k-major
  float* ws = xs + CK * kGRow;     // [2][kTK][kGRow] staged weights
  const int tid = threadIdx.x;
  const int64_t ntokall = N * N, tok0 = (int64_t)blockIdx.x * kGT;
  const int ntok = (int)(ntokall - tok0 < kGT ? ntokall - tok0 : kGT);
  tiled_load_rows<T>(xs, x, C, CK, ntok, [=](int t) {
    const int64_t tok = tok0 + t;
    return (tok / N) * sx0 + (tok % N) * sx1;
  });
  __syncthreads();
  if (apply_ln) tiled_ln_affine<T>(xs, C, CK, w_ln, b_ln, eps);
  __syncthreads();
  for (int e = tid; e < kGT * C; e += 256) {
    const int t = e / C, c = e % C;
    if (t < ntok) xln[(tok0 + t) * C + c] = (T)xs[c * kGRow + t];
  }
  const int HD = H * D;
  // Q / K / V of all heads from LN(x) rounded to the I/O type; weight row f = (h, which, d).  The
  // destination is picked by integer selects on address offsets (a pointer choice among the three
  // becomes a table in private memory)
  const uint64_t aq = (uint64_t)qo, dk = (uint64_t)ko - aq, dv = (uint64_t)vo - aq;
  tiled_gemm64<T, true>(xs, C, CK, wqkv, 3 * HD, ws, ntok, [=](int t, int f, float v) {
    const int h = f / (3 * D), which = (f / D) % 3, d = f % D;
    const uint64_t base = aq + (which == 1 ? dk : 0) + (which == 2 ? dv : 0);
    reinterpret_cast<T*>(base)[(tok0 + t) * HD + h * D + d] = (T)v;
  });
  // the row-shared pair bias from the unrounded LN(x), fp32
  tiled_gemm64<T, false>(xs, C, CK, WZ, H, ws, ntok,
                         [=](int t, int h, float v) { bias[(int64_t)h * ntokall + tok0 + t] = v + (BZ ? BZ[h] : 0.f); });
}

template <typename T>
__global__ __launch_bounds__(256) void gate_gen_tiled_kernel(const T* __restrict__ o, int64_t so0, int64_t so1,
                                                            const T* __restrict__ gin, int64_t sg0, int64_t sg1,
                                                            const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                            float eps, int apply_ln, const T* __restrict__ Wg,
                                                            const T* __restrict__ bg, const T* __restrict__ Wo,
                                                            const T* __restrict__ bo, const T* __restrict__ res,
                                                            int64_t sr0, int64_t sr1, T* __restrict__ out,
                                                            int64_t sd0, int64_t sd1, int64_t M1, int64_t M2, int Cin,
                                                            int HD, int Cout) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int CinK = (Cin + kTK - 1) / kTK * kTK, HDK = (HD + kTK - 1) / kTK * kTK;
  float* gs = sm;                  // [CinK][kGRow] gate input (normalised), k-major
  float* ys = gs + CinK * kGRow;   // [HDK][kGRow]  o, then the gated activations
  float* ws = ys + HDK * kGRow;    // [kTK][kGRow]
  const int tid = threadIdx.x;
  const int64_t M = M1 * M2, tok0 = (int64_t)blockIdx.x * kGT;
  const int ntok = (int)(M - tok0 < kGT ? M - tok0 : kGT);
  tiled_load_rows<T>(gs, gin, Cin, CinK, ntok, [=](int t) {
    const int64_t tok = tok0 + t;
    return (tok / M2) * sg0 + (tok % M2) * sg1;
  });
  tiled_load_rows<T>(ys, o, HD, HDK, ntok, [=](int t) {
    const int64_t tok = tok0 + t;
    return (tok / M2) * so0 + (tok % M2) * so1;
  });
  __syncthreads();
  if (apply_ln) tiled_ln_affine<T>(gs, Cin, CinK, w_ln, b_ln, eps);
  // gate: ys[j][t] = io(o * sigmoid(io(g) . Wg[j] + bg[j])), each element rewritten by the thread that reads it
  tiled_gemm64<T, true, 1>(gs, Cin, CinK, Wg, HD, ws, kGT, [=](int t, int j, float v) {
    const float g = v + (bg ? (float)bg[j] : 0.f);
    ys[j * kGRow + t] = (float)(T)(ys[j * kGRow + t] * sigmoid(g));
  });
  // output projection of the gated tile; with a residual, the result is rounded first
  tiled_gemm64<T, false, 1>(ys, HD, HDK, Wo, Cout, ws, ntok, [=](int t, int c, float v) {
    const T r = (T)(v + (bo ? (float)bo[c] : 0.f));
    const int64_t tok = tok0 + t, m1 = tok / M2, m2 = tok % M2;
    out[m1 * sd0 + m2 * sd1 + c] = res ? (T)((float)res[m1 * sr0 + m2 * sr1 + c] + (float)r) : r;
  });
}

template <typename T>
static int tri_generic_prep_t(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln,
                              int apply_ln, const void* wqkv, const void* WZ, const float* BZ, void* xln, void* q,
                              void* k, void* v, float* bias, int64_t N, int C, int H, int D, float eps,
                              hipStream_t st) {
  const int64_t tiles = (N * N + kGT - 1) / kGT;
  if (C <= 256 && tiles >= num_cus()) {  // tiled kernel: 64 tokens per block
    const int CK = (C + kTK - 1) / kTK * kTK;
    const size_t lds = (size_t)(CK + 2 * kTK) * kGRow * sizeof(float);
    hipFuncSetAttribute((const void*)tri_gen_prep_tiled_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)lds);
    hipLaunchKernelGGL((tri_gen_prep_tiled_kernel<T>), dim3((unsigned)tiles), dim3(256), lds, st, (const T*)x, sx0, sx1,
                       (const T*)w_ln, (const T*)b_ln, apply_ln, (const T*)wqkv, (const T*)WZ, BZ, (T*)xln, (T*)q,
                       (T*)k, (T*)v, bias, N, C, H, D, eps);
    return launched("tops_tri_generic_prep");
  }
  const int64_t blocks = (N * N + kGenTok - 1) / kGenTok;
  if (blocks == 0) return TOPS_OK;
  hipLaunchKernelGGL((tri_generic_prep_kernel<T>), dim3((unsigned)blocks), dim3(256), kGenTok * C * sizeof(float), st,
                     (const T*)x, sx0, sx1, (const T*)w_ln, (const T*)b_ln, apply_ln, (const T*)wqkv, (const T*)WZ,
                     BZ, (T*)xln, (T*)q, (T*)k, (T*)v, bias, N, C, H, D, eps);
  return launched("tops_tri_generic_prep");
}

template <typename T>
static int tri_generic_attention_t(const void* q, const void* k, const void* v, const float* bias, const void* mask,
                                   int64_t sm0, int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int H,
                                   int D, float scale, hipStream_t st) {
  const int64_t blocks = N * H * ((N + 63) / 64);
  if (blocks == 0) return TOPS_OK;
  TOPS_REQUIRE(blocks < (1LL << 31), "tops_tri_generic_attention: too many query blocks");
#define TOPS_GEN_ATTN(DMV)                                                                                           \
  hipLaunchKernelGGL((tri_generic_attn_kernel<T, DMV, false>), dim3((unsigned)blocks), dim3(256), 0, st,            \
                     (const T*)q, (const T*)k, (const T*)v, bias, (const int8_t*)mask, sm0, sm1, (T*)out, so0, so1, \
                     N, N, H, D, scale)
  if (D <= 16)
    TOPS_GEN_ATTN(16);
  else if (D <= 32)
    TOPS_GEN_ATTN(32);
  else
    TOPS_GEN_ATTN(64);
#undef TOPS_GEN_ATTN
  return launched("tops_tri_generic_attention");
}

template <typename T>
static int gate_generic_t(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                          const void* w_ln, const void* b_ln, float eps, int apply_ln, const void* Wg, const void* bg,
                          const void* Wo, const void* bo, const void* res, int64_t sr0, int64_t sr1, void* out,
                          int64_t sd0, int64_t sd1, int64_t M1, int64_t M2, int Cin, int HD, int Cout,
                          hipStream_t st) {
  const int64_t tiles = (M1 * M2 + kGT - 1) / kGT;
  if (Cin <= 256 && HD <= 256 && tiles >= num_cus()) {  // tiled kernel: 64 tokens per block
    const int CinK = (Cin + kTK - 1) / kTK * kTK, HDK = (HD + kTK - 1) / kTK * kTK;
    const size_t lds = (size_t)(CinK + HDK + kTK) * kGRow * sizeof(float);
    hipFuncSetAttribute((const void*)gate_gen_tiled_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((gate_gen_tiled_kernel<T>), dim3((unsigned)tiles), dim3(256), lds, st, (const T*)o, so0, so1,
                       (const T*)gin, sg0, sg1, (const T*)w_ln, (const T*)b_ln, eps, apply_ln, (const T*)Wg,
                       (const T*)bg, (const T*)Wo, (const T*)bo, (const T*)res, sr0, sr1, (T*)out, sd0, sd1, M1, M2,
                       Cin, HD, Cout);
    return launched(res ? "tops_gate_out_generic_residual" : "tops_gate_out_generic");
  }
  const int64_t blocks = (M1 * M2 + kGenTok - 1) / kGenTok;
  if (blocks == 0) return TOPS_OK;
  hipLaunchKernelGGL((gate_generic_kernel<T>), dim3((unsigned)blocks), dim3(256),
                     (size_t)kGenTok * (Cin + HD) * sizeof(float), st, (const T*)o, so0, so1, (const T*)gin, sg0, sg1,
                     (const T*)w_ln, (const T*)b_ln, eps, apply_ln, (const T*)Wg, (const T*)bg, (const T*)Wo,
                     (const T*)bo, (const T*)res, sr0, sr1, (T*)out, sd0, sd1, M1, M2, Cin, HD, Cout);
  return launched(res ? "tops_gate_out_generic_residual" : "tops_gate_out_generic");
}

// ---------------------------------------------------------------------------------------------
// attention_pair_bias, any (C_s, C_z, H, D) (attn_pair_bias/kernel.py:205-257):
//   apb_generic_qkv_kernel   per token m: q / k / v [m][h][d] = X[m] . W (rounded to the I/O type)
//   apb_generic_bias_kernel  per pair (q, k): bias[h][q][k] = zn . Wc[h] + Bc[h], zn = (z - mean) * rstd
//                            of z = Z[q, k, :] (the LN affine is folded into Wc / Bc)
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void apb_generic_qkv_kernel(const T* __restrict__ X, const T* __restrict__ wqkv,
                                                             T* __restrict__ qo, T* __restrict__ ko,
                                                             T* __restrict__ vo, int64_t M, int C, int H, int D) {
  const int HD = H * D;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * 3 * HD) return;
  const int64_t m = idx / (3 * HD);
  const int f = (int)(idx % (3 * HD));  // row of the (H, 3, D, C) weight
  const int h = f / (3 * D), which = (f / D) % 3, d = f % D;
  const T* xr = X + m * C;
  const T* w = wqkv + (int64_t)f * C;
  float acc = 0.f;
  for (int c = 0; c < C; ++c) acc = fmaf((float)xr[c], (float)w[c], acc);
  T* dst = which == 0 ? qo : which == 1 ? ko : vo;
  dst[m * HD + h * D + d] = (T)acc;
}

template <typename T>
__global__ __launch_bounds__(256) void apb_generic_bias_kernel(const T* __restrict__ Z, int64_t sz0, int64_t sz1,
                                                              const float* __restrict__ Wc,
                                                              const float* __restrict__ Bc, float* __restrict__ bias,
                                                              int64_t M, int Cz, int H, float eps) {
  extern __shared__ float zs[];  // [kGenTok][Cz]
  const int tid = threadIdx.x;
  const int64_t npair = M * M, p0 = (int64_t)blockIdx.x * kGenTok;
  for (int e = tid; e < kGenTok * Cz; e += 256) {
    const int64_t pr = p0 + e / Cz;
    zs[e] = pr < npair ? (float)Z[(pr / M) * sz0 + (pr % M) * sz1 + e % Cz] : 0.f;
  }
  __syncthreads();
  gen_layer_norm<T>(zs, Cz, Cz, nullptr, nullptr, eps);
  __syncthreads();
  for (int e = tid; e < kGenTok * H; e += 256) {
    const int t = e / H, h = e % H;
    const int64_t pr = p0 + t;
    if (pr >= npair) continue;
    const float* z = zs + t * Cz;
    const float* w = Wc + (int64_t)h * Cz;
    float acc = Bc[h];
    for (int c = 0; c < Cz; ++c) acc = fmaf(z[c], w[c], acc);
    bias[(int64_t)h * npair + pr] = acc;
  }
}

// Tiled apb pre-pass kernels (C_s, C_z <= 256): Q / K / V as a block GEMM over 64 tokens and 64
// weight rows; the pair bias as a LayerNorm of 64 pairs in LDS, then per head (one wave each) the
// dot products of its 64 pairs (lanes) with the head's weights (wave-uniform: scalar loads).
template <typename T>
__global__ __launch_bounds__(256) void apb_gen_qkv_tiled_kernel(const T* __restrict__ X, const T* __restrict__ wqkv,
                                                               T* __restrict__ qo, T* __restrict__ ko,
                                                               T* __restrict__ vo, int64_t M, int C, int H, int D) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int CK = (C + kTK - 1) / kTK * kTK;
  float* xs = sm;               // [CK][kGRow]  X, k-major
  float* ws = xs + CK * kGRow;  // [2][kTK][kGRow]
  const int tid = threadIdx.x;
  const int64_t tok0 = (int64_t)blockIdx.x * kGT;
  const int ntok = (int)(M - tok0 < kGT ? M - tok0 : kGT);
  tiled_load_rows<T>(xs, X, C, CK, ntok, [=](int t) { return (tok0 + t) * (int64_t)C; });
  const int HD = H * D;
  const uint64_t aq = (uint64_t)qo, dk = (uint64_t)ko - aq, dv = (uint64_t)vo - aq;
  // this block's 64 weight rows (blockIdx.y): more blocks than tokens / 64 alone would give
  const int fb = 64 * (int)blockIdx.y, nf = 3 * HD - fb < 64 ? 3 * HD - fb : 64;
  tiled_gemm64<T, false>(xs, C, CK, wqkv + (int64_t)fb * C, nf, ws, ntok, [=](int t, int fl, float v) {
    const int f = fb + fl, h = f / (3 * D), which = (f / D) % 3, d = f % D;
    const uint64_t base = aq + (which == 1 ? dk : 0) + (which == 2 ? dv : 0);
    reinterpret_cast<T*>(base)[(tok0 + t) * HD + h * D + d] = (T)v;
  });
}

template <typename T>
__global__ __launch_bounds__(256) void apb_gen_bias_tiled_kernel(const T* __restrict__ Z, int64_t sz0, int64_t sz1,
                                                                const float* __restrict__ Wc,
                                                                const float* __restrict__ Bc, float* __restrict__ bias,
                                                                int64_t M, int Cz, int H, float eps) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int CzK = (Cz + kTK - 1) / kTK * kTK;
  float* zs = sm;  // [CzK][kGRow]  LN(Z) of 64 pairs, k-major
  const int tid = threadIdx.x;
  const int64_t npair = M * M, p0 = (int64_t)blockIdx.x * kGT;
  const int np = (int)(npair - p0 < kGT ? npair - p0 : kGT);
  tiled_load_rows<T>(zs, Z, Cz, CzK, np, [=](int t) {
    const int64_t pr = p0 + t;
    return (pr / M) * sz0 + (pr % M) * sz1;
  });
  __syncthreads();
  tiled_ln_affine<T>(zs, Cz, CzK, nullptr, nullptr, eps);
  __syncthreads();
  const int lane = tid & 63;
  for (int h = __builtin_amdgcn_readfirstlane(tid >> 6); h < H; h += 4) {
    const float* w = Wc + (int64_t)h * Cz;
    float acc[4] = {Bc[h], 0.f, 0.f, 0.f};
    int c = 0;
    for (; c + 4 <= Cz; c += 4)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = fmaf(zs[(c + j) * kGRow + lane], w[c + j], acc[j]);
    for (; c < Cz; ++c) acc[0] = fmaf(zs[c * kGRow + lane], w[c], acc[0]);
    if (lane < np) bias[(int64_t)h * npair + p0 + lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
}

template <typename T>
static int apb_generic_prep_t(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                              const float* Wc, const float* Bc, void* q, void* k, void* v, float* bias, int64_t M,
                              int C, int Cz, int H, int D, float eps, hipStream_t st) {
  // the tiled bias kernel takes 64 pairs per block: used where that still gives every CU a block
  const int64_t t1 = (M + kGT - 1) / kGT, t2 = (M * M + kGT - 1) / kGT;
  if (t1 == 0) return TOPS_OK;
  if (C <= 256) {
    const int CK = (C + kTK - 1) / kTK * kTK;
    const size_t l1 = (size_t)(CK + 2 * kTK) * kGRow * sizeof(float);
    hipFuncSetAttribute((const void*)apb_gen_qkv_tiled_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)l1);
    hipLaunchKernelGGL((apb_gen_qkv_tiled_kernel<T>), dim3((unsigned)t1, (unsigned)((3 * H * D + 63) / 64)), dim3(256),
                       l1, st, (const T*)X, (const T*)wqkv, (T*)q, (T*)k, (T*)v, M, C, H, D);
  } else {
    const int64_t b1 = (M * 3 * H * D + 255) / 256;
    hipLaunchKernelGGL((apb_generic_qkv_kernel<T>), dim3((unsigned)b1), dim3(256), 0, st, (const T*)X,
                       (const T*)wqkv, (T*)q, (T*)k, (T*)v, M, C, H, D);
  }
  if (Cz <= 256 && t2 >= num_cus()) {
    const int CzK = (Cz + kTK - 1) / kTK * kTK;
    const size_t l2 = (size_t)CzK * kGRow * sizeof(float);
    hipFuncSetAttribute((const void*)apb_gen_bias_tiled_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)l2);
    hipLaunchKernelGGL((apb_gen_bias_tiled_kernel<T>), dim3((unsigned)t2), dim3(256), l2, st, (const T*)Z, sz0, sz1, Wc,
                       Bc, bias, M, Cz, H, eps);
  } else {
    const int64_t b2 = (M * M + kGenTok - 1) / kGenTok;
    hipLaunchKernelGGL((apb_generic_bias_kernel<T>), dim3((unsigned)b2), dim3(256),
                       (size_t)kGenTok * Cz * sizeof(float), st, (const T*)Z, sz0, sz1, Wc, Bc, bias, M, Cz, H, eps);
  }
  return launched("tops_apb_generic_prep");
}

template <typename T>
static int apb_generic_attention_t(const void* q, const void* k, const void* v, const float* bias, const void* mask,
                                   void* Og, int64_t M, int H, int D, float scale, hipStream_t st) {
  const int64_t blocks = H * ((M + 63) / 64);
  if (blocks == 0) return TOPS_OK;
  const int64_t HD = (int64_t)H * D;
#define TOPS_GEN_APB(DMV)                                                                                         \
  hipLaunchKernelGGL((tri_generic_attn_kernel<T, DMV, true>), dim3((unsigned)blocks), dim3(256), 0, st,          \
                     (const T*)q, (const T*)k, (const T*)v, bias, (const int8_t*)mask, 0, 1, (T*)Og, 0, HD, 1, M, \
                     H, D, scale)
  if (D <= 16)
    TOPS_GEN_APB(16);
  else if (D <= 32)
    TOPS_GEN_APB(32);
  else
    TOPS_GEN_APB(64);
#undef TOPS_GEN_APB
  return launched("tops_apb_generic_attention");
}

// ---------------------------------------------------------------------------------------------
// triangle_multiplicative_update, any C (triangle_mul/module.py:8-12: x is (B, L, L, D), any D;
// triangle_mul/kernel.py:235-326).  Tokens t = (b, i, j) in row-major order.
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void tmu_generic_in_kernel(const T* __restrict__ x, const int8_t* __restrict__ mask,
                                                            const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                            const float* __restrict__ Bp, const float* __restrict__ Bg,
                                                            T* __restrict__ ab, int64_t B, int64_t L, int C, int Cout,
                                                            int64_t ld, int transpose, float eps) {
  extern __shared__ float xs[];  // [kGenTok][C]
  const int tid = threadIdx.x;
  const int64_t ntok = B * L * L, tok0 = (int64_t)blockIdx.x * kGenTok;
  for (int e = tid; e < kGenTok * C; e += 256) {
    const int64_t tok = tok0 + e / C;
    xs[e] = tok < ntok ? (float)x[tok * C + e % C] : 0.f;
  }
  __syncthreads();
  gen_layer_norm<T>(xs, C, C, nullptr, nullptr, eps);
  __syncthreads();
  for (int e = tid; e < kGenTok * C; e += 256) xs[e] = (float)(T)xs[e];  // GEMM operand in the I/O type
  __syncthreads();
  const int64_t fstride = B * L * ld;
  for (int e = tid; e < kGenTok * Cout; e += 256) {
    const int t = e / Cout, f = e % Cout;
    const int64_t tok = tok0 + t;
    if (tok >= ntok) continue;
    const float* r = xs + t * C;
    const T* wp = Wp + (int64_t)f * C;
    const T* wg = Wg + (int64_t)f * C;
    float p = Bp[f], g = Bg[f];
    for (int c = 0; c < C; ++c) {
      p = fmaf(r[c], (float)wp[c], p);
      g = fmaf(r[c], (float)wg[c], g);
    }
    const float m = mask ? (mask[tok] != 0 ? 1.f : 0.f) : 1.f;
    const int64_t b = tok / (L * L), rem = tok % (L * L), i = rem / L, j = rem % L;
    const int64_t row = transpose ? j : i, col = transpose ? i : j;
    T* dst = ab + f * fstride + (b * L + row) * ld;
    dst[col] = (T)(p * sigmoid(g) * m);
    if (col == L - 1)  // zero k-padding of this row for the einsum
      for (int64_t c = L; c < ld; ++c) dst[c] = (T)0.f;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void tmu_generic_out_kernel(const T* __restrict__ y, const T* __restrict__ x,
                                                             const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                             const float* __restrict__ Bp,
                                                             const float* __restrict__ Bg, const T* __restrict__ res,
                                                             T* __restrict__ out, int64_t B, int64_t L, int C,
                                                             int Cout, int64_t ldy, float eps) {
  extern __shared__ float sm[];
  float* ys = sm;                 // [kGenTok][C]  y of the tile's tokens (token-major)
  float* xs = sm + kGenTok * C;   // [kGenTok][C]  x
  const int tid = threadIdx.x;
  const int64_t ntok = B * L * L, tok0 = (int64_t)blockIdx.x * kGenTok, cstride = B * L * ldy;
  for (int e = tid; e < kGenTok * C; e += 256) {
    const int t = e % kGenTok, c = e / kGenTok;  // token fastest: y is channel-major
    const int64_t tok = tok0 + t;
    float v = 0.f;
    if (tok < ntok) {
      const int64_t b = tok / (L * L), rem = tok % (L * L);
      v = (float)y[c * cstride + (b * L + rem / L) * ldy + rem % L];
    }
    ys[t * C + c] = v;
  }
  for (int e = tid; e < kGenTok * C; e += 256) {
    const int64_t tok = tok0 + e / C;
    xs[e] = tok < ntok ? (float)x[tok * C + e % C] : 0.f;
  }
  __syncthreads();
  gen_layer_norm<T>(ys, C, C, nullptr, nullptr, eps);
  gen_layer_norm<T>(xs, C, C, nullptr, nullptr, eps);
  __syncthreads();
  for (int e = tid; e < 2 * kGenTok * C; e += 256) sm[e] = (float)(T)sm[e];
  __syncthreads();
  for (int e = tid; e < kGenTok * Cout; e += 256) {
    const int t = e / Cout, f = e % Cout;
    const int64_t tok = tok0 + t;
    if (tok >= ntok) continue;
    const float* yr = ys + t * C;
    const float* xr = xs + t * C;
    const T* wp = Wp + (int64_t)f * C;
    const T* wg = Wg + (int64_t)f * C;
    float p = Bp[f], g = Bg[f];
    for (int c = 0; c < C; ++c) {
      p = fmaf(yr[c], (float)wp[c], p);
      g = fmaf(xr[c], (float)wg[c], g);
    }
    const T r = (T)(p * sigmoid(g));
    out[tok * Cout + f] = res ? (T)((float)res[tok * Cout + f] + (float)r) : r;
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled forms of the two phases for C <= 256 (the kernels above remain for wider C): a block
// takes a tile of tokens, normalises them into LDS k-major ([channel][token], fp32, rounded to
// the I/O type as the products' operand, exactly as above), stages the weights of a chunk of
// output features k-major through LDS in 32-deep k-tiles, and each thread accumulates 4 tokens
// x 4 features of P and of G in registers (fp32 FMAs), then applies bias, gate and mask.
//   input phase:  64 tokens of one row r of the (B, L, ld) store grid (tokens (r, c) or,
//                 transposed, (c, r), c = c0 .. c0 + 63; c >= L stores zeros), 64-feature chunks,
//                 each thread's 4 tokens stored as one vector per feature (contiguous in ab)
//   output phase: 32 tokens (b, i, j0 .. j0 + 31), y read channel-major 32 tokens per channel,
//                 128-feature chunks, each thread's 4 features stored as one vector per token
// ---------------------------------------------------------------------------------------------
constexpr int kTinTok = 64, kTinRow = kTinTok + 4;    // input phase: tokens per tile, LDS row
constexpr int kToutTok = 32, kToutRow = kToutTok + 4;  // output phase
constexpr int kTF = 128, kTFRow = kTF + 4;              // output phase: features per chunk, LDS row

// LayerNorm of the `ntok` token columns of a k-major LDS tile (4 threads per token, two-pass),
// rounding the normalised values to T; rows k in [C, CK) are set to zero.
template <typename T>
__device__ inline void tiled_layer_norm(float* xs, int row, int ntok, int C, int CK, float eps) {
  const int t = threadIdx.x >> 2, part = threadIdx.x & 3;
  if (t >= ntok) return;  // whole quads drop out together, so the quad sums stay exact
  float s = 0.f;
  for (int k = part; k < C; k += 4) s += xs[k * row + t];
  const float mean = group_sum<4>(s) / (float)C;
  float q = 0.f;
  for (int k = part; k < C; k += 4) {
    const float d = xs[k * row + t] - mean;
    q = fmaf(d, d, q);
  }
  const float rstd = rsqrtf(group_sum<4>(q) / (float)C + eps);
  for (int k = part; k < CK; k += 4) xs[k * row + t] = k < C ? (float)(T)((xs[k * row + t] - mean) * rstd) : 0.f;
}

template <typename T>
__global__ __launch_bounds__(256) void tmu_gen_in_tiled_kernel(const T* __restrict__ x, const int8_t* __restrict__ mask,
                                                              const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                              const float* __restrict__ Bp, const float* __restrict__ Bg,
                                                              T* __restrict__ ab, int64_t L, int C, int Cout, int64_t ld,
                                                              int64_t fstride, int transpose, float eps) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int CK = (C + kTK - 1) / kTK * kTK;
  float* xs = sm;                     // [CK][kTinRow]  normalised tile
  float* wps = xs + CK * kTinRow;     // [kTK][kTinRow] P weights of the chunk, k-major
  float* wgs = wps + kTK * kTinRow;   // [kTK][kTinRow] G weights
  float* msk = wgs + kTK * kTinRow;   // [kTinTok] 1 for a valid, unmasked token
  const int tid = threadIdx.x;
  const int64_t tpr = ld / kTinTok, rr = blockIdx.x / tpr, r = rr % L, b = rr / L;
  const int64_t c0 = (blockIdx.x % tpr) * kTinTok;
  auto token = [&](int t) -> int64_t {  // x / mask index of tile token t (t >= L - c0: position L - 1)
    int64_t c = c0 + t;
    c = c < L ? c : L - 1;
    return transpose ? (b * L + c) * L + r : (b * L + r) * L + c;
  };
  for (int e = tid; e < kTinTok * C; e += 256) {  // row-major reads, k-major LDS
    const int t = e / C, k = e % C;
    xs[k * kTinRow + t] = (float)x[token(t) * C + k];
  }
  if (tid < kTinTok) msk[tid] = c0 + tid < L ? (mask ? (mask[token(tid)] != 0 ? 1.f : 0.f) : 1.f) : 0.f;
  __syncthreads();
  tiled_layer_norm<T>(xs, kTinRow, kTinTok, C, CK, eps);

  const int ty = tid >> 4, tx = tid & 15;  // tokens 4 ty .. + 3, chunk features 4 tx .. + 3
  T* abt = ab + (b * L + r) * ld + c0 + 4 * ty;
  // (64-feature chunk, 32-deep k-tile) steps in one sequence; each step's P and G weights are
  // loaded into registers during the previous step and stored k-major into LDS after a barrier
  const int nk = CK / kTK, nsteps = ((Cout + 63) / 64) * nk;
  float wr[16];  // P (0-7) and G (8-15) weights (f, k) = (e / kTK, e % kTK), e = tid + 256 i
  auto wload = [&](int step) __attribute__((always_inline)) {
    const int f0 = (step / nk) * 64, k0 = (step % nk) * kTK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = tid + 256 * i, ff = f0 + e / kTK, kk = k0 + e % kTK;
      const bool ok = ff < Cout && kk < C;
      wr[i] = ok ? (float)Wp[(int64_t)ff * C + kk] : 0.f;
      wr[8 + i] = ok ? (float)Wg[(int64_t)ff * C + kk] : 0.f;
    }
  };
  wload(0);
  float ap[4][4] = {}, ag[4][4] = {};
  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();  // the previous step's weights are consumed (step 0: the tile is normalised)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = tid + 256 * i;
      wps[(e % kTK) * kTinRow + e / kTK] = wr[i];
      wgs[(e % kTK) * kTinRow + e / kTK] = wr[8 + i];
    }
    __syncthreads();
    if (step + 1 < nsteps) wload(step + 1);
    const int k0 = (step % nk) * kTK;
#pragma unroll 8
    for (int k = 0; k < kTK; ++k) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&xs[(k0 + k) * kTinRow + 4 * ty]);
      const f32x4 wp = *reinterpret_cast<const f32x4*>(&wps[k * kTinRow + 4 * tx]);
      const f32x4 wg = *reinterpret_cast<const f32x4*>(&wgs[k * kTinRow + 4 * tx]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          ap[u][v] = fmaf(a[u], wp[v], ap[u][v]);
          ag[u][v] = fmaf(a[u], wg[v], ag[u][v]);
        }
    }
    if (step % nk != nk - 1) continue;
    const int f0 = (step / nk) * 64;  // the chunk's last k-tile: bias, gate, mask, store
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int f = f0 + 4 * tx + v;
      if (f < Cout) {
        const float bp = Bp[f], bg = Bg[f];
        vec<T, 4> o;
#pragma unroll
        for (int u = 0; u < 4; ++u) o[u] = (T)((ap[u][v] + bp) * sigmoid(ag[u][v] + bg) * msk[4 * ty + u]);
        *reinterpret_cast<vec<T, 4>*>(abt + (int64_t)f * fstride) = o;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) ap[u][v] = ag[u][v] = 0.f;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void tmu_gen_out_tiled_kernel(const T* __restrict__ y, const T* __restrict__ x,
                                                               const T* __restrict__ Wp, const T* __restrict__ Wg,
                                                               const float* __restrict__ Bp,
                                                               const float* __restrict__ Bg, const T* __restrict__ res,
                                                               T* __restrict__ out, int64_t L, int C, int Cout,
                                                               int64_t ldy, int64_t cstride, float eps) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int CK = (C + kTK - 1) / kTK * kTK;
  float* ys = sm;                      // [CK][kToutRow]  LN_out(y), k-major
  float* xs = ys + CK * kToutRow;      // [CK][kToutRow]  LN_in(x)
  float* wps = xs + CK * kToutRow;     // [kTK][kTFRow]
  float* wgs = wps + kTK * kTFRow;     // [kTK][kTFRow]
  const int tid = threadIdx.x;
  const int64_t tpr = (L + kToutTok - 1) / kToutTok, bi = blockIdx.x / tpr;  // bi = b * L + i
  const int64_t j0 = (blockIdx.x % tpr) * kToutTok;
  const int ntok = (int)(L - j0 < kToutTok ? L - j0 : kToutTok);
  for (int e = tid; e < kToutTok * C; e += 256) {  // y channel-major: 32 consecutive tokens per channel
    const int k = e / kToutTok, t = e % kToutTok;
    ys[k * kToutRow + t] = t < ntok ? (float)y[(int64_t)k * cstride + bi * ldy + j0 + t] : 0.f;
  }
  for (int e = tid; e < kToutTok * C; e += 256) {  // x token-major
    const int t = e / C, k = e % C;
    xs[k * kToutRow + t] = t < ntok ? (float)x[(bi * L + j0 + t) * C + k] : 0.f;
  }
  __syncthreads();
  tiled_layer_norm<T>(ys, kToutRow, kToutTok, C, CK, eps);
  tiled_layer_norm<T>(xs, kToutRow, kToutTok, C, CK, eps);

  const int ty = tid >> 5, tx = tid & 31;  // tokens 4 ty .. + 3, chunk features 4 tx .. + 3
  // (128-feature chunk, 32-deep k-tile) steps in one sequence, weights prefetched into registers
  const int nk = CK / kTK, nsteps = ((Cout + kTF - 1) / kTF) * nk;
  float wr[32];  // P (0-15) and G (16-31) weights (f, k) = (e / kTK, e % kTK), e = tid + 256 i
  auto wload = [&](int step) __attribute__((always_inline)) {
    const int f0 = (step / nk) * kTF, k0 = (step % nk) * kTK;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = tid + 256 * i, ff = f0 + e / kTK, kk = k0 + e % kTK;
      const bool ok = ff < Cout && kk < C;
      wr[i] = ok ? (float)Wp[(int64_t)ff * C + kk] : 0.f;
      wr[16 + i] = ok ? (float)Wg[(int64_t)ff * C + kk] : 0.f;
    }
  };
  wload(0);
  float ap[4][4] = {}, ag[4][4] = {};
  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();  // the previous step's weights are consumed (step 0: the tiles are normalised)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = tid + 256 * i;
      wps[(e % kTK) * kTFRow + e / kTK] = wr[i];
      wgs[(e % kTK) * kTFRow + e / kTK] = wr[16 + i];
    }
    __syncthreads();
    if (step + 1 < nsteps) wload(step + 1);
    const int k0 = (step % nk) * kTK;
#pragma unroll 8
    for (int k = 0; k < kTK; ++k) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&ys[(k0 + k) * kToutRow + 4 * ty]);
      const f32x4 g = *reinterpret_cast<const f32x4*>(&xs[(k0 + k) * kToutRow + 4 * ty]);
      const f32x4 wp = *reinterpret_cast<const f32x4*>(&wps[k * kTFRow + 4 * tx]);
      const f32x4 wg = *reinterpret_cast<const f32x4*>(&wgs[k * kTFRow + 4 * tx]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          ap[u][v] = fmaf(a[u], wp[v], ap[u][v]);
          ag[u][v] = fmaf(g[u], wg[v], ag[u][v]);
        }
    }
    if (step % nk != nk - 1) continue;
    const int f0 = (step / nk) * kTF;  // the chunk's last k-tile: bias, gate, residual, store
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * ty + u;
      const int64_t o = (bi * L + j0 + t) * Cout;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int f = f0 + 4 * tx + v;
        if (t < ntok && f < Cout) {
          const T rv = (T)((ap[u][v] + Bp[f]) * sigmoid(ag[u][v] + Bg[f]));
          out[o + f] = res ? (T)((float)res[o + f] + (float)rv) : rv;
        }
        ap[u][v] = ag[u][v] = 0.f;
      }
    }
  }
}

int tmu_generic_input_phase(const void* x, const void* mask, const void* Wp, const void* Wg, const float* Bp,
                            const float* Bg, void* ab, int64_t B, int64_t L, int64_t C, int64_t C_out, int64_t ld,
                            int transpose, float eps, int dtype, hipStream_t st) {
  TOPS_REQUIRE(C >= 1 && C <= 1024 && C_out >= 1 && C_out <= 4096,
               "tops_tmu_input_phase: supports C <= 1024, C_out <= 4096 (got %lld, %lld)", (long long)C,
               (long long)C_out);
  if (C <= 256) {  // tiled kernel
    const int64_t tiles = B * L * (ld / kTinTok);
    if (tiles == 0) return TOPS_OK;
    TOPS_REQUIRE(tiles < (1LL << 31), "tops_tmu_input_phase: too many tokens");
    const int CK = (int)((C + kTK - 1) / kTK * kTK);
    const size_t lds = ((size_t)(CK + 2 * kTK) * kTinRow + kTinTok) * sizeof(float);
    const int64_t fstride = B * L * ld;
#define TOPS_GEN_IN_T(TT)                                                                                        \
  do {                                                                                                           \
    hipFuncSetAttribute((const void*)tmu_gen_in_tiled_kernel<TT>, hipFuncAttributeMaxDynamicSharedMemorySize,    \
                        (int)lds);                                                                               \
    hipLaunchKernelGGL((tmu_gen_in_tiled_kernel<TT>), dim3((unsigned)tiles), dim3(256), lds, st, (const TT*)x,     \
                       (const int8_t*)mask, (const TT*)Wp, (const TT*)Wg, Bp, Bg, (TT*)ab, L, (int)C, (int)C_out, ld, \
                       fstride, transpose, eps);                                                                  \
  } while (0)
    if (dtype == TOPS_DTYPE_BF16)
      TOPS_GEN_IN_T(__bf16);
    else if (dtype == TOPS_DTYPE_F16)
      TOPS_GEN_IN_T(_Float16);
    else if (dtype == TOPS_DTYPE_F32)
      TOPS_GEN_IN_T(float);
    else
      return fail(TOPS_EUNSUPPORTED, "tops_tmu_input_phase: unsupported dtype code %d", dtype);
#undef TOPS_GEN_IN_T
    return launched("tops_tmu_input_phase");
  }
  const int64_t blocks = (B * L * L + kGenTok - 1) / kGenTok;
  if (blocks == 0) return TOPS_OK;
  const size_t lds = (size_t)kGenTok * C * sizeof(float);
#define TOPS_GEN_IN(TT)                                                                                            hipLaunchKernelGGL((tmu_generic_in_kernel<TT>), dim3((unsigned)blocks), dim3(256), lds, st, (const TT*)x,                           (const int8_t*)mask, (const TT*)Wp, (const TT*)Wg, Bp, Bg, (TT*)ab, B, L, (int)C, (int)C_out,                      ld, transpose, eps)
  if (dtype == TOPS_DTYPE_BF16)
    TOPS_GEN_IN(__bf16);
  else if (dtype == TOPS_DTYPE_F16)
    TOPS_GEN_IN(_Float16);
  else if (dtype == TOPS_DTYPE_F32)
    TOPS_GEN_IN(float);
  else
    return fail(TOPS_EUNSUPPORTED, "tops_tmu_input_phase: unsupported dtype code %d", dtype);
#undef TOPS_GEN_IN
  return launched("tops_tmu_input_phase");
}

int tmu_generic_output_phase(const void* y, const void* x, const void* Wp, const void* Wg, const float* Bp,
                             const float* Bg, const void* res, void* out, int64_t B, int64_t L, int64_t C,
                             int64_t C_out, int64_t ldy, float eps, int dtype, hipStream_t st) {
  TOPS_REQUIRE(C >= 1 && C <= 512 && C_out >= 1 && C_out <= 4096,
               "tops_tmu_output_phase: supports C <= 512, C_out <= 4096 (got %lld, %lld)", (long long)C,
               (long long)C_out);
  if (C <= 256) {  // tiled kernel
    const int64_t tiles = B * L * ((L + kToutTok - 1) / kToutTok);
    if (tiles == 0) return TOPS_OK;
    TOPS_REQUIRE(tiles < (1LL << 31), "tops_tmu_output_phase: too many tokens");
    const int CK = (int)((C + kTK - 1) / kTK * kTK);
    const size_t lds = ((size_t)2 * CK * kToutRow + (size_t)2 * kTK * kTFRow) * sizeof(float);
    const int64_t cstride = B * L * ldy;
#define TOPS_GEN_OUT_T(TT)                                                                                       \
  do {                                                                                                           \
    hipFuncSetAttribute((const void*)tmu_gen_out_tiled_kernel<TT>, hipFuncAttributeMaxDynamicSharedMemorySize,   \
                        (int)lds);                                                                               \
    hipLaunchKernelGGL((tmu_gen_out_tiled_kernel<TT>), dim3((unsigned)tiles), dim3(256), lds, st, (const TT*)y,    \
                       (const TT*)x, (const TT*)Wp, (const TT*)Wg, Bp, Bg, (const TT*)res, (TT*)out, L, (int)C,    \
                       (int)C_out, ldy, cstride, eps);                                                            \
  } while (0)
    if (dtype == TOPS_DTYPE_BF16)
      TOPS_GEN_OUT_T(__bf16);
    else if (dtype == TOPS_DTYPE_F16)
      TOPS_GEN_OUT_T(_Float16);
    else if (dtype == TOPS_DTYPE_F32)
      TOPS_GEN_OUT_T(float);
    else
      return fail(TOPS_EUNSUPPORTED, "tops_tmu_output_phase: unsupported dtype code %d", dtype);
#undef TOPS_GEN_OUT_T
    return launched("tops_tmu_output_phase");
  }
  const int64_t blocks = (B * L * L + kGenTok - 1) / kGenTok;
  if (blocks == 0) return TOPS_OK;
  const size_t lds = (size_t)2 * kGenTok * C * sizeof(float);
#define TOPS_GEN_OUT(TT)                                                                                        hipLaunchKernelGGL((tmu_generic_out_kernel<TT>), dim3((unsigned)blocks), dim3(256), lds, st, (const TT*)y,                      (const TT*)x, (const TT*)Wp, (const TT*)Wg, Bp, Bg, (const TT*)res, (TT*)out, B, L, (int)C, (int)C_out, ldy, eps)
  if (dtype == TOPS_DTYPE_BF16)
    TOPS_GEN_OUT(__bf16);
  else if (dtype == TOPS_DTYPE_F16)
    TOPS_GEN_OUT(_Float16);
  else if (dtype == TOPS_DTYPE_F32)
    TOPS_GEN_OUT(float);
  else
    return fail(TOPS_EUNSUPPORTED, "tops_tmu_output_phase: unsupported dtype code %d", dtype);
#undef TOPS_GEN_OUT
  return launched("tops_tmu_output_phase");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_tri_generic_prep(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln,
                                     int apply_ln, const void* wqkv, const void* WZ, const float* BZ, void* xln,
                                     void* q, void* k, void* v, float* bias, int64_t N, int64_t C, int64_t H,
                                     int64_t D, float eps, int dtype, void* stream) {
  TOPS_REQUIRE(x && wqkv && WZ && xln && q && k && v && bias, "tops_tri_generic_prep: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_tri_generic_prep: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(N >= 0 && N <= 65536, "tops_tri_generic_prep: bad N %lld", (long long)N);
  TOPS_REQUIRE(C >= 1 && C <= 1024 && H >= 1 && H <= 64 && D >= 1 && D <= 64,
               "tops_tri_generic_prep: supports C <= 1024, H <= 64, D <= 64 (got %lld, %lld, %lld)", (long long)C,
               (long long)H, (long long)D);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_generic_prep_t<__bf16>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, xln, q, k, v, bias, N, (int)C,
                                      (int)H, (int)D, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_generic_prep_t<_Float16>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, xln, q, k, v, bias, N,
                                        (int)C, (int)H, (int)D, eps, st);
  if (dtype == TOPS_DTYPE_F32)
    return tri_generic_prep_t<float>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, xln, q, k, v, bias, N, (int)C,
                                     (int)H, (int)D, eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_generic_prep: unsupported dtype code %d", dtype);
}

extern "C" int tops_tri_generic_attention(const void* q, const void* k, const void* v, const float* bias,
                                          const void* mask, int64_t sm0, int64_t sm1, void* out, int64_t so0,
                                          int64_t so1, int64_t N, int64_t H, int64_t D, float scale, int dtype,
                                          void* stream) {
  TOPS_REQUIRE(q && k && v && bias && out, "tops_tri_generic_attention: null pointer argument");
  TOPS_REQUIRE(N >= 0 && N <= 65536 && H >= 1 && H <= 64 && D >= 1 && D <= 64,
               "tops_tri_generic_attention: supports H <= 64, D <= 64 (got N=%lld H=%lld D=%lld)", (long long)N,
               (long long)H, (long long)D);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_generic_attention_t<__bf16>(q, k, v, bias, mask, sm0, sm1, out, so0, so1, N, (int)H, (int)D, scale,
                                           st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_generic_attention_t<_Float16>(q, k, v, bias, mask, sm0, sm1, out, so0, so1, N, (int)H, (int)D, scale,
                                             st);
  if (dtype == TOPS_DTYPE_F32)
    return tri_generic_attention_t<float>(q, k, v, bias, mask, sm0, sm1, out, so0, so1, N, (int)H, (int)D, scale, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_generic_attention: unsupported dtype code %d", dtype);
}

extern "C" int tops_apb_generic_prep(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                                     const float* Wc, const float* Bc, void* q, void* k, void* v, float* bias,
                                     int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D, float eps, int dtype,
                                     void* stream) {
  TOPS_REQUIRE(X && wqkv && Z && Wc && Bc && q && k && v && bias, "tops_apb_generic_prep: null pointer argument");
  TOPS_REQUIRE(M >= 0 && M <= 65536 && C >= 1 && C <= 4096 && Cz >= 1 && Cz <= 1024 && H >= 1 && H <= 64 && D >= 1 &&
                   D <= 64,
               "tops_apb_generic_prep: supports C <= 4096, Cz <= 1024, H <= 64, D <= 64 (got M=%lld C=%lld Cz=%lld "
               "H=%lld D=%lld)",
               (long long)M, (long long)C, (long long)Cz, (long long)H, (long long)D);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return apb_generic_prep_t<__bf16>(X, wqkv, Z, sz0, sz1, Wc, Bc, q, k, v, bias, M, (int)C, (int)Cz, (int)H, (int)D,
                                      eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return apb_generic_prep_t<_Float16>(X, wqkv, Z, sz0, sz1, Wc, Bc, q, k, v, bias, M, (int)C, (int)Cz, (int)H,
                                        (int)D, eps, st);
  if (dtype == TOPS_DTYPE_F32)
    return apb_generic_prep_t<float>(X, wqkv, Z, sz0, sz1, Wc, Bc, q, k, v, bias, M, (int)C, (int)Cz, (int)H, (int)D,
                                     eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_apb_generic_prep: unsupported dtype code %d", dtype);
}

extern "C" int tops_apb_generic_attention(const void* q, const void* k, const void* v, const float* bias,
                                          const void* mask, void* Og, int64_t M, int64_t H, int64_t D, float scale,
                                          int dtype, void* stream) {
  TOPS_REQUIRE(q && k && v && bias && Og, "tops_apb_generic_attention: null pointer argument");
  TOPS_REQUIRE(M >= 0 && M <= 65536 && H >= 1 && H <= 64 && D >= 1 && D <= 64,
               "tops_apb_generic_attention: supports H <= 64, D <= 64 (got M=%lld H=%lld D=%lld)", (long long)M,
               (long long)H, (long long)D);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return apb_generic_attention_t<__bf16>(q, k, v, bias, mask, Og, M, (int)H, (int)D, scale, st);
  if (dtype == TOPS_DTYPE_F16)
    return apb_generic_attention_t<_Float16>(q, k, v, bias, mask, Og, M, (int)H, (int)D, scale, st);
  if (dtype == TOPS_DTYPE_F32)
    return apb_generic_attention_t<float>(q, k, v, bias, mask, Og, M, (int)H, (int)D, scale, st);
  return fail(TOPS_EUNSUPPORTED, "tops_apb_generic_attention: unsupported dtype code %d", dtype);
}

static int gate_generic_dispatch(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                                 const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg,
                                 const void* bg, const void* Wo, const void* bo, const void* res, int64_t sr0,
                                 int64_t sr1, void* out, int64_t sd0, int64_t sd1, int64_t M1, int64_t M2, int64_t Cin,
                                 int64_t HD, int64_t Cout, int dtype, hipStream_t st) {
  if (dtype == TOPS_DTYPE_BF16)
    return gate_generic_t<__bf16>(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, res, sr0,
                                  sr1, out, sd0, sd1, M1, M2, (int)Cin, (int)HD, (int)Cout, st);
  if (dtype == TOPS_DTYPE_F16)
    return gate_generic_t<_Float16>(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, res,
                                    sr0, sr1, out, sd0, sd1, M1, M2, (int)Cin, (int)HD, (int)Cout, st);
  if (dtype == TOPS_DTYPE_F32)
    return gate_generic_t<float>(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, res, sr0,
                                 sr1, out, sd0, sd1, M1, M2, (int)Cin, (int)HD, (int)Cout, st);
  return fail(TOPS_EUNSUPPORTED, "tops_gate_out_generic: unsupported dtype code %d", dtype);
}

extern "C" int tops_gate_out_generic(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0,
                                     int64_t sg1, const void* w_ln, const void* b_ln, float ln_eps, int apply_ln,
                                     const void* Wg, const void* bg, const void* Wo, const void* bo, void* out,
                                     int64_t M1, int64_t M2, int64_t Cin, int64_t HD, int64_t Cout, int dtype,
                                     void* stream) {
  TOPS_REQUIRE(o && gin && Wg && Wo && out, "tops_gate_out_generic: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_gate_out_generic: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(M1 >= 0 && M2 >= 0, "tops_gate_out_generic: bad sizes");
  TOPS_REQUIRE(Cin >= 1 && HD >= 1 && Cout >= 1 && Cin + HD <= 1024 && Cout <= 4096,
               "tops_gate_out_generic: supports C_in + H*D <= 1024, C_out <= 4096 (got %lld, %lld, %lld)",
               (long long)Cin, (long long)HD, (long long)Cout);
  return gate_generic_dispatch(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, nullptr, 0, 0,
                               out, M2 * Cout, Cout, M1, M2, Cin, HD, Cout, dtype, (hipStream_t)stream);
}

extern "C" int tops_gate_out_generic_residual(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0,
                                              int64_t sg1, const void* w_ln, const void* b_ln, float ln_eps,
                                              int apply_ln, const void* Wg, const void* bg, const void* Wo,
                                              const void* bo, const void* res, int64_t sr0, int64_t sr1, void* out,
                                              int64_t sd0, int64_t sd1, int64_t M1, int64_t M2, int64_t Cin,
                                              int64_t HD, int64_t Cout, int dtype, void* stream) {
  TOPS_REQUIRE(o && gin && Wg && Wo && res && out, "tops_gate_out_generic_residual: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_gate_out_generic_residual: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(M1 >= 0 && M2 >= 0, "tops_gate_out_generic_residual: bad sizes");
  TOPS_REQUIRE(Cin >= 1 && HD >= 1 && Cout >= 1 && Cin + HD <= 1024 && Cout <= 4096,
               "tops_gate_out_generic_residual: supports C_in + H*D <= 1024, C_out <= 4096 (got %lld, %lld, %lld)",
               (long long)Cin, (long long)HD, (long long)Cout);
  return gate_generic_dispatch(o, so0, so1, gin, sg0, sg1, w_ln, b_ln, ln_eps, apply_ln, Wg, bg, Wo, bo, res, sr0, sr1,
                               out, sd0, sd1, M1, M2, Cin, HD, Cout, dtype, (hipStream_t)stream);
}
