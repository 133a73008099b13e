// triangle_attention (starting node) on gfx950: two launches before the gate.
//
//   tri_prep_kernel   one pass over x per (row i, 64 positions): LN(x), the row-shared pair bias
//                     (fp32 dot), and Q, K, V of all heads as one K = 128 MFMA GEMM.  Outputs
//                     are written in the order the attention kernel consumes them:
//                       Qp  [i][h][q][32]    Q * scale * log2(e), d permuted (below)
//                       KV  [i][h][kb][4096] per 64-key block: K [64 keys][32 d permuted] then
//                                            V^T [32 d][64 keys permuted]
//                       bias[h][qt][kt][1024] log2(e) * bias per 32 x 32 (query, key) tile, in
//                                            the order of the MFMA B operand (below); keys
//                                            >= N hold zeros
//   tri_attn_kernel   4 waves per (row i, head h, query chunk): the KV block of each 64 keys is
//                     copied into LDS (double-buffered, one barrier per block), each wave
//                     streams its query tiles over it with an online softmax in the exp2
//                     domain.  No projection and no x_ln reads, so blocks are small enough for
//                     two to share a CU and hide each other's barriers.
//
// Element permutation within each group of 32 (d for Q/K, keys for V^T):
//   [0-3, 8-11, 4-7, 12-15, 16-19, 24-27, 20-23, 28-31]
// i.e. position 16 j + 8 hl + e (j = 0, 1; hl = lane / 32; e < 8) holds the element that the
// MFMA D register v = 8 j + e of lane half hl holds (8 (v / 4) + 4 hl + v % 4), so every MFMA
// operand of the attention kernel is one 16-byte load.
// Bias tile (query tile qt, key tile kt): element (q, k) = (32 qt + c, 32 kt + 16 j + 8 hl + e)
// sits at (64 j + 32 hl + c) * 8 + e, so the B operand of half j for lane (c, hl) is 16 bytes
// and one load instruction of a wave reads 1 KB contiguous.
//
// Reference: triangle_attn/module.py:57-125 (forward), triangle_attn/kernel.py:36-98 (bias),
// :110-253 (attention), :230-238 and :369 (additive -1e9 pair mask, -inf outside the row).
#include "capi.hpp"
#include "common.hpp"

namespace tops {

constexpr int kKVBlock = 4096;  // elements per (row, head, 64-key) KV block: 64x32 K + 32x64 V^T

// ---------------------------------------------------------------------------------------------
// Pre-pass.  One tile = (row i, positions [64 kb, 64 kb + 64)), 256 threads: the LN mapping is
// 4 threads per position (32 channels each); the GEMM mapping is wave w = head w with its
// WQ^T / WK^T / WV^T rows in registers and the normalized tile read from LDS as MFMA operands.
// Positions >= N are processed from zeros (finite values, masked by the attention kernel).
// ---------------------------------------------------------------------------------------------
template <typename T, int H>
__global__ __launch_bounds__(256, 1) void tri_prep_kernel(const T* __restrict__ x, int64_t sx0, int64_t sx1,
                                                         const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                         int apply_ln, const T* __restrict__ wqkv,
                                                         const T* __restrict__ WZ, const float* __restrict__ BZ,
                                                         T* __restrict__ Qp, T* __restrict__ KV, T* __restrict__ bias,
                                                         int64_t N, int64_t ldn, float eps, float qscale,
                                                         float bias_scale, int64_t ntiles) {
  constexpr int C = 128, D = 32, ROW = C * 2;
  static_assert(H == 4, "one wave per head");
  using V8 = vec<T, 8>;
  __shared__ __attribute__((aligned(16))) char xs[64 * ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int h = wave;
  const int64_t nkb = ldn / 64, nkt = ldn / 32, nqt = (N + 31) / 32;

  V8 wq[8], wk[8], wv[8];
  {
    const T* wh = wqkv + (int64_t)h * 3 * D * C + (int64_t)col * C + 8 * hl;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      wq[s] = ldg<V8>(wh + 16 * s);
      wk[s] = ldg<V8>(wh + D * C + 16 * s);
      wv[s] = ldg<V8>(wh + 2 * D * C + 16 * s);
    }
  }
  const int tok = tid >> 2, part = tid & 3;  // LN mapping

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t i = tile / nkb, kb = tile % nkb;
    const int64_t p = kb * 64 + tok;  // position of this thread's token
    // ---- LN + bias (fp32), normalized tile -> LDS ----
    {
      float v[32];
      if (p < N) {
        const T* src = x + i * sx0 + p * sx1 + 32 * part;
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
        const float rstd = rsqrtf(group_sum<4>(q) * (1.0f / C) + eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const V8 w8 = ldg<V8>(w_ln + 32 * part + 8 * e);
          const V8 b8 = b_ln ? ldg<V8>(b_ln + 32 * part + 8 * e) : V8{};
#pragma unroll
          for (int j = 0; j < 8; ++j) v[8 * e + j] = (v[8 * e + j] - mean) * rstd * (float)w8[j] + (float)b8[j];
        }
      }
#pragma unroll
      for (int hh = 0; hh < H; ++hh) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const V8 w8 = ldg<V8>(WZ + hh * C + 32 * part + 8 * e);
#pragma unroll
          for (int j = 0; j < 8; ++j) d += v[8 * e + j] * (float)w8[j];
        }
        d = group_sum<4>(d);
        if (part == 0) {
          const int64_t off = (((int64_t)hh * nqt + i / 32) * nkt + p / 32) * 1024 +
                              ((((p % 32) / 16) * 64 + ((p % 16) / 8) * 32 + i % 32) * 8 + p % 8);
          bias[off] = p < N ? (T)((d + (BZ ? BZ[hh] : 0.f)) * bias_scale) : (T)0.f;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        V8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (T)v[8 * e + j];
        const int chunk = 4 * part + e;
        *reinterpret_cast<V8*>(&xs[tok * ROW + ((chunk ^ (tok & 7)) << 4)]) = o;
      }
    }
    __syncthreads();
    // ---- Q, K, V of head h for the 64 positions ----
    T* qdst = Qp + ((i * H + h) * ldn + kb * 64) * D;
    T* kvdst = KV + ((i * H + h) * nkb + kb) * kKVBlock;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int t = sub * 32 + col;
      f32x16 aq = {}, ak = {}, av = {};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const V8 xb = *reinterpret_cast<const V8*>(&xs[t * ROW + (((2 * s + hl) ^ (t & 7)) << 4)]);
        aq = Mma<T>::m32(wq[s], xb, aq);  // Q^T: lane -> position t, d rows
        ak = Mma<T>::m32(wk[s], xb, ak);  // K^T: lane -> key t, d rows
        av = Mma<T>::m32(xb, wv[s], av);  // V:   lane -> d = col, key rows
      }
      V8 q0, q1, k0, k1, v0, v1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        q0[e] = (T)(aq[e] * qscale);
        q1[e] = (T)(aq[8 + e] * qscale);
        k0[e] = (T)ak[e];
        k1[e] = (T)ak[8 + e];
        v0[e] = (T)av[e];
        v1[e] = (T)av[8 + e];
      }
      stg<V8>(qdst + t * D + 8 * hl, q0);
      stg<V8>(qdst + t * D + 16 + 8 * hl, q1);
      stg<V8>(kvdst + t * D + 8 * hl, k0);
      stg<V8>(kvdst + t * D + 16 + 8 * hl, k1);
      stg<V8>(kvdst + 64 * D + col * 64 + sub * 32 + 8 * hl, v0);
      stg<V8>(kvdst + 64 * D + col * 64 + sub * 32 + 16 + 8 * hl, v1);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// Attention core.  4 waves, QT query tiles (32 queries) per wave, 64-key blocks of two 32-key
// tiles.
//
// Per (32-key tile, query tile) a wave runs
//     S^T  = C0 + I . bias^T          2 MFMAs, A = identity, B = 16 bias bytes per lane
//          + K . Q^T                  2 MFMAs, K from LDS, Q^T in registers
//     P    = exp2(S^T), l += rowsum   16 v_exp per lane, no max / subtract per element
//     O^T += V^T . P^T                2 MFMAs, V^T from LDS, P^T = S^T's D registers
// where C0 = -m (the running row max, broadcast) enters as the accumulator initialiser.  m
// is exact from the first tile with a valid key on and is only raised when a tile's
// probabilities could overflow the I/O type (then O and l are rescaled and the tile
// recomputed), so the common path needs neither a max nor a subtraction per score.  Masked
// keys get probability exactly 0 (equal to the reference's exp(-1e9 - m) in fp32 whenever the
// row has a valid key); a row without valid keys takes the uniform average of V over all N
// keys, as the reference's -1e9 add gives.  The identity MFMA multiplies every bias element
// of the tile by 0 or 1, so the bias padding must be finite (the pre-pass writes zeros).
//
// Each tile is one straight-line phase in which the score MFMAs of the NEXT tile are
// interleaved (sched_group_barrier) with the exponentials of the current one, so the matrix
// cores and the VALU of one wave work at the same time; the rare paths (partial tile, first
// max, overflow) branch around the phase.
// ---------------------------------------------------------------------------------------------
constexpr int kKPad = 40;  // LDS row of K: 32 d + 8 pad (conflict-free 16-byte operand reads)
constexpr int kVPad = 72;  // LDS row of V^T: 64 keys + 8 pad
constexpr int kKVLds = 64 * kKPad + 32 * kVPad;

// scheduling-group masks of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100;

template <typename T, int QT>
__global__ __launch_bounds__(256, 2) void tri_attn_kernel(const T* __restrict__ Qp, const T* __restrict__ KV,
                                                         const T* __restrict__ bias, const int8_t* __restrict__ mask,
                                                         int64_t sm0, int64_t sm1, T* __restrict__ out, int64_t so0,
                                                         int64_t so1, int64_t N, int64_t ldn, int H, int nqc) {
  constexpr int D = 32, NW = 4;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;

  __shared__ __attribute__((aligned(16))) T kvs[3][kKVLds];
  __shared__ unsigned long long kvalid[64];  // per 64-key block (N <= 4096)
  __shared__ short vblk[64];                 // indices of blocks with a valid key
  __shared__ int nvblk, row_any;

  // ---- block -> (row i, head h, query chunk); XCD-aware: an XCD works through a contiguous
  // ---- range of rows of one head, all query chunks of a row at once, so each KV block is read
  // ---- from HBM once and shared in that XCD's L2, as is the head's bias across rows.
  const int64_t total = N * H * nqc;
  int64_t id = blockIdx.x;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  const int qc = (int)(id % nqc);
  const int64_t ih = id / nqc;
  const int64_t i = ih % N;
  const int h = (int)(ih / N);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int nkb = (int)(ldn / 64);

  // ---- key validity per 64-key block; compact list of blocks to visit ----
  if (tid == 0) row_any = 0;
  __syncthreads();
  for (int kb = wave; kb < nkb; kb += NW) {
    const int64_t k = (int64_t)kb * 64 + lane;
    bool ok = k < N;
    if (ok && mask) ok = mask[i * sm0 + k * sm1] != 0;
    const unsigned long long bits = __ballot(ok);
    if (lane == 0) {
      kvalid[kb] = bits;
      if (bits) row_any = 1;
    }
  }
  __syncthreads();
  const bool uniform = row_any == 0;  // no valid key: every score is -1e9, weights 1/N
  if (tid == 0) {
    int n = 0;
    for (int kb = 0; kb < nkb; ++kb) {
      if (uniform) kvalid[kb] = (N - 64LL * kb >= 64) ? ~0ull : ((1ull << (N - 64LL * kb)) - 1ull);
      if (kvalid[kb]) vblk[n++] = (short)kb;
    }
    nvblk = n;
  }
  __syncthreads();
  const int nv = nvblk;  // >= 1 whenever N >= 1

  const T* kvrow = KV + ((int64_t)i * H + h) * nkb * kKVBlock;
  const int64_t nqt = (N + 31) / 32;

  // ---- Q^T operands (already scaled by scale * log2 e and d-permuted) and bias pointers.
  // ---- A row without valid keys zeroes Q and the identity, so its scores are all C0. ----
  const int64_t qbase = (int64_t)qc * (NW * 32 * QT) + (int64_t)wave * 32 * QT;
  V8 qop[QT][2];
  const T* bq[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    int64_t q = qbase + 32 * t + col;
    q = q < N ? q : N - 1;
    const T* qr = Qp + (((int64_t)i * H + h) * ldn + q) * D + 8 * hl;
    qop[t][0] = uniform ? V8{} : ldg<V8>(qr);
    qop[t][1] = uniform ? V8{} : ldg<V8>(qr + 16);
    bq[t] = bias + ((int64_t)h * nqt + q / 32) * (2 * nkb) * 1024 + (32 * hl + q % 32) * 8;
  }
  // identity A operands: (I . B)[key][q] = B[key - 16 j][q] for the keys of half j
  V8 ident[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) ident[j][e] = (T)((!uniform && col == 16 * j + 8 * hl + e) ? 1.f : 0.f);

  // KV block copy: thread t moves 16-byte chunks t (K: row t / 4) and 256 + t (V^T: row t / 8);
  // each load instruction of a wave reads 1 KB contiguous.
  auto kv_load = [&](int kb, V8* r) {
    const T* src = kvrow + (int64_t)kb * kKVBlock + 8 * tid;
    r[0] = ldg<V8>(src);
    r[1] = ldg<V8>(src + 64 * D);
  };
  auto kv_store = [&](int buf, const V8* r) {
    *reinterpret_cast<V8*>(&kvs[buf][(tid / 4) * kKPad + 8 * (tid % 4)]) = r[0];
    *reinterpret_cast<V8*>(&kvs[buf][64 * kKPad + (tid / 8) * kVPad + 8 * (tid % 8)]) = r[1];
  };
  // bias B operands of one 32-key tile: [query tile t][half j], 16 bytes per lane
  auto load_bias = [&](int kb, int kt, V8 (*bb)[2]) {
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) bb[t][j] = ldg<V8>(bq[t] + (int64_t)(2 * kb + kt) * 1024 + 512 * j);
  };
  f32x16 o[QT], cinit[QT];
  float l[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    o[t] = f32x16{};
    cinit[t] = f32x16{};
    l[t] = 0.f;
  }
  bool first = true;

  // scores of one 32-key tile for all query tiles
  auto scores = [&](const V8* kop, V8 (*bb)[2], f32x16* s) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      s[t] = Mma<T>::m32(ident[0], bb[t][0], cinit[t]);
      s[t] = Mma<T>::m32(ident[1], bb[t][1], s[t]);
      s[t] = Mma<T>::m32(kop[0], qop[t][0], s[t]);
      s[t] = Mma<T>::m32(kop[1], qop[t][1], s[t]);
    }
  };

  // One tile.  buf / kt / tb: its LDS buffer, tile within the block and valid-key bits; s: its
  // scores.  nbuf / nkt / bn / snext: the next tile's buffer, tile, bias operands and score
  // registers.  (rkb, rkt): the bias tile loaded into bn once the score MFMAs have read it.
  auto phase = [&](int buf, int kt, unsigned int tb, f32x16* s, int nbuf, int nkt, V8 (*bn)[2], f32x16* snext,
                   int rkb, int rkt) {
    if (tb != 0xffffffffu) {  // partial tile (wave-uniform): masked keys get probability 0
      const unsigned int lb = tb >> (4 * hl);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const bool ok = (lb >> (8 * (v / 4) + (v % 4))) & 1u;
#pragma unroll
        for (int t = 0; t < QT; ++t) s[t][v] = ok ? s[t][v] : -INFINITY;
      }
    }
    // ---- straight line: next tile's score MFMAs interleaved with this tile's exponentials ----
    V8 kop[2], vop[2];
    {
      const T* kr = &kvs[nbuf][(32 * nkt + col) * kKPad + 8 * hl];
      kop[0] = *reinterpret_cast<const V8*>(kr);
      kop[1] = *reinterpret_cast<const V8*>(kr + 16);
      const T* vr = &kvs[buf][64 * kKPad + col * kVPad + 32 * kt + 8 * hl];
      vop[0] = *reinterpret_cast<const V8*>(vr);
      vop[1] = *reinterpret_cast<const V8*>(vr + 16);
    }
    scores(kop, bn, snext);
    load_bias(rkb, rkt, bn);
    V8 p[QT][2];
    float ps[QT];
    bool over = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        p[t][0][v] = (T)fast_exp2(s[t][v]);
        p[t][1][v] = (T)fast_exp2(s[t][8 + v]);
      }
      // row sum of the rounded weights the PV product uses (packed dot products)
      ps[t] = sum8<T>(p[t][0], 0.f) + sum8<T>(p[t][1], 0.f);
      over |= !(ps[t] <= Mma<T>::kMaxP);
      pin(p[t][0]);
      pin(p[t][1]);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
    for (int m = 0; m < 2 * QT; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 9, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 2 * QT, 0);
#pragma unroll
    for (int m = 0; m < 2 * QT; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 9, 0);
    }
    // ---- rare: the first tile with a valid key sets the exact max; later tiles raise it only
    // ---- when a probability could overflow the I/O type ----
    const bool rare = (__ballot(over) != 0) | (first & (tb != 0));
    if (rare) {
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        float mr = s[t][0];
#pragma unroll
        for (int v = 1; v < 16; ++v) mr = fmaxf(mr, s[t][v]);
        mr = halves_max(mr);
        const float mt = first ? mr : fmaxf(mr, 0.f);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          p[t][0][v] = (T)fast_exp2(s[t][v] - mt);
          p[t][1][v] = (T)fast_exp2(s[t][8 + v] - mt);
        }
        ps[t] = sum8<T>(p[t][0], 0.f) + sum8<T>(p[t][1], 0.f);
        if (!first) {  // O and l are still zero before the first valid tile
          const float alpha = fast_exp2(-mt);
          o[t] *= alpha;
          l[t] *= alpha;
        }
        cinit[t] -= mt;
        snext[t] -= mt;
      }
      first = false;
    }
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      l[t] += ps[t];
      o[t] = Mma<T>::m32(vop[0], p[t][0], o[t]);
      o[t] = Mma<T>::m32(vop[1], p[t][1], o[t]);
    }
  };

  // Tiles (j, 0), (j, 1) of the visited blocks j in order.  Scores of tile (j, 0) live in sA,
  // of (j, 1) in sB, their bias operands in bA / bB, each loaded two tiles ahead.  KV blocks
  // rotate through three LDS buffers (the buffer written at block j was last read before the
  // previous barrier) and are loaded into registers two blocks ahead.  One barrier per block.
  // Past the last block the pipeline recomputes a tile of the last block (results unused).
  f32x16 sA[QT], sB[QT];
  V8 bA[QT][2], bB[QT][2];
  V8 kvA[2], kvB[2];
  auto blk = [&](int j) { return (int)vblk[j < nv ? j : nv - 1]; };
  kv_load(blk(0), kvA);
  load_bias(blk(0), 0, bA);
  load_bias(blk(0), 1, bB);
  if (nv > 1) kv_load(blk(1), kvB);
  kv_store(0, kvA);
  __syncthreads();
  {
    V8 kop[2];
    const T* kr = &kvs[0][col * kKPad + 8 * hl];
    kop[0] = *reinterpret_cast<const V8*>(kr);
    kop[1] = *reinterpret_cast<const V8*>(kr + 16);
    scores(kop, bA, sA);
    load_bias(blk(1), 0, bA);
  }
  auto block = [&](int j, V8* kload, const V8* kstore) {
    const int buf = j % 3, nbuf = (j + 1) % 3;
    const bool more = j + 1 < nv;
    const unsigned long long kbits = kvalid[vblk[j]];
    const int kb1 = blk(j + 1), kb2 = blk(j + 2);
    if (j + 2 < nv) kv_load(kb2, kload);
    phase(buf, 0, (unsigned int)kbits, sA, buf, 1, bB, sB, kb1, 1);
    if (more) kv_store(nbuf, kstore);
    __syncthreads();
    phase(buf, 1, (unsigned int)(kbits >> 32), sB, more ? nbuf : buf, 0, bA, sA, kb2, 0);
  };
  for (int j = 0; j < nv; j += 2) {
    block(j, kvA, kvB);
    if (j + 1 < nv) block(j + 1, kvB, kvA);
  }

  // ---- normalise and store O[i, q, h*D + d] ----
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int64_t q = qbase + 32 * t + col;
    const float inv = 1.0f / halves_sum(l[t]);
    if (q < N) {
      T* dst = out + i * so0 + q * so1 + (int64_t)h * D + 4 * hl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        V4 w4 = {(T)(o[t][4 * g] * inv), (T)(o[t][4 * g + 1] * inv), (T)(o[t][4 * g + 2] * inv),
                 (T)(o[t][4 * g + 3] * inv)};
        stg<V4>(dst + 8 * g, w4);
      }
    }
  }
}
template <typename T>
static int tri_prep_t(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln, int apply_ln,
                      const void* wqkv, const void* WZ, const float* BZ, void* Qp, void* KV, void* bias, int64_t N,
                      int64_t ldn, float eps, float qscale, hipStream_t st) {
  const int64_t ntiles = N * (ldn / 64);
  if (ntiles == 0) return TOPS_OK;
  const int64_t grid = ntiles < 2LL * num_cus() ? ntiles : 2LL * num_cus();
  hipLaunchKernelGGL((tri_prep_kernel<T, 4>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)x, sx0, sx1,
                     (const T*)w_ln, (const T*)b_ln, apply_ln, (const T*)wqkv, (const T*)WZ, BZ, (T*)Qp, (T*)KV,
                     (T*)bias, N, ldn, eps, qscale, kLog2e, ntiles);
  return launched("tops_tri_prep");
}

template <typename T>
static int tri_attention_t(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0,
                           int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H,
                           hipStream_t st) {
  const int qt = N <= 128 ? 1 : 2;
  const int64_t per_block = 4 * 32 * qt;
  const int nqc = (int)((N + per_block - 1) / per_block);
  const int64_t grid = N * H * nqc;
  if (grid == 0) return TOPS_OK;
#define TOPS_TRI(QTV)                                                                                     \
  hipLaunchKernelGGL((tri_attn_kernel<T, QTV>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)Qp,      \
                     (const T*)KV, (const T*)bias, (const int8_t*)mask, sm0, sm1, (T*)out, so0, so1, N, ldn, \
                     (int)H, nqc)
  if (qt == 1)
    TOPS_TRI(1);
  else
    TOPS_TRI(2);
#undef TOPS_TRI
  return launched("tops_tri_attention");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_tri_prep(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln,
                             int apply_ln, const void* wqkv, const void* WZ, const float* BZ, void* Qp, void* KV,
                             void* bias, int64_t N, int64_t ldn, int64_t C, int64_t H, int64_t D, float eps,
                             float scale, int dtype, void* stream) {
  TOPS_REQUIRE(x && wqkv && WZ && Qp && KV && bias, "tops_tri_prep: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_tri_prep: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(C == 128 && H == 4 && D == 32,
               "tops_tri_prep: supports C == 128, H == 4, D == 32 (got %lld, %lld, %lld)", (long long)C,
               (long long)H, (long long)D);
  TOPS_REQUIRE(N >= 0 && N <= 4096 && ldn >= N && ldn % 64 == 0, "tops_tri_prep: bad N / ldn");
  TOPS_REQUIRE(sx0 % 8 == 0 && sx1 % 8 == 0, "tops_tri_prep: x token strides must be multiples of 8");
  hipStream_t st = (hipStream_t)stream;
  const float qscale = scale * kLog2e;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_prep_t<__bf16>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, Qp, KV, bias, N, ldn, eps, qscale, st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_prep_t<_Float16>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, Qp, KV, bias, N, ldn, eps, qscale,
                                st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_prep: unsupported dtype code %d", dtype);
}

extern "C" int tops_tri_attention(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0,
                                  int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H,
                                  int64_t D, int dtype, void* stream) {
  TOPS_REQUIRE(Qp && KV && bias && out, "tops_tri_attention: null pointer argument");
  TOPS_REQUIRE(D == 32 && H >= 1 && H <= 64, "tops_tri_attention: supports D == 32 (got D=%lld H=%lld)", (long long)D,
               (long long)H);
  TOPS_REQUIRE(N >= 0 && N <= 4096 && ldn >= N && ldn % 64 == 0, "tops_tri_attention: bad N / ldn");
  TOPS_REQUIRE(so0 % 4 == 0 && so1 % 4 == 0, "tops_tri_attention: out strides must be multiples of 4");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_attention_t<__bf16>(Qp, KV, bias, mask, sm0, sm1, out, so0, so1, N, ldn, H, st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_attention_t<_Float16>(Qp, KV, bias, mask, sm0, sm1, out, so0, so1, N, ldn, H, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_attention: unsupported dtype code %d", dtype);
}
