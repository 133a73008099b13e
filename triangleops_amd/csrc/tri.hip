// triangle_attention (starting node) on gfx950: two launches before the gate.
//
//   tri_prep_kernel   one pass over x per (row i, 64 positions): LN(x), the row-shared pair bias
//                     (fp32 dot), and Q, K, V of all heads as one K = 128 MFMA GEMM.  Outputs
//                     are written in the order the attention kernel consumes them:
//                       Qp  [i][h][q][32]    Q * scale * log2(e), d permuted (below)
//                       KV  [i][h][kb][4096] per 64-key block: K [64 keys][32 d permuted] then
//                                            V^T [32 d][64 keys permuted]
//                       bias[h][qt][kt][1024] log2(e) * bias per 32 x 32 (query, key) tile, in
//                                            the order of the score MFMA's D registers
//                                            (below); keys >= N hold zeros
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
// Bias tile (query tile qt, key tile kt): element (q, k) = (32 qt + c, 32 kt + p) sits at
// (64 j + 32 hl + c) * 8 + e for the key p = perm(16 j + 8 hl + e) that D register v = 8 j + e of
// lane (c, hl) holds (the permutation above), so the 16 score slots of a lane are two 16-byte
// loads, widened to fp32 they are the score MFMAs' accumulator initialiser, and one load
// instruction of a wave reads 1 KB contiguous.
//
// Reference: triangle_attn/module.py:57-125 (forward), triangle_attn/kernel.py:36-98 (bias),
// :110-253 (attention), :230-238 and :369 (additive -1e9 pair mask, -inf outside the row).
#include <type_traits>

#include "capi.hpp"
#include "common.hpp"

namespace tops {

constexpr int kKVBlock = 4096;  // elements per (row, head, 64-key) KV block: 64x32 K + 32x64 V^T
constexpr int kMaxN = 16384;    // largest N of the tuned kernels (per-row key-block tables in LDS)
constexpr int kMaxKB = kMaxN / 64;

// The pre-pass buffers' key stride: N rounded up to a multiple of 64 (at least 64).
#ifndef TRI_NW8_MIN_N
#define TRI_NW8_MIN_N 4096  // from this N on, 8-wave attention blocks (half the KV block copies per query)
#endif
static inline int64_t tri_ldn(int64_t N) { return N <= 64 ? 64 : (N + 63) / 64 * 64; }
#ifndef TRI_WPE
#define TRI_WPE(QT, NW) (8 / (NW))  // waves per SIMD the attention kernel's registers are sized for
#endif

// ---------------------------------------------------------------------------------------------
// Pre-pass.  One tile = (row i, positions [64 kb, 64 kb + 64)), 8 waves in two roles:
//   waves 0-3 (loaders) fetch x four tiles ahead (C / 8 lanes per 2C-byte token row; positions
//   >= N reload position N - 1, so every fetch issues the same loads), take the LayerNorm and
//   the 4 heads' pair bias in fp32, and stage the normalised tile in LDS (double-buffered);
//   waves 4-7 (head w - 4) run that head's Q / K / V GEMM over the 64 positions with its WQ /
//   WK / WV rows in registers, stage the results in a private LDS block in the HBM image of
//   the tile (XOR-swizzled 16-byte chunks) and store it back, 1 KB per store instruction.
// No wave has loads and stores in flight together, so each register stage is waited for only
// when it is consumed, and the loaders' LayerNorm of tile n + 1 overlaps the writers' GEMM of
// tile n: one barrier per tile.  Positions >= N are computed from zeros (finite values, masked
// by the attention kernel).
// C (the pair channel count) is 128 or 64.  The outputs always have the 32-wide head layout the
// attention kernel reads; with a head width D < 32 the weight rows d >= D are zeros, so Q, K and
// V are exact zeros there and add nothing to the scores or to O.
// ---------------------------------------------------------------------------------------------
template <typename T, bool LN, int C>
__global__ __launch_bounds__(512) void tri_prep_kernel(const T* __restrict__ x, int64_t sx0, int64_t sx1,
                                                      const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                      const T* __restrict__ wqkv, const T* __restrict__ WZ,
                                                      const float* __restrict__ BZ, T* __restrict__ Qp,
                                                      T* __restrict__ KV, T* __restrict__ bias, uint32_t N,
                                                      uint32_t ldn, float eps, float qscale, float bias_scale,
                                                      uint32_t ntiles, FastDiv nkbd, int dh) {
  constexpr int D = 32, H = 4, ROW = C * 2, KS = C / 16;
  constexpr int LPT = C / 8;       // loader lanes per token row (16 bytes each)
  constexpr int TPP = 256 / LPT;   // tokens per loader pass
  constexpr int NP = 64 / TPP;     // loader passes per tile
  constexpr int PD = 4;            // loader register stages in flight
  constexpr int PART = 64 * D * 2; // bytes of one head's Q, K or V^T block of a tile
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;

  __shared__ __attribute__((aligned(16))) char xs[2][64 * ROW];    // normalised x tiles
  __shared__ __attribute__((aligned(16))) char os[H][3 * PART];   // per writer wave: Q | K | V^T
  // pair bias [head][position]: head rows 72 elements apart (dword banks 0 / 36 / 8 / 44), so the
  // four heads' stores of a pass fall in distinct banks
  constexpr int BSR = 72;
  __shared__ __attribute__((aligned(16))) T bs[2][H * BSR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t nkb = ldn / 64, nkt = ldn / 32, nqt = (N + 31) / 32;
  const uint32_t G = gridDim.x;
  uint32_t t = blockIdx.x;

  if (wave < 4) {
    // ================= loaders =================
    const int ch = tid % LPT, tq = tid / LPT;  // 16-byte chunk ch of tokens TPP k + tq, k < NP
    V8 lnw = {}, lnb = {}, wz[H];
    if constexpr (LN) {
      lnw = ldg<V8>(w_ln + 8 * ch);
      if (b_ln) lnb = ldg<V8>(b_ln + 8 * ch);
    }
#pragma unroll
    for (int hh = 0; hh < H; ++hh) wz[hh] = ldg<V8>(WZ + hh * C + 8 * ch);
    const float bz = BZ ? BZ[ch & 3] : 0.f;
    struct Stage {
      V8 x[NP];
    };
    auto fetch = [&](uint32_t tt, Stage& sg) {
      tt = tt < ntiles ? tt : ntiles - 1;
      const uint32_t i = nkbd.div(tt), kb = tt - i * nkb;
      const T* row = x + (int64_t)i * sx0 + 8 * ch;
#pragma unroll
      for (int k = 0; k < NP; ++k) {
        uint32_t p = kb * 64 + TPP * k + tq;
        p = p < N ? p : N - 1;
        sg.x[k] = ldg<V8>(row + (int64_t)p * sx1);
      }
    };
    auto step = [&](uint32_t tt, int bb, Stage& sg) {
      const uint32_t kb = tt - nkbd.div(tt) * nkb;
#pragma unroll
      for (int k = 0; k < NP; ++k) {
        const int tk = TPP * k + tq;
        const bool valid = kb * 64 + tk < N;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = valid ? (float)sg.x[k][e] : 0.f;
        if constexpr (LN) {  // two-pass statistics over the token's LPT lanes
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) s += v[e];
          const float mean = group_sum<LPT>(s) * (1.0f / C);
          float q = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) q = fmaf(v[e] - mean, v[e] - mean, q);
          const float rstd = rsqrtf(group_sum<LPT>(q) * (1.0f / C) + eps);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (v[e] - mean) * rstd * (float)lnw[e] + (float)lnb[e];
        }
        // pair bias of the 4 heads (fp32 dot products); lanes ch, ch + 4, ... all hold head ch & 3,
        // and lane ch < 4 stores it
        float bsel = 0.f;
#pragma unroll
        for (int hh = 0; hh < H; ++hh) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(v[e], (float)wz[hh][e], d);
          d = group_sum<LPT>(d);
          bsel = (ch & 3) == hh ? d : bsel;
        }
        if (ch < 4) bs[bb][ch * BSR + tk] = valid ? (T)((bsel + bz) * bias_scale) : (T)0.f;
        V8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (T)v[e];
        *reinterpret_cast<V8*>(&xs[bb][tk * ROW + ((ch ^ row_key<C>(tk)) << 4)]) = o;
      }
      __syncthreads();  // tile tt staged; the writers are done with the tile before tt - 1
      fetch(tt + PD * G, sg);  // refill this stage
      __builtin_amdgcn_sched_barrier(0);
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
    uint32_t n = (ntiles - t + G - 1) / G;
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
    // ================= writers: wave 4 + h owns head h =================
    const int h = wave - 4, hl = lane >> 5, col = lane & 31;
    // weight rows (H, 3, dh, C): row col < dh of head h's Q, K and V blocks; rows col >= dh
    // (a head narrower than 32) are zeros and are not read
    V8 wq[KS], wk[KS], wv[KS];
    {
      const bool live = col < dh;
      const T* wh = wqkv + ((int64_t)h * 3 * dh + (live ? col : 0)) * C + 8 * hl;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        wq[s] = live ? ldg<V8>(wh + 16 * s) : V8{};
        wk[s] = live ? ldg<V8>(wh + (int64_t)dh * C + 16 * s) : V8{};
        wv[s] = live ? ldg<V8>(wh + 2 * (int64_t)dh * C + 16 * s) : V8{};
      }
    }
    char* oh = os[h];
    int bb = 0;
    for (; t < ntiles; t += G) {
      __syncthreads();  // tile t staged
      // Q^T = WQ . x^T and K^T (lane -> position, slots -> d), V = x . WV^T (lane -> d, slots
      // -> positions).  Slot v = 8 j + e of lane half hl is element 16 j + 8 hl + e of the
      // permuted group of 32: 16-byte chunk 2 j + hl of the position's (or d's) 32 elements.
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int tp = sub * 32 + col;
        f32x16 aq = {}, ak = {}, av = {};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const V8 xb = *reinterpret_cast<const V8*>(&xs[bb][tp * ROW + (((2 * s + hl) ^ row_key<C>(tp)) << 4)]);
          aq = Mma<T>::m32(wq[s], xb, aq);
          ak = Mma<T>::m32(wk[s], xb, ak);
          av = Mma<T>::m32(xb, wv[s], av);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          V8 q, k, v;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            q[e] = (T)(aq[8 * j + e] * qscale);
            k[e] = (T)ak[8 * j + e];
            v[e] = (T)av[8 * j + e];
          }
          // Q / K rows are 64 bytes (4 chunks, swizzled by (row >> 2) & 3), V^T rows 128 bytes
          // (8 chunks, swizzled by (row >> 1) & 7): 16 lanes of a store hit 16 distinct chunks
          const int cq = (2 * j + hl) ^ ((tp >> 2) & 3);
          *reinterpret_cast<V8*>(oh + tp * 64 + (cq << 4)) = q;
          *reinterpret_cast<V8*>(oh + PART + tp * 64 + (cq << 4)) = k;
          const int cv = (4 * sub + 2 * j + hl) ^ ((col >> 1) & 7);
          *reinterpret_cast<V8*>(oh + 2 * PART + col * 128 + (cv << 4)) = v;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t i = nkbd.div(t), kb = t - i * nkb;
      const uint64_t ih = (uint64_t)i * H + h;
      T* qdst = Qp + (ih * ldn + kb * 64) * D;
      T* kvdst = KV + (ih * nkb + kb) * kKVBlock;
#pragma unroll
      for (int part = 0; part < 3; ++part) {
        T* dst = part == 0 ? qdst : kvdst + (part - 1) * 64 * D;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ci = r * 64 + lane;  // 16-byte chunk of the 4 KB block
          int a;
          if (part < 2) {
            const int row = ci >> 2, c = ci & 3;
            a = row * 64 + ((c ^ ((row >> 2) & 3)) << 4);
          } else {
            const int row = ci >> 3, c = ci & 7;
            a = row * 128 + ((c ^ ((row >> 1) & 7)) << 4);
          }
          stg<V8>(dst + 8 * ci, *reinterpret_cast<const V8*>(oh + part * PART + a));
        }
      }
      if (lane < 8) {  // bias: lane g stores chunk (j, hl) = ((g >> 1) & 1, g & 1) of query i in key
        // tile 2 kb + (g >> 2): positions 16 j + 4 hl + 0..3 and + 8 of that tile (16 bytes)
        const int g = lane, kt = g >> 2, j = (g >> 1) & 1, hh = g & 1;
        const uint64_t off = (((uint64_t)h * nqt + i / 32) * nkt + 2 * kb + kt) * 1024 + (j * 64 + hh * 32 + (i & 31)) * 8;
        const T* src = &bs[bb][h * BSR + 32 * kt + 16 * j + 4 * hh];
        const V4 lo = *reinterpret_cast<const V4*>(src), hi = *reinterpret_cast<const V4*>(src + 8);
        stg<V8>(bias + off, V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
      }
      bb ^= 1;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Attention core.  NW waves (4, two blocks per CU; or 8 from N = TRI_NW8_MIN_N on, one block per
// CU: each KV block copied into LDS then serves twice the queries), QT query tiles (32 queries)
// per wave, 64-key blocks of two 32-key tiles.  Both block sizes give the same bits.
//
// Per (32-key tile, query tile) a wave runs
//     S^T  = bias + C0 + K . Q^T      2 MFMAs, K from LDS, Q^T in registers; the accumulator
//                                     starts at the lane's 16 bias values (bias_acc)
//     P    = exp2(S^T)                16 v_exp per lane, no max / subtract per element
//     O^T += V^T . P^T                2 MFMAs, V^T from LDS, P^T = S^T's D registers
//     l   += 1 . P^T                  2 16x16x32 MFMAs on the same P^T (bf16; row_sum_selector)
// Softmax is invariant to a per-row shift m of the scores; m only keeps exp2 in range.
//   bf16 (OPT): m = 0 throughout.  bf16 has fp32's exponent range, so P = 2^s, the row sums and
//   O stay exact in relative terms for scores s in about (-60, 100) (log2 units); the row sum l
//   (fp32 sums of the rounded weights the PV product uses, by the matrix cores) is checked once
//   at the end, and a wave whose l left [2^-60, 2^100] (or is not finite) recomputes its tiles
//   with an exact running max (tri_exact_tile, out of line).  The loop itself then has no max,
//   no subtraction and no per-tile overflow test (C0 = 0).
//   fp16: C0 = -m (the running row max, broadcast) is added to the initialiser.  m is
//   exact from the first tile with a valid key on and is only raised when a tile's
//   probabilities could overflow fp16 (then O and l are rescaled and the tile recomputed).
// Masked keys get probability exactly 0 (equal to the reference's exp(-1e9 - m) in fp32
// whenever the row has a valid key); a row without valid keys takes the uniform average of V
// over all N keys, as the reference's -1e9 add gives.  Keys >= N hold zero bias (the pre-pass and
// the repack write zeros) and are masked like the others.
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

// A row whose keys are all masked: the reference adds -1e9 to every score, which leaves them all
// equal in fp32, so each key k < N weighs exactly 1 and each key >= N 0, in every query column
// alike: O[q] = (sum over k < N of V[k]) / N, one vector for the whole row.  The waves of the
// block split the visited blocks (wave w takes w, w + nw, ...; two blocks' loads in flight per
// lane), each lane (d = lane % 32, key half lane / 32) adds its 32 positions of the block's V^T
// row d in fp32, the halves and waves are added through LDS, and each wave writes its query tiles.
// Every wave of the block calls this (one block barrier inside).  Kept out of line so the main
// loop's register allocation does not see it.
template <typename T, int QT>
__device__ __noinline__ void tri_uniform_row(const T* __restrict__ kvrow, const short* vblk, int nv, int64_t N,
                                             T* __restrict__ out, int64_t i, int64_t so0, int64_t so1, int h,
                                             int dv, int64_t qbase, int lane) {
  constexpr int D = 32;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;
  __shared__ __attribute__((aligned(16))) float usum[16][D];  // per wave (<= 16 waves), per d
  const int nw = (int)(blockDim.x >> 6), wave = (int)(threadIdx.x >> 6);
  const int hl = lane >> 5, col = lane & 31;
  constexpr int NB = 2;  // blocks whose loads are in flight together per lane
  float acc = 0.f;
  for (int j0 = wave; j0 < nv; j0 += NB * nw) {
    V8 r[NB][4];
    int kbs[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int j = j0 + b * nw;
      kbs[b] = j < nv ? (int)vblk[j] : -1;
      const T* vt = kvrow + (int64_t)(kbs[b] < 0 ? 0 : kbs[b]) * kKVBlock + 64 * D + col * 64 + 8 * hl;
#pragma unroll
      for (int c = 0; c < 4; ++c) r[b][c] = ldg<V8>(vt + 16 * c);  // positions 16 c + 8 hl + e
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (kbs[b] < 0) continue;  // wave-uniform
      const int64_t nk = N - 64LL * kbs[b];  // keys < N in this block (>= 1: it was visited)
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // V^T position 32 kt + 16 jj + 8 hl + e (c = 2 kt + jj) holds key 32 kt + 16 jj + 8 (e / 4) + 4 hl + e % 4
          const int key = 16 * c + 8 * (e / 4) + 4 * hl + (e % 4);
          acc += key < nk ? (float)r[b][c][e] : 0.f;
        }
    }
  }
  acc = halves_sum(acc);
  if (hl == 0) usum[wave][col] = acc;
  __syncthreads();
  // O = sum / N for every query of the wave; lane (query col, half hl) stores d = 8 g + 4 hl + x
  const float inv = 1.0f / (float)N;
  f32x4 m[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    m[g] = f32x4{};
    for (int w = 0; w < nw; ++w) m[g] += *reinterpret_cast<const f32x4*>(&usum[w][8 * g + 4 * hl]);
  }
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int64_t q = qbase + 32 * t + col;
    if (q < N) {
      T* dst = out + i * so0 + q * so1 + (int64_t)h * dv + 4 * hl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (8 * g >= dv) break;
        V4 w4 = {(T)(m[g][0] * inv), (T)(m[g][1] * inv), (T)(m[g][2] * inv), (T)(m[g][3] * inv)};
        stg<V4>(dst + 8 * g, w4);
      }
    }
  }
}

// Row sums of the weights on the matrix cores.  One v_mfma_f32_16x16x32 per 16-key half takes the
// P^T operand of the PV product as its B (as a 32x32x16 B, lane L holds keys 8 (L / 32) + e of
// query L % 32; read as a 16x16x32 B, rows 8 (L / 16) + e of column L % 16) against this 0/1
// selector as A: its rows 0 and 8 add up the B rows that belong to queries 0-15 (L / 16 even),
// rows 4 and 12 those of queries 16-31 (L / 16 odd).  The D element in row 4 (L / 16), column
// L % 16 -- slot 0 of lane L -- then accumulates the sum of query L % 32's rounded weights, in
// every lane, with fp32 adds inside the matrix core and no VALU work.
template <typename T>
__device__ inline vec<T, 8> row_sum_selector(int lane) {
  const int m = lane & 15, g = lane >> 4;  // A row m, k rows 8 g .. 8 g + 7
  const bool one = ((m == 0 || m == 8) && (g & 1) == 0) || ((m == 4 || m == 12) && (g & 1) == 1);
  vec<T, 8> a;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = (T)(one ? 1.f : 0.f);
  return a;
}

// The 16 fp32 bias values of a lane's score slots (D layout of a 32 x 32 score tile: slot v =
// 8 j + e is element e of the tile's 16-byte load j), exactly widened from the 16-bit tile; they
// initialise the score MFMAs' accumulator, so S = bias + K . Q^T with no MFMA spent on the bias.
template <typename T>
__device__ inline f32x16 bias_acc(vec<T, 8> b0, vec<T, 8> b1) {
  f32x16 c;
  if constexpr (std::is_same<T, __bf16>::value) {  // bf16 -> fp32 is a 16-bit shift
    const auto w0 = __builtin_bit_cast(vec<uint32_t, 4>, b0), w1 = __builtin_bit_cast(vec<uint32_t, 4>, b1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      c[2 * e] = __uint_as_float(w0[e] << 16);
      c[2 * e + 1] = __uint_as_float(w0[e] & 0xffff0000u);
      c[8 + 2 * e] = __uint_as_float(w1[e] << 16);
      c[8 + 2 * e + 1] = __uint_as_float(w1[e] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      c[e] = (float)b0[e];
      c[8 + e] = (float)b1[e];
    }
  }
  return c;
}

// One query tile (32 queries of row i, head h) recomputed with an exact running max: the
// classic online softmax over the visited tiles in the main loop's order, its operands read from
// global memory (K and V^T from the row's KV blocks, whose rows are 32 / 64 elements wide there,
// the bias tile, Q^T in registers).  For the waves of the bf16 kernel whose shift-free row sums
// left their safe range (scores beyond about +-60 / 100 in log2 units); out of line, so the main
// loop's register allocation does not see it.  `bqt`: this lane's bias operand address in the
// tile (query tile, key tile 0), as the main loop's bq.
template <typename T>
__device__ __noinline__ void tri_exact_tile(const T* __restrict__ kvrow, const T* __restrict__ bqt,
                                            vec<T, 8> q0, vec<T, 8> q1,
                                            const short* vblk, const unsigned long long* kvalid, int nv, int64_t N,
                                            T* __restrict__ out, int64_t i, int64_t so0, int64_t so1, int h, int dv,
                                            int64_t q, int lane) {
  constexpr int D = 32;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;
  const int hl = lane >> 5, col = lane & 31;
  f32x16 o = {};
  float m = -INFINITY, l = 0.f;
  for (int j = 0; j < nv; ++j) {
    const int kb = vblk[j];
    const unsigned long long kbits = kvalid[kb];
    for (int kt = 0; kt < 2; ++kt) {
      const unsigned int tb = (unsigned int)(kbits >> (32 * kt));
      if (tb == 0) continue;  // wave-uniform: no valid key in this tile
      const T* kr = kvrow + (int64_t)kb * kKVBlock + (32 * kt + col) * D + 8 * hl;
      const T* vr = kvrow + (int64_t)kb * kKVBlock + 64 * D + col * 64 + 32 * kt + 8 * hl;
      const T* br = bqt + (int64_t)(2 * kb + kt) * 1024;
      f32x16 s = bias_acc<T>(ldg<V8>(br), ldg<V8>(br + 512));
      s = Mma<T>::m32(ldg<V8>(kr), q0, s);
      s = Mma<T>::m32(ldg<V8>(kr + 16), q1, s);
      const unsigned int lb = tb >> (4 * hl);
      float mt = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s[v] = ((lb >> (8 * (v / 4) + (v % 4))) & 1u) ? s[v] : -INFINITY;
        mt = fmaxf(mt, s[v]);
      }
      const float mn = fmaxf(m, halves_max(mt));  // finite: the tile has a valid key
      const float alpha = fast_exp2(m - mn);      // 0 before the first valid tile (m = -inf)
      o *= alpha;
      l *= alpha;
      V8 p0, p1;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const float e0 = fast_exp2(s[v] - mn), e1 = fast_exp2(s[8 + v] - mn);
        p0[v] = (T)e0;
        p1[v] = (T)e1;
        l += e0 + e1;
      }
      o = Mma<T>::m32(ldg<V8>(vr), p0, o);
      o = Mma<T>::m32(ldg<V8>(vr + 16), p1, o);
      m = mn;
    }
  }
  const float inv = 1.0f / halves_sum(l);
  if (q < N) {
    T* dst = out + i * so0 + q * so1 + (int64_t)h * dv + 4 * hl;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (8 * g >= dv) break;
      V4 w4 = {(T)(o[4 * g] * inv), (T)(o[4 * g + 1] * inv), (T)(o[4 * g + 2] * inv), (T)(o[4 * g + 3] * inv)};
      stg<V4>(dst + 8 * g, w4);
    }
  }
}

template <typename T, int QT, int NW>
__global__ __launch_bounds__(64 * NW, TRI_WPE(QT, NW)) void tri_attn_kernel(const T* __restrict__ Qp, const T* __restrict__ KV,
                                                         const T* __restrict__ bias, const int8_t* __restrict__ mask,
                                                         int64_t sm0, int64_t sm1, T* __restrict__ out, int64_t so0,
                                                         int64_t so1, int64_t N, int64_t ldn, int H, int nqc,
                                                         int dv) {
  constexpr int D = 32;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves per block");
  constexpr int KVR = 8 / NW;  // 16-byte chunks of a KV block per thread
#ifndef TOPS_TRI_EXACT_MAX
  constexpr bool OPT = std::is_same<T, __bf16>::value;  // shift-free softmax (bf16), see above
#else
  constexpr bool OPT = false;
#endif
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;

  __shared__ __attribute__((aligned(16))) T kvs[3][kKVLds];
  __shared__ unsigned long long kvalid[kMaxKB];  // per 64-key block (N <= kMaxN)
  __shared__ short vblk[kMaxKB];                 // indices of blocks with a valid key
  __shared__ int nvblk, row_any;
  // 4-wave blocks, per wave: its QT query tiles of O (32 queries x 32 d each) on the way to HBM
  __shared__ __attribute__((aligned(16))) T ostg[NW == 4 ? NW : 1][NW == 4 ? QT * 32 * 32 : 8];

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

  const T* kvrow = KV + ((int64_t)i * H + h) * nkb * kKVBlock;
  const int64_t nqt = (N + 31) / 32;

  // ---- the mask bytes of the wave's first kMaskU key blocks (wave + u NW), loaded first: vector
  // ---- loads complete in issue order, so their wait does not include the Q, bias and KV loads
  // ---- issued after them (a loop with one load per block waited for all of those each time) ----
  constexpr int kMaskU = 8;
  int mval[kMaskU];
#pragma unroll
  for (int u = 0; u < kMaskU; ++u) {
    const int64_t k = (int64_t)(wave + u * NW) * 64 + lane;
    mval[u] = 0;
    if (wave + u * NW < nkb && k < N) mval[u] = mask ? (int)mask[i * sm0 + k * sm1] : 1;
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- Q^T operands (already scaled by scale * log2 e and d-permuted) and bias pointers, loaded
  // ---- before the key-validity pass so the loads overlap it (a row without valid keys skips
  // ---- the main loop: tri_uniform_row below) ----
  const int64_t qbase = (int64_t)qc * (NW * 32 * QT) + (int64_t)wave * 32 * QT;
  V8 qop[QT][2];
  const T* bq[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    int64_t q = qbase + 32 * t + col;
    q = q < N ? q : N - 1;
    const T* qr = Qp + (((int64_t)i * H + h) * ldn + q) * D + 8 * hl;
    qop[t][0] = ldg<V8>(qr);
    qop[t][1] = ldg<V8>(qr + 16);
    bq[t] = bias + ((int64_t)h * nqt + q / 32) * (2 * nkb) * 1024 + (32 * hl + q % 32) * 8;
  }

  // KV block copy (8 KiB: 256 chunks of K, then 256 of V^T, 16 bytes each): with 4 waves thread t
  // moves chunks t (K: row t / 4) and 256 + t (V^T: row t / 8); with 8 waves, chunk t (waves 0-3
  // K, waves 4-7 V^T).  Each load instruction of a wave reads 1 KB contiguous.
  auto kv_load = [&](int kb, V8* r) {
    const T* src = kvrow + (int64_t)kb * kKVBlock + 8 * tid;
    r[0] = ldg<V8>(src);
    if constexpr (KVR == 2) r[1] = ldg<V8>(src + 64 * D);
  };
  auto kv_store = [&](int buf, const V8* r) {
    if (KVR == 2 || tid < 256)  // wave-uniform
      *reinterpret_cast<V8*>(&kvs[buf][(tid / 4) * kKPad + 8 * (tid % 4)]) = r[0];
    const int tv = KVR == 2 ? tid : tid - 256;  // V^T chunk of this thread
    if (KVR == 2 || tid >= 256)
      *reinterpret_cast<V8*>(&kvs[buf][64 * kKPad + (tv / 8) * kVPad + 8 * (tv % 8)]) = r[KVR - 1];
  };
  // bias B operands of one 32-key tile: [query tile t][half j], 16 bytes per lane
  auto load_bias = [&](int kb, int kt, V8 (*bb)[2]) {
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) bb[t][j] = ldg<V8>(bq[t] + (int64_t)(2 * kb + kt) * 1024 + 512 * j);
  };
  // The first visited block is block 0 unless all its keys are masked: its KV and bias operands
  // are loaded now, speculatively, and reloaded below in the rare other case.
  V8 bA[QT][2], bB[QT][2];
  V8 kvA[KVR], kvB[KVR];
  kv_load(0, kvA);
  load_bias(0, 0, bA);
  load_bias(0, 1, bB);

  // ---- key validity per 64-key block ----
#pragma unroll
  for (int u = 0; u < kMaskU; ++u) {
    const int kb = wave + u * NW;
    const unsigned long long bits = __ballot(mval[u] != 0);
    if (kb < nkb && lane == 0) kvalid[kb] = bits;
  }
  for (int kb = wave + kMaskU * NW; kb < nkb; kb += NW) {  // N > 64 kMaskU NW
    const int64_t k = (int64_t)kb * 64 + lane;
    bool ok = k < N;
    if (ok && mask) ok = mask[i * sm0 + k * sm1] != 0;
    const unsigned long long bits = __ballot(ok);
    if (lane == 0) kvalid[kb] = bits;
  }
  __syncthreads();
  // ---- wave 0: the list of blocks to visit, compacted 64 blocks per step (ballot + prefix
  // ---- count); a row without valid keys visits every block with keys < N ----
  if (wave == 0) {
    unsigned long long seen = 0;
    for (int g = 0; g < nkb; g += 64) seen |= __ballot(g + lane < nkb && kvalid[g + lane] != 0);
    const bool unif = seen == 0;
    int n = 0;
    for (int g = 0; g < nkb; g += 64) {
      const int kb = g + lane;
      bool vis = false;
      if (kb < nkb) {
        if (unif) kvalid[kb] = (N - 64LL * kb >= 64) ? ~0ull : ((1ull << (N - 64LL * kb)) - 1ull);
        vis = kvalid[kb] != 0;
      }
      const unsigned long long bal = __ballot(vis);
      const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
      if (vis) vblk[n + pos] = (short)kb;
      n += __popcll(bal);
    }
    if (lane == 0) {
      nvblk = n;
      row_any = unif ? 0 : 1;
    }
  }
  __syncthreads();
  const bool uniform = row_any == 0;  // no valid key: every score is -1e9, weights 1/N
  const int nv = nvblk;               // >= 1 whenever N >= 1
  if (uniform) {  // block-uniform: the mean of V over the N keys, without the main loop
    tri_uniform_row<T, QT>(kvrow, vblk, nv, N, out, i, so0, so1, h, dv, qbase, lane);
    return;
  }

  f32x16 o[QT], cinit[QT];
  float l[QT];   // fp16: row sums (lanes l and l ^ 32 hold halves)
  f32x4 ls[QT];  // bf16: row sums accumulated by the matrix cores, slot 0 = the query's whole sum
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    o[t] = f32x16{};
    cinit[t] = f32x16{};
    l[t] = 0.f;
    ls[t] = f32x4{};
  }
  bool first = true;
  const V8 lsel = row_sum_selector<T>(lane);  // bf16: row sums on the matrix cores

  // scores of one 32-key tile for all query tiles
  auto scores = [&](const V8* kop, V8 (*bb)[2], f32x16* s) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      f32x16 c = bias_acc<T>(bb[t][0], bb[t][1]);
      if constexpr (!OPT) c += cinit[t];
      s[t] = Mma<T>::m32(kop[0], qop[t][0], c);
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
      if constexpr (OPT) {
        // weights 2^s; their row sums go to the matrix cores with the PV product below
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          p[t][0][v] = (T)fast_exp2(s[t][v]);
          p[t][1][v] = (T)fast_exp2(s[t][8 + v]);
        }
        ps[t] = 0.f;
      } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          p[t][0][v] = (T)fast_exp2(s[t][v]);
          p[t][1][v] = (T)fast_exp2(s[t][8 + v]);
        }
        // row sum of the rounded weights the PV product uses (packed dot products)
        ps[t] = sum8<T>(p[t][0], 0.f) + sum8<T>(p[t][1], 0.f);
        over |= !(ps[t] <= Mma<T>::kMaxP);
      }
      pin(p[t][0]);
      pin(p[t][1]);
    }
    // VALU instructions per score MFMA in the interleave (exponentials, converts and the next
    // tile's bias widening)
    constexpr int VPM = OPT ? (NW == 4 ? 24 : 20) : 26;
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
    for (int m = 0; m < QT; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, VPM, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 2 * QT, 0);
#pragma unroll
    for (int m = 0; m < QT; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, VPM, 0);
    }
    // ---- rare (fp16): the first tile with a valid key sets the exact max; later tiles raise it
    // ---- only when a probability could overflow the I/O type ----
    const bool rare = !OPT && ((__ballot(over) != 0) | (first & (tb != 0)));
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
      o[t] = Mma<T>::m32(vop[0], p[t][0], o[t]);
      o[t] = Mma<T>::m32(vop[1], p[t][1], o[t]);
      if constexpr (OPT) {
        ls[t] = Mma<T>::m16(lsel, p[t][0], ls[t]);
        ls[t] = Mma<T>::m16(lsel, p[t][1], ls[t]);
      } else {
        l[t] += ps[t];
      }
    }
  };

  // Tiles (j, 0), (j, 1) of the visited blocks j in order.  Scores of tile (j, 0) live in sA,
  // of (j, 1) in sB, their bias operands in bA / bB, each loaded two tiles ahead.  KV blocks
  // rotate through three LDS buffers (the buffer written at block j was last read before the
  // previous barrier) and are loaded into registers two blocks ahead.  One barrier per block.
  // Past the last block the pipeline recomputes a tile of the last block (results unused).
  f32x16 sA[QT], sB[QT];
  auto blk = [&](int j) { return (int)vblk[j < nv ? j : nv - 1]; };
  if (blk(0) != 0) {  // block-uniform: block 0 has no valid key
    kv_load(blk(0), kvA);
    load_bias(blk(0), 0, bA);
    load_bias(blk(0), 1, bB);
  }
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

  // ---- bf16: a wave whose shift-free row sums left [2^-60, 2^100] (or are not finite: a
  // ---- weight overflowed) recomputes its query tiles with an exact running max ----
  if constexpr (OPT) {
    bool bad = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const float lt = ls[t][0];
      bad |= !(lt >= 0x1p-60f && lt <= 0x1p100f);
    }
    if (__ballot(bad) != 0) {  // wave-uniform
#pragma unroll
      for (int t = 0; t < QT; ++t)
        tri_exact_tile<T>(kvrow, bq[t], qop[t][0], qop[t][1], vblk,
                          kvalid, nv, N, out, i, so0, so1, h, dv, qbase + 32 * t + col, lane);
      return;
    }
  }
  // ---- normalise and store O[i, q, h*dv + d], d < dv: the head's first dv of its 32 lanes
  // ---- (dv < 32 when the head is narrower and its Q / K / V are zero-padded to 32).  dv = 32 in
  // ---- 4-wave blocks: through the wave's LDS tile (16-byte chunk g of query row r at g ^ (r & 3)),
  // ---- so each store instruction writes 16 queries' whole 64-byte head segments instead of 32
  // ---- queries' 16-byte pieces (0.903 -> 0.883 ms at N = 1024; no gain in the 8-wave blocks) ----
  if constexpr (NW == 4) {
    if (dv == D) {
      T* sb = ostg[wave];
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const float inv = 1.0f / (OPT ? ls[t][0] : halves_sum(l[t]));
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const V4 w4 = {(T)(o[t][4 * g] * inv), (T)(o[t][4 * g + 1] * inv), (T)(o[t][4 * g + 2] * inv),
                         (T)(o[t][4 * g + 3] * inv)};
          *reinterpret_cast<V4*>(&sb[(t * 32 + col) * 32 + ((g ^ (col & 3)) << 3) + 4 * hl]) = w4;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int t = 0; t < QT; ++t) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int r = 16 * u + (lane >> 2), c = lane & 3;
          const int64_t q = qbase + 32 * t + r;
          const V8 v = *reinterpret_cast<const V8*>(&sb[(t * 32 + r) * 32 + ((c ^ (r & 3)) << 3)]);
          if (q < N) stg<V8>(out + i * so0 + q * so1 + (int64_t)h * D + 8 * c, v);
        }
      }
      return;
    }
  }
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int64_t q = qbase + 32 * t + col;
    const float inv = 1.0f / (OPT ? ls[t][0] : halves_sum(l[t]));
    if (q < N) {
      T* dst = out + i * so0 + q * so1 + (int64_t)h * dv + 4 * hl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (8 * g >= dv) break;  // wave-uniform: slots 4 g .. 4 g + 3 hold d = 8 g + 4 hl + 0..3
        V4 w4 = {(T)(o[t][4 * g] * inv), (T)(o[t][4 * g + 1] * inv), (T)(o[t][4 * g + 2] * inv),
                 (T)(o[t][4 * g + 3] * inv)};
        stg<V4>(dst + 8 * g, w4);
      }
    }
  }
}
// ---------------------------------------------------------------------------------------------
// Attention core, two rows per wave (bf16, D = 32).  A block = 4 waves = rows (i0, i1 = i0 + 1) x
// 128 queries of one head; wave w owns query tile qt = 4 qc + w of both rows.  Per 32-key tile the
// wave runs, for row r = 0 then 1 (a "stage" each):
//     S_r^T = I . B^T + K_r . Q_r^T              4 MFMAs
//     P_r   = 2^(S_r^T)                          16 v_exp, 8 packed converts
//     O_r^T += V_r^T . P_r^T, l_r += 1 . P_r^T    2 MFMAs + 2 16x16x32 MFMAs (row_sum_selector)
// with the one-row kernel's shift-free softmax (weights 2^s, row sums l checked once at the end;
// a wave whose l left [2^-60, 2^100] recomputes its tiles with an exact running max).  The bias
// operand B (16 bytes per lane and half) is loaded once per tile for both rows, so a bias tile costs
// 1 KB of L2 reads per 32 x 32 (row, query, key) tile instead of 2 KB.  K and V^T of both rows go
// straight into LDS with the compiler's global_load_lds builtin (1 KB per wave instruction; the
// compiler sets M0 and inserts the wait states and the waits its own reads of a slot need), each
// lane fetching the 16-byte chunk that belongs at its LDS position under the operand reads' XOR
// swizzle (K rows 64 B: chunk ^ ((key >> 2) & 3); V^T rows 128 B: chunk ^ ((d >> 1) & 7)), so the
// operand reads are free of bank conflicts without padding.  A ring of 4 LDS slots of 64-key
// blocks, one barrier per block, copies issued three blocks ahead.  Stages are software-pipelined:
// stage (row r, tile t) issues the PV MFMAs of the previous stage and the score MFMAs of the next
// one (the other row) between its own exponentials.  A row without valid keys (the uniform average
// of V over the N keys, as the reference's -1e9 add gives) runs in the loop when its pair partner
// has valid keys, its result unused, and its O is then written by tri_uniform_row.
// Masked keys get weight exactly 0.
// ---------------------------------------------------------------------------------------------
constexpr int kRing = 4;  // LDS slots of 64-key KV blocks (per block: 2 rows x 8 KB each)
template <int V>
using IC = std::integral_constant<int, V>;

template <typename T>
__global__ __launch_bounds__(256, 2) void tri_attn2_kernel(const T* __restrict__ Qp, const T* __restrict__ KV,
                                                          const T* __restrict__ bias, const int8_t* __restrict__ mask,
                                                          int64_t sm0, int64_t sm1, T* __restrict__ out, int64_t so0,
                                                          int64_t so1, int N, int ldn, int H, int nqc, int nrp) {
  constexpr int D = 32, NW = 4, KVB = kKVBlock * 2;  // bytes of one (row, 64-key) KV block
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;
  using LdsPtr = __attribute__((address_space(3))) void*;

  // four separate arrays, indexed at compile time: the compiler then sees that the LDS reads of
  // one slot do not alias the asynchronous copies into the others
  __shared__ __attribute__((aligned(16))) char slot0[2][KVB];
  __shared__ __attribute__((aligned(16))) char slot1[2][KVB];
  __shared__ __attribute__((aligned(16))) char slot2[2][KVB];
  __shared__ __attribute__((aligned(16))) char slot3[2][KVB];
  __shared__ unsigned long long kvalid[2][kMaxKB];
  __shared__ short vblk[kMaxKB];
  __shared__ int nvblk, row_any[2];
  auto slot = [&](auto sc) -> char(*)[KVB] {
    constexpr int S = decltype(sc)::value;
    if constexpr (S == 0) return slot0;
    else if constexpr (S == 1) return slot1;
    else if constexpr (S == 2) return slot2;
    else return slot3;
  };

  // ---- block -> (head, row pair, query chunk), XCD-aware: consecutive ids on one XCD share
  // ---- the head (its bias stays in that XCD's L2) and each row pair's chunks run together.
  const int total = H * nrp * nqc;
  int id = blockIdx.x;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  const int qc = id % nqc, rp = (id / nqc) % nrp, h = id / (nqc * nrp);
  const int i0 = 2 * rp, i1v = 2 * rp + 1, i1 = i1v < N ? i1v : N - 1;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int nkb = ldn / 64, nqt = (N + 31) / 32, nkt = ldn / 32;
  const int qt = qc * NW + wave;

  // ---- Q^T operands of both rows (scaled, d-permuted), loaded before the key-validity pass and
  // ---- waited for after it, before the main loop's loads (which the compiler does not track) ----
  const int irow[2] = {i0, i1};
  int q = 32 * qt + col;
  q = q < N ? q : N - 1;
  V8 qop[2][2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const T* qr = Qp + (((int64_t)irow[r] * H + h) * ldn + q) * D + 8 * hl;
    qop[r][0] = ldg<V8>(qr);
    qop[r][1] = ldg<V8>(qr + 16);
  }

  // ---- key validity of both rows per 64-key block; the visit list is their union ----
  if (tid < 2) row_any[tid] = 0;
  __syncthreads();
  for (int idx = wave; idx < 2 * nkb; idx += NW) {
    const int r = idx & 1, kb = idx >> 1;
    const int64_t k = 64LL * kb + lane;
    bool ok = k < N;
    if (ok && mask) ok = mask[(int64_t)(r ? i1 : i0) * sm0 + k * sm1] != 0;
    const unsigned long long bits = __ballot(ok);
    if (lane == 0) {
      kvalid[r][kb] = bits;
      if (bits) row_any[r] = 1;
    }
  }
  __syncthreads();
  const bool uni[2] = {row_any[0] == 0, row_any[1] == 0};  // no valid key: weights 1/N
  if (tid == 0) {
    int n = 0;
    for (int kb = 0; kb < nkb; ++kb) {
      const unsigned long long all = (N - 64 * kb >= 64) ? ~0ull : ((1ull << (N - 64 * kb)) - 1ull);
      if (uni[0]) kvalid[0][kb] = all;
      if (uni[1]) kvalid[1][kb] = all;
      if (kvalid[0][kb] | kvalid[1][kb]) vblk[n++] = (short)kb;
    }
    nvblk = n;
  }
  __syncthreads();
  const int nv = nvblk;  // >= 1 whenever N >= 1
  // visit j's block and its valid-key bits of both rows, held by lane j of every wave (nv <= 64,
  // N <= 4096) and read with v_readlane in the loop: no LDS reads there besides the K / V operands
  // (the compiler orders LDS reads it cannot separate from the asynchronous copies behind them)
  const int mj = lane < nv ? lane : nv - 1;
  const int vb_l = vblk[mj];
  const unsigned long long kv0_l = kvalid[0][vb_l], kv1_l = kvalid[1][vb_l];
  auto visit = [&](int vj) { return __builtin_amdgcn_readlane(vb_l, vj < nv ? vj : nv - 1); };
  auto bits64 = [&](unsigned long long v, int vj) {
    return ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), vj) << 32) |
           (unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, vj);
  };

  // ---- rows without a valid key take the uniform average of V over the N keys (tri_uniform_row):
  // ---- a pair of such rows skips the main loop; in a mixed pair the main loop's result for the
  // ---- uniform row is replaced at the end ----
  const int64_t kvoff[2] = {((int64_t)i0 * H + h) * nkb * kKVBlock, ((int64_t)i1 * H + h) * nkb * kKVBlock};
  if (uni[0] && uni[1]) {  // block-uniform
    tri_uniform_row<T, 1>(KV + kvoff[0], vblk, nv, N, out, i0, so0, so1, h, D, 32 * qt, lane);
    if (i1v < N) tri_uniform_row<T, 1>(KV + kvoff[1], vblk, nv, N, out, i1, so0, so1, h, D, 32 * qt, lane);
    return;
  }

  const int qtc = qt < nqt ? qt : nqt - 1;
  const T* bq = bias + ((int64_t)h * nqt + qtc) * nkt * 1024 + (32 * hl + col) * 8;

  // ---- KV block copy: wave w moves (row w >> 1, part w & 1 = K or V^T), 4 KB in four 1 KB
  // ---- instructions; lane l of instruction s fills LDS chunk p = 64 s + l of the part with the
  // ---- global chunk that the swizzle places there.
  const int crow = wave >> 1, cpart = wave & 1;
  const char* kvsrc = reinterpret_cast<const char*>(KV + kvoff[crow] + cpart * 2048);
  uint32_t gofs[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int p = 64 * s + lane;
    gofs[s] = 16u * (uint32_t)(cpart == 0 ? ((p & ~3) | ((p & 3) ^ ((p >> 4) & 3))) : ((p & ~7) | ((p & 7) ^ ((p >> 4) & 7))));
  }
  // The copies and the bias loads of the main loop are inline asm, so the compiler neither sees
  // nor waits for them: with copies in flight its own wait counts would not be exact (it falls
  // back to waiting for every load), and every wait of the loop is written out below.  The copy
  // takes a 64-bit per-lane address in VGPRs (no SGPR base), and its `s_nop 4` puts 5 wait states
  // between the write of M0 (the slot address, which the compiler moves there) and the load.
  auto dma = [&](int vj, auto sc) {
    const int kb = visit(vj);
    const char* src = kvsrc + (int64_t)kb * kKVBlock * (int64_t)sizeof(T);
    const uint32_t dst = (uint32_t)reinterpret_cast<uintptr_t>(&slot(sc)[crow][cpart * 4096]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const char* a = src + gofs[s];
      const uint32_t m = dst + 1024u * s;
      asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(a), "{m0}"(m) : "memory");
    }
  };
  // operand reads: K of row r, 32-key tile kt (A operand of S^T, k-steps j = 0, 1); V^T of
  // row r, tile kt (A operand of O^T)
  auto read_k = [&](auto sc, int r, int kt, V8* k) {
    const int key = 32 * kt + col;
    const char* base = &slot(sc)[r][key * 64];
#pragma unroll
    for (int j = 0; j < 2; ++j) k[j] = *reinterpret_cast<const V8*>(base + (((2 * j + hl) ^ ((key >> 2) & 3)) << 4));
  };
  auto read_v = [&](auto sc, int r, int kt, V8* v) {
    const char* base = &slot(sc)[r][4096 + col * 128];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      v[j] = *reinterpret_cast<const V8*>(base + (((4 * kt + 2 * j + hl) ^ ((col >> 1) & 7)) << 4));
  };
  auto load_bias = [&](int vj, int kt, V8* b) {
    const int kb = visit(vj);
    const T* p = bq + (int64_t)(2 * kb + kt) * 1024;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(b[0]) : "v"(p) : "memory");
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(b[1]) : "v"(p + 512) : "memory");
  };
  // after the explicit wait for a bias set: redefine its registers, so that no use of them can
  // be scheduled above the wait
  auto ready = [&](V8 (*b)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      pin(b[t][0]);
      pin(b[t][1]);
    }
  };

  f32x16 o[2], S[2];
  f32x4 ls[2];  // row sums by the matrix cores (slot 0 = the query's sum), as in tri_attn_kernel
  const vec<T, 8> lsel = row_sum_selector<T>(lane);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    o[r] = f32x16{};
    ls[r] = f32x4{};
  }
  V8 P[2][2], vop[2][2];
  V8 bset[2][2][2];  // bias operands of visits vj, vj + 1 (set vj % 2): [tile][half]

  auto scores = [&](int r, const V8* k, const V8* b) {
    f32x16 s = bias_acc<T>(b[0], b[1]);
    s = Mma<T>::m32(k[0], qop[r][0], s);
    return Mma<T>::m32(k[1], qop[r][1], s);
  };

  // One stage: weights of row r's tile (key bits tb) from S[r]; the PV MFMAs of the other row's
  // previous tile (P[1 - r], vop[1 - r]) and the score MFMAs of the next tile (row rn, K operands
  // kn, bias bn, into S[rn]) are interleaved with its exponentials.
  auto stage = [&](int r, unsigned int tb, bool pv, int rn, const V8* kn, const V8* bn) {
    if (pv) {
      o[1 - r] = Mma<T>::m32(vop[1 - r][0], P[1 - r][0], o[1 - r]);
      o[1 - r] = Mma<T>::m32(vop[1 - r][1], P[1 - r][1], o[1 - r]);
      ls[1 - r] = Mma<T>::m16(lsel, P[1 - r][0], ls[1 - r]);
      ls[1 - r] = Mma<T>::m16(lsel, P[1 - r][1], ls[1 - r]);
    }
    f32x16 s = S[r];
    if (tb != 0xffffffffu) {  // partial tile (wave-uniform): masked keys get weight 0
      const unsigned int lb = tb >> (4 * hl);
#pragma unroll
      for (int v = 0; v < 16; ++v) s[v] = ((lb >> (8 * (v / 4) + (v % 4))) & 1u) ? s[v] : -INFINITY;
    }
    S[rn] = scores(rn, kn, bn);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      P[r][0][v] = (T)fast_exp2(s[v]);
      P[r][1][v] = (T)fast_exp2(s[8 + v]);
    }
    pin(P[r][0]);
    pin(P[r][1]);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 2, 0);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 5, 0);
    }
  };

  // ---- prologue.  Every global load of the main loop is issued in one place per block, after
  // ---- the block's barrier: the bias of visit vj + 2 (first needed in the next block's last
  // ---- stage), then the copy of block vj + 3 (needed two blocks later).  Vector-memory loads
  // ---- complete in issue order, so a wait for one load also waits for every load issued before
  // ---- it: the bias load that follows a copy is not needed before the copy itself, so the
  // ---- copies keep their full lead.  The prologue issues the same sequence from visit 0. ----
  vmcnt_wait<0>();  // Q (and the validity pass's mask loads) have landed
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    pin(qop[r][0]);
    pin(qop[r][1]);
  }
  __builtin_amdgcn_sched_barrier(0);
  dma(0, IC<0>{});
  __builtin_amdgcn_sched_barrier(0);  // (each group issues in program order)
  load_bias(0, 0, bset[0][0]);
  load_bias(0, 1, bset[0][1]);
  __builtin_amdgcn_sched_barrier(0);
  dma(1, IC<1>{});
  __builtin_amdgcn_sched_barrier(0);
  load_bias(1, 0, bset[1][0]);
  load_bias(1, 1, bset[1][1]);
  __builtin_amdgcn_sched_barrier(0);
  dma(2, IC<2>{});
  __builtin_amdgcn_sched_barrier(0);
  vmcnt_wait<12>();  // this wave's copy of block 0 and bias set 0 have landed (12 loads behind them)
  ready(bset[0]);
  __syncthreads();
  {
    V8 k[2];
    read_k(IC<0>{}, 0, 0, k);
    S[0] = scores(0, k, bset[0][0]);
  }

  // One 64-key block (visit vj in LDS slot SL = vj % 4 and bias set BS = vj % 2): four stages (kt,
  // r), each computing the scores of the next.  Bias set BS was last read by the third stage; after
  // the barrier it takes visit vj + 2, and slot (vj + 3) % 4, whose block vj - 1 was last read
  // before that barrier, the copy of block vj + 3.  At the barrier this wave's copy of block vj + 1
  // (issued at the barrier two blocks earlier) has exactly 8 loads behind it: the bias of visit
  // vj + 1 and the copy of block vj + 2.
  auto block = [&](int vj, auto slc) {
    constexpr int SL = decltype(slc)::value, BS = SL % 2, BN = (BS + 1) % 2;
    using SN = IC<(SL + 1) % kRing>;
    using SC = IC<(SL + 3) % kRing>;
    const unsigned long long kv0 = bits64(kv0_l, vj), kv1 = bits64(kv1_l, vj);
    V8 k[2];
    // stage (kt 0, row 0): next = (0, row 1)
    read_k(slc, 1, 0, k);
    read_v(slc, 0, 0, vop[0]);
    stage(0, (unsigned int)kv0, vj > 0, 1, k, bset[BS][0]);
    // stage (kt 0, row 1): next = (1, row 0)
    read_k(slc, 0, 1, k);
    read_v(slc, 1, 0, vop[1]);
    stage(1, (unsigned int)kv1, true, 0, k, bset[BS][1]);
    // stage (kt 1, row 0): next = (1, row 1)
    read_k(slc, 1, 1, k);
    read_v(slc, 0, 1, vop[0]);
    stage(0, (unsigned int)(kv0 >> 32), true, 1, k, bset[BS][1]);
    __builtin_amdgcn_sched_barrier(0);
    vmcnt_wait<8>();  // this wave's copy of block vj + 1 has landed (behind it: bias vj + 1, copy vj + 2)
    __syncthreads();
    load_bias(vj + 2, 0, bset[BS][0]);
    load_bias(vj + 2, 1, bset[BS][1]);
    dma(vj + 3, SC{});
    vmcnt_wait<12>();  // bias set of visit vj + 1 has landed (behind it: copy vj + 2, bias vj + 2, copy vj + 3)
    ready(bset[BN]);
    __builtin_amdgcn_sched_barrier(0);
    // stage (kt 1, row 1): next = (visit vj + 1, kt 0, row 0)
    read_k(SN{}, 0, 0, k);
    read_v(slc, 1, 1, vop[1]);
    stage(1, (unsigned int)(kv1 >> 32), true, 0, k, bset[BN][0]);
  };
  for (int vj = 0; vj < nv; vj += 4) {
    block(vj, IC<0>{});
    if (vj + 1 < nv) block(vj + 1, IC<1>{});
    if (vj + 2 < nv) block(vj + 2, IC<2>{});
    if (vj + 3 < nv) block(vj + 3, IC<3>{});
  }
  vmcnt_wait<0>();  // no copy may still be writing the block's LDS when its waves finish
  // ---- epilogue: PV of the last stage (row 1) ----
  o[1] = Mma<T>::m32(vop[1][0], P[1][0], o[1]);
  o[1] = Mma<T>::m32(vop[1][1], P[1][1], o[1]);
  ls[1] = Mma<T>::m16(lsel, P[1][0], ls[1]);
  ls[1] = Mma<T>::m16(lsel, P[1][1], ls[1]);

  // ---- per row: the uniform average (a row without valid keys), an exact-max recomputation
  // ---- (a wave whose shift-free row sums left [2^-60, 2^100] or are not finite), or O / l ----
  const int qo = 32 * qt + col;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (r == 1 && i1v >= N) break;  // block-uniform: the pair's second row is past the grid
    if (uni[r]) {
      tri_uniform_row<T, 1>(KV + kvoff[r], vblk, nv, N, out, irow[r], so0, so1, h, D, 32 * qt, lane);
      continue;
    }
    const float lt = ls[r][0];
    if (__ballot(!(lt >= 0x1p-60f && lt <= 0x1p100f)) != 0) {  // wave-uniform
      tri_exact_tile<T>(KV + kvoff[r], bq, qop[r][0], qop[r][1], vblk, kvalid[r], nv, N, out,
                        irow[r], so0, so1, h, D, qo, lane);
      continue;
    }
    const float inv = 1.0f / lt;
    if (qo < N) {
      T* dst = out + (int64_t)irow[r] * so0 + (int64_t)qo * so1 + (int64_t)h * D + 4 * hl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        V4 w4 = {(T)(o[r][4 * g] * inv), (T)(o[r][4 * g + 1] * inv), (T)(o[r][4 * g + 2] * inv),
                 (T)(o[r][4 * g + 3] * inv)};
        stg<V4>(dst + 8 * g, w4);
      }
    }
  }
}


// ---------------------------------------------------------------------------------------------
// Repack for the shapes the pre-pass does not cover: the any-shape pre-pass's plain Q / K / V
// (N, N, H, D) and fp32 pair bias (H, N, N) rewritten into the attention kernel's layouts with
// D zero-padded to 32 (any D <= 32, any H), so that triangle attention at those shapes (e.g. the
// D = 16, C_in = 64 "Apo" shape) runs on the MFMA attention kernel; the padded dimensions are
// zero in Q, K and V, so they add nothing to the scores and give zero output columns.
// One thread per 16-byte output chunk; reads past N or D give zeros (finite padding, as the
// attention kernel requires).
//   what 0: Qp    chunk (row r = (i H + h) ldn + p, c < 4): d-permuted elements 8c .. 8c + 7
//   what 1: KV    chunk (block (i H + h) nkb + kb, m < 512): m < 256 -> K row m / 4, chunk m % 4;
//                 else V^T row d = (m - 256) / 8, chunk (m - 256) % 8 (keys permuted per 32)
//   what 2: bias  chunk (tile (h nqt + qt) nkt + kt, ch < 128): elements 8 ch .. 8 ch + 7 (keys
//                 permuted per 32)
// ---------------------------------------------------------------------------------------------
__device__ inline int perm32(int x) {  // position x of a permuted group of 32 -> natural index
  const int j = x >> 4, hl = (x >> 3) & 1, e = x & 7;
  return 16 * j + 8 * (e >> 2) + 4 * hl + (e & 3);
}

template <typename T>
__global__ __launch_bounds__(256) void tri_repack_kernel(int what, const T* __restrict__ q, const T* __restrict__ k,
                                                        const T* __restrict__ v, const float* __restrict__ bias,
                                                        T* __restrict__ dst, int64_t nchunks, int N, int ldn, int H,
                                                        int D, float qscale) {
  using V8 = vec<T, 8>;
  const int nkb = ldn / 64, nqt = (N + 31) / 32, nkt = ldn / 32;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < nchunks; idx += (int64_t)gridDim.x * 256) {
    V8 out;
    if (what == 0) {
      const int c = (int)(idx & 3);
      const int64_t r = idx >> 2;
      const int p = (int)(r % ldn);
      const int64_t ih = r / ldn;
      const int h = (int)(ih % H);
      const int64_t i = ih / H;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = perm32(8 * c + e);
        out[e] = (p < N && d < D) ? (T)((float)q[((i * N + p) * H + h) * D + d] * qscale) : (T)0.f;
      }
    } else if (what == 1) {
      const int m = (int)(idx & 511);
      const int64_t blk = idx >> 9;
      const int kb = (int)(blk % nkb);
      const int64_t ih = blk / nkb;
      const int h = (int)(ih % H);
      const int64_t i = ih / H;
      if (m < 256) {
        const int key = 64 * kb + (m >> 2), c = m & 3;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = perm32(8 * c + e);
          out[e] = (key < N && d < D) ? k[((i * N + key) * H + h) * D + d] : (T)0.f;
        }
      } else {
        const int d = (m - 256) >> 3, c = (m - 256) & 7;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int kappa = 8 * c + e;
          const int key = 64 * kb + 32 * (kappa >> 5) + perm32(kappa & 31);
          out[e] = (key < N && d < D) ? v[((i * N + key) * H + h) * D + d] : (T)0.f;
        }
      }
    } else {
      const int ch = (int)(idx & 127);
      const int64_t tile = idx >> 7;
      const int kt = (int)(tile % nkt);
      const int64_t hq = tile / nkt;
      const int qt = (int)(hq % nqt);
      const int h = (int)(hq / nqt);
      const int j = ch >> 6, hl = (ch >> 5) & 1, c = ch & 31;
      const int qq = 32 * qt + c;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kk = 32 * kt + perm32(16 * j + 8 * hl + e);
        out[e] = (qq < N && kk < N) ? (T)(kLog2e * bias[((int64_t)h * N + qq) * N + kk]) : (T)0.f;
      }
    }
    stg<V8>(dst + 8 * idx, out);
  }
}

template <typename T>
static int tri_repack_t(const void* q, const void* k, const void* v, const float* bias, void* Qp, void* KV,
                        void* btiles, int64_t N, int64_t ldn, int64_t H, int64_t D, float qscale, hipStream_t st) {
  const int64_t nkb = ldn / 64, nqt = (N + 31) / 32, nkt = ldn / 32;
  const int64_t n[3] = {N * H * ldn * 4, N * H * nkb * 512, H * nqt * nkt * 128};
  void* dst[3] = {Qp, KV, btiles};
  for (int w = 0; w < 3; ++w) {
    if (n[w] == 0) continue;
    const int64_t want = (n[w] + 255) / 256, cap = 64LL * num_cus();
    const unsigned grid = (unsigned)(want < cap ? want : cap);
    hipLaunchKernelGGL((tri_repack_kernel<T>), dim3(grid), dim3(256), 0, st, w, (const T*)q, (const T*)k,
                       (const T*)v, bias, (T*)dst[w], n[w], (int)N, (int)ldn, (int)H, (int)D, qscale);
    const int rc = launched("tops_tri_repack");
    if (rc != TOPS_OK) return rc;
  }
  return TOPS_OK;
}

template <typename T>
static int tri_prep_t(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln, int apply_ln,
                      const void* wqkv, const void* WZ, const float* BZ, void* Qp, void* KV, void* bias, int64_t N,
                      int64_t ldn, int64_t C, int64_t D, float eps, float qscale, hipStream_t st) {
  const int64_t ntiles = N * (ldn / 64);
  if (ntiles == 0) return TOPS_OK;
  const int64_t grid = ntiles < (int64_t)num_cus() ? ntiles : (int64_t)num_cus();
  auto kern = C == 128 ? (apply_ln ? tri_prep_kernel<T, true, 128> : tri_prep_kernel<T, false, 128>)
                       : (apply_ln ? tri_prep_kernel<T, true, 64> : tri_prep_kernel<T, false, 64>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(512), 0, st, (const T*)x, sx0, sx1, (const T*)w_ln,
                     (const T*)b_ln, (const T*)wqkv, (const T*)WZ, BZ, (T*)Qp, (T*)KV, (T*)bias, (uint32_t)N,
                     (uint32_t)ldn, eps, qscale, kLog2e, (uint32_t)ntiles, FastDiv((uint32_t)(ldn / 64)), (int)D);
  return launched("tops_tri_prep");
}

template <typename T>
static int tri_attention_t(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0,
                           int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H,
                           int64_t dv, hipStream_t st) {
  const int qt = N <= 128 ? 1 : 2;
  const int nw = N >= TRI_NW8_MIN_N ? 8 : 4;  // waves (query tiles of 32 x qt) per block
  const int64_t per_block = nw * 32 * qt;
  const int nqc = (int)((N + per_block - 1) / per_block);
  const int64_t grid = N * H * nqc;
  if (grid == 0) return TOPS_OK;
#define TOPS_TRI(QTV, NWV)                                                                                    \
  hipLaunchKernelGGL((tri_attn_kernel<T, QTV, NWV>), dim3((unsigned)grid), dim3(64 * NWV), 0, st, (const T*)Qp, \
                     (const T*)KV, (const T*)bias, (const int8_t*)mask, sm0, sm1, (T*)out, so0, so1, N, ldn,     \
                     (int)H, nqc, (int)dv)
  if (qt == 1)
    TOPS_TRI(1, 4);
  else if (nw == 4)
    TOPS_TRI(2, 4);
  else
    TOPS_TRI(2, 8);
#undef TOPS_TRI
  return launched("tops_tri_attention");
}

// The two-row kernel (bf16, D = 32): 4 waves per (row pair, 128 queries, head).
static int tri_attention2(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0, int64_t sm1,
                          void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H, hipStream_t st) {
  const int nqc = (int)((N + 127) / 128), nrp = (int)((N + 1) / 2);
  const int64_t grid = H * nrp * nqc;
  if (grid == 0) return TOPS_OK;
  hipLaunchKernelGGL((tri_attn2_kernel<__bf16>), dim3((unsigned)grid), dim3(256), 0, st, (const __bf16*)Qp,
                     (const __bf16*)KV, (const __bf16*)bias, (const int8_t*)mask, sm0, sm1, (__bf16*)out, so0, so1,
                     (int)N, (int)ldn, (int)H, nqc, nrp);
  return launched("tops_tri_attention_two_row");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_tri_prep(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln,
                             int apply_ln, const void* wqkv, const void* WZ, const float* BZ, void* Qp, void* KV,
                             void* bias, int64_t N, int64_t ldn, int64_t C, int64_t H, int64_t D, float eps,
                             float scale, int dtype, void* stream) {
  TOPS_REQUIRE(x && wqkv && WZ && Qp && KV && bias, "tops_tri_prep: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_tri_prep: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE((C == 128 || C == 64) && H == 4 && (D == 32 || D == 16),
               "tops_tri_prep: supports C in {128, 64}, H == 4, D in {32, 16} (got %lld, %lld, %lld)", (long long)C,
               (long long)H, (long long)D);
  TOPS_REQUIRE(N >= 0 && N <= kMaxN, "tops_tri_prep: supports N <= %d (got %lld)", kMaxN, (long long)N);
  TOPS_REQUIRE(ldn == tri_ldn(N), "tops_tri_prep: ldn must be max(64, round_up(N, 64)) = %lld (got %lld)",
               (long long)tri_ldn(N), (long long)ldn);
  TOPS_REQUIRE(sx0 % 8 == 0 && sx1 % 8 == 0 && (uintptr_t)x % 16 == 0,
               "tops_tri_prep: x needs token strides that are multiples of 8 and a 16-byte aligned base");
  hipStream_t st = (hipStream_t)stream;
  const float qscale = scale * kLog2e;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_prep_t<__bf16>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, Qp, KV, bias, N, ldn, C, D, eps, qscale,
                              st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_prep_t<_Float16>(x, sx0, sx1, w_ln, b_ln, apply_ln, wqkv, WZ, BZ, Qp, KV, bias, N, ldn, C, D, eps,
                                qscale, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_prep: unsupported dtype code %d", dtype);
}

extern "C" int tops_tri_attention(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0,
                                  int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H,
                                  int64_t D, int dtype, void* stream) {
  TOPS_REQUIRE(Qp && KV && bias && out, "tops_tri_attention: null pointer argument");
  TOPS_REQUIRE((D == 32 || D == 24 || D == 16 || D == 8) && H >= 1 && H <= 64,
               "tops_tri_attention: supports D in {8, 16, 24, 32} and H <= 64 (got D=%lld H=%lld)", (long long)D,
               (long long)H);
  TOPS_REQUIRE(N >= 0 && N <= kMaxN, "tops_tri_attention: supports N <= %d (got %lld)", kMaxN, (long long)N);
  TOPS_REQUIRE(ldn == tri_ldn(N), "tops_tri_attention: ldn must be max(64, round_up(N, 64)) = %lld (got %lld)",
               (long long)tri_ldn(N), (long long)ldn);
  TOPS_REQUIRE(so0 % 4 == 0 && so1 % 4 == 0, "tops_tri_attention: out strides must be multiples of 4");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_attention_t<__bf16>(Qp, KV, bias, mask, sm0, sm1, out, so0, so1, N, ldn, H, D, st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_attention_t<_Float16>(Qp, KV, bias, mask, sm0, sm1, out, so0, so1, N, ldn, H, D, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_attention: unsupported dtype code %d", dtype);
}

extern "C" int tops_tri_attention_two_row(const void* Qp, const void* KV, const void* bias, const void* mask,
                                          int64_t sm0, int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N,
                                          int64_t ldn, int64_t H, int64_t D, int dtype, void* stream) {
  TOPS_REQUIRE(Qp && KV && bias && out, "tops_tri_attention_two_row: null pointer argument");
  TOPS_REQUIRE(dtype == TOPS_DTYPE_BF16 && D == 32,
               "tops_tri_attention_two_row: bf16 with D = 32 only (got dtype %d, D=%lld)", dtype, (long long)D);
  TOPS_REQUIRE(H >= 1 && H <= 64 && N >= 0 && N <= 4096,
               "tops_tri_attention_two_row: supports H <= 64 and N <= 4096 (got H=%lld N=%lld)", (long long)H,
               (long long)N);
  TOPS_REQUIRE(ldn == tri_ldn(N), "tops_tri_attention_two_row: ldn must be max(64, round_up(N, 64)) = %lld (got %lld)",
               (long long)tri_ldn(N), (long long)ldn);
  TOPS_REQUIRE(so0 % 4 == 0 && so1 % 4 == 0, "tops_tri_attention_two_row: out strides must be multiples of 4");
  return tri_attention2(Qp, KV, bias, mask, sm0, sm1, out, so0, so1, N, ldn, H, (hipStream_t)stream);
}

extern "C" int tops_tri_repack(const void* q, const void* k, const void* v, const float* bias, void* Qp, void* KV,
                               void* btiles, int64_t N, int64_t ldn, int64_t H, int64_t D, float scale, int dtype,
                               void* stream) {
  TOPS_REQUIRE(q && k && v && bias && Qp && KV && btiles, "tops_tri_repack: null pointer argument");
  TOPS_REQUIRE(N >= 0 && N <= kMaxN, "tops_tri_repack: supports N <= %d (got %lld)", kMaxN, (long long)N);
  TOPS_REQUIRE(ldn == tri_ldn(N), "tops_tri_repack: ldn must be max(64, round_up(N, 64)) = %lld (got %lld)",
               (long long)tri_ldn(N), (long long)ldn);
  TOPS_REQUIRE(H >= 1 && H <= 64 && D >= 1 && D <= 32, "tops_tri_repack: supports H <= 64, D <= 32 (got %lld, %lld)",
               (long long)H, (long long)D);
  hipStream_t st = (hipStream_t)stream;
  const float qscale = scale * kLog2e;
  if (dtype == TOPS_DTYPE_BF16) return tri_repack_t<__bf16>(q, k, v, bias, Qp, KV, btiles, N, ldn, H, D, qscale, st);
  if (dtype == TOPS_DTYPE_F16) return tri_repack_t<_Float16>(q, k, v, bias, Qp, KV, btiles, N, ldn, H, D, qscale, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_repack: unsupported dtype code %d", dtype);
}
