// attention_pair_bias core on gfx950.
//
// Two kernels (three when the key range is split):
//   apb_qkv_kernel: Q = X.Wq^T (+ b_q, scaled), K = X.Wk^T, V = X.Wv^T for all M tokens once,
//     (M, H*D) rows each, 32 tokens per block and one wave per head (MFMA, fp32 accumulation);
//     the qk-norm variant (benchmarks/references.py:230-277) also takes the Q bias and a
//     LayerNorm over the full H*D channel of Q and K (statistics exchanged between the head
//     waves through LDS) here.
//   apb_attn_kernel: one block per (32-query block, key split).  Z is the dominant HBM stream
//     (M^2 * Cz * 2 bytes); every block reads its Z[q-block, key-range, :] exactly once for ALL
//     heads:
//   * per (query, 16 keys) the 16 x 128 Z slice is an MFMA A operand loaded straight from HBM;
//     a 16x16x32 MFMA against [Wc_hi; Wc_lo] (the fp32 LN-folded weight split into two
//     io-typed terms, accumulated into the same tile) gives z . Wc_h for the 4 heads, and the
//     LayerNorm statistics are reduced from the same registers (sum and sum of squares, fp32);
//   * bias[h,q,k] = rstd * (z . Wc_h - mean * sum(Wc_h)) + Bc_h goes through LDS to the wave
//     of head h, which runs S^T = bias + K . Q^T, the online softmax and O^T += V^T . P^T.  The
//     wave brings head h's Q, K and V into MFMA operand layout with two MFMA k-steps against a
//     block-identity operand built in registers (an exact transpose through the matrix core),
//     so there is no LDS traffic for Q/K/V/P.
// Split partials (running max m, sum l, unnormalised O) are merged by apb_combine_kernel into Og,
// or, on the fused path (tops_apb_forward_gated), by apb_merge_gate_kernel, which goes on to the
// gate and the output projection of attn_pair_bias/module.py:69-70 in the same launch.
//
// Reference: attn_pair_bias/kernel.py:24-202 (`_apb_kernel`), :205-257 (`apb_forward`);
// the key mask follows benchmarks/references.py:273-274 (masked keys -> -inf).
#include <mutex>
#include <type_traits>

#include "capi.hpp"
#include "common.hpp"

namespace tops {

constexpr int kApbBRow = 36;  // LDS bias row: 32 keys + 4 pad (fp32)

struct ApbSplit {
  int nsplit, keys_per_split;
};

static ApbSplit apb_split(int64_t M) {
  const int64_t qblocks = (M + 31) / 32, kblocks = (M + 31) / 32;
  int64_t ns = (2LL * num_cus() + qblocks - 1) / (qblocks > 0 ? qblocks : 1);
  if (ns < 1) ns = 1;
  if (ns > kblocks) ns = kblocks > 0 ? kblocks : 1;
  if (ns > 64) ns = 64;
  const int64_t kb_per = (kblocks + ns - 1) / ns;
  ns = (kblocks + kb_per - 1) / kb_per;
  if (ns < 1) ns = 1;
  return ApbSplit{(int)ns, (int)(kb_per * 32)};
}

template <typename T>
__global__ __launch_bounds__(256, 2) void apb_attn_kernel(const T* __restrict__ Qm, const T* __restrict__ Km,
                                                      const T* __restrict__ Vm,
                                                      const T* __restrict__ Z, int64_t sz0, int64_t sz1,
                                                      const float* __restrict__ Wc, const float* __restrict__ sWc,
                                                      const float* __restrict__ Bc, const int8_t* __restrict__ mask,
                                                      T* __restrict__ Og, float* __restrict__ ws, int64_t M,
                                                      int nsplit, int keys_per_split, float scale, float eps) {
  constexpr int C = 128, D = 32, H = 4;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;
  __shared__ __attribute__((aligned(16))) float bias_s[H][32 * kApbBRow];

  const int qb = blockIdx.x / nsplit, sp = blockIdx.x % nsplit;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int l16 = lane & 15, g16 = lane >> 4;
  const int h = wave;  // attention role: head of this wave
  // head h's 32 channels are k-steps 2h, 2h + 1 of the (M, 128) rows; `eye` is the matching block of
  // the identity in operand layout (lane: row col, channels 16 s + 8 hl + e), so A . eye^T and
  // eye . B^T reproduce the rows exactly in the MFMA output layout
  const int s0 = 2 * h;
  const int64_t q0 = (int64_t)qb * 32;
  const int64_t kbeg = (int64_t)sp * keys_per_split;
  const int64_t kend = kbeg + keys_per_split < M ? kbeg + keys_per_split : M;
  // Z slice of pair-bias step u of the 32-key block at kb0: query 8 w + u / 2, keys 16 (u % 2) .. +15
  auto zload = [&](int64_t kb0, int u, V8* za) {
    const int lq = 8 * wave + (u >> 1), kh = u & 1;
    int64_t q = q0 + lq;
    q = q < M ? q : M - 1;
    int64_t key = kb0 + 16 * kh + l16;
    key = key < M ? key : M - 1;
    const T* zr = Z + q * sz0 + key * sz1 + 8 * g16;
#pragma unroll
    for (int s = 0; s < 4; ++s) za[s] = ldg<V8>(zr + 32 * s);
  };
  // the first block's first Z slice is loaded before everything else (the kernel runs as about
  // one round of blocks, so each block's first HBM round trip is on the critical path)
  V8 za[4], zb[4];
  zload(kbeg, 0, za);
  V8 eye[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) eye[s][e] = (T)(16 * s + 8 * hl + e == col ? 1.0f : 0.0f);

  // ---- Q^T for the block's 32 queries, head h (B operand of S^T = K . Q^T) ----
  V8 qop[2];
  {
    int64_t q = q0 + col;
    q = q < M ? q : M - 1;
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 2; ++s) acc = Mma<T>::m32(eye[s], ldg<V8>(Qm + q * C + 16 * (s0 + s) + 8 * hl), acc);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qop[0][e] = (T)(acc[e] * scale);
      qop[1][e] = (T)(acc[8 + e] * scale);
    }
  }
  // ---- [Wc_hi; Wc_lo] as the B operand of the bias MFMA (16x16x32: col = head) ----
  V8 whi[4], wlo[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float w = l16 < H ? Wc[l16 * C + 32 * s + 8 * g16 + e] : 0.f;
      const T hi = (T)w;
      whi[s][e] = hi;
      wlo[s][e] = (T)(w - (float)hi);
    }
  const float my_swc = l16 < H ? sWc[l16] : 0.f, my_bc = l16 < H ? Bc[l16] : 0.f;

  f32x16 o = {};
  float m = -INFINITY, l = 0.f;

  // key validity of a 32-key block (same in every wave); the next block's mask bytes are loaded
  // at the start of this one, so no block waits for its own
  auto mload = [&](int64_t kb0) {
    const int64_t k = kb0 + (lane & 31);
    return k < kend && lane < 32 ? (mask ? (int)mask[k] : 1) : 0;
  };
  int mcur = mload(kbeg);
  for (int64_t k0 = kbeg; k0 < kend; k0 += 32) {
    const unsigned int kbits = (unsigned int)__ballot(mcur != 0);
    mcur = mload(k0 + 32);
    if (kbits == 0) continue;  // block-uniform

    // ---- pair bias for the 32 x 32 (query, key) tile: wave w -> queries 8w .. 8w+7 ----
    // step u covers query 8w + u / 2 and keys 16 (u % 2) .. +15; the Z slice of step u + 1 is
    // loaded while step u is reduced (two register sets, so a load is always in flight)
    auto zbias = [&](int u, const V8* za) {
      const int lq = 8 * wave + (u >> 1), kh = u & 1;
      // LayerNorm statistics in one pass, sum and sum of squares with clamped variance, as the
      // reference accumulates them (attn_pair_bias/kernel.py:168-173): packed dot products take two
      // channels per instruction with fp32 products and sums
      const vec<T, 2> one = {(T)1.0f, (T)1.0f};
      float sum = 0.f, sq = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const vec<T, 2> pr = {za[s][e], za[s][e + 1]};
          sum = Mma<T>::dot2(pr, one, sum);
          sq = Mma<T>::dot2(pr, pr, sq);
        }
      sum += __shfl_xor(sum, 16);
      sq += __shfl_xor(sq, 16);
      sum += __shfl_xor(sum, 32);
      sq += __shfl_xor(sq, 32);
      const float mean = sum * (1.0f / C);
      const float var = fmaxf(sq * (1.0f / C) - mean * mean, 0.f);
      const float rstd = rsqrtf(var + eps);
      f32x4 acc = {};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = Mma<T>::m16(za[s], whi[s], acc);
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = Mma<T>::m16(za[s], wlo[s], acc);
      // acc slot v: key 4*g16 + v of the 16, head l16; its stats live in lane (4*g16 + v)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float mu = __shfl(mean, 4 * g16 + v);
        const float rs = __shfl(rstd, 4 * g16 + v);
        if (l16 < H) bias_s[l16][lq * kApbBRow + 16 * kh + 4 * g16 + v] = rs * (acc[v] - mu * my_swc) + my_bc;
      }
    };
    {
      if (k0 != kbeg) zload(k0, 0, za);  // (the first block's was loaded at the start)
#pragma unroll 1
      for (int u = 0; u < 16; u += 2) {
        zload(k0, u + 1, zb);
        zbias(u, za);
        if (u + 2 < 16) zload(k0, u + 2, za);
        zbias(u + 1, zb);
      }
    }

    // ---- K^T and V of the 32 keys for head h (registers only) ----
    V8 kop[2], vop[2];
    {
      int64_t key = k0 + col;
      key = key < M ? key : M - 1;
      f32x16 ka = {}, va = {};
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int64_t off = key * C + 16 * (s0 + s) + 8 * hl;
        ka = Mma<T>::m32(eye[s], ldg<V8>(Km + off), ka);
        va = Mma<T>::m32(ldg<V8>(Vm + off), eye[s], va);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kop[0][e] = (T)ka[e];
        kop[1][e] = (T)ka[8 + e];
        vop[0][e] = (T)va[e];
        vop[1][e] = (T)va[8 + e];
      }
    }
    __syncthreads();

    // ---- scores, online softmax, P.V for head h ----
    f32x16 s;
    {
      const float* br = &bias_s[h][col * kApbBRow];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(br + 8 * g + 4 * hl);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * g + e] = b[e];
      }
    }
    s = Mma<T>::m32(kop[0], qop[0], s);
    s = Mma<T>::m32(kop[1], qop[1], s);
    if (kbits != 0xffffffffu) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kk = 8 * (v / 4) + 4 * hl + (v % 4);
        if (!((kbits >> kk) & 1u)) s[v] = -INFINITY;
      }
    }
    float mt = s[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mt = fmaxf(mt, s[v]);
    mt = halves_max(mt);
    const float mnew = fmaxf(m, mt);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = fast_exp2((m - muse) * kLog2e);
    const float nb = -muse * kLog2e;
    float ps = 0.f;
    V8 p0, p1;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = fast_exp2(fmaf(s[v], kLog2e, nb));
      ps += p;
      if (v < 8)
        p0[v] = (T)p;
      else
        p1[v - 8] = (T)p;
    }
    l = l * alpha + ps;
    m = mnew;
#pragma unroll
    for (int v = 0; v < 16; ++v) o[v] *= alpha;
    o = Mma<T>::m32(vop[0], p0, o);
    o = Mma<T>::m32(vop[1], p1, o);
    __syncthreads();
  }

  l = halves_sum(l);
  const int64_t q = q0 + col;
  if (q >= M) return;
  if (nsplit == 1) {
    const float inv = 1.0f / l;
    T* dst = Og + q * (H * D) + h * D + 4 * hl;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      V4 r = {(T)(o[4 * g] * inv), (T)(o[4 * g + 1] * inv), (T)(o[4 * g + 2] * inv), (T)(o[4 * g + 3] * inv)};
      stg<V4>(dst + 8 * g, r);
    }
  } else {
    float* wo = ws + ((int64_t)sp * M + q) * (H * D) + h * D + 4 * hl;
#pragma unroll
    for (int g = 0; g < 4; ++g) stg<f32x4>(wo + 8 * g, f32x4{o[4 * g], o[4 * g + 1], o[4 * g + 2], o[4 * g + 3]});
    if (hl == 0) {
      float* wml = ws + (int64_t)nsplit * M * (H * D) + (((int64_t)sp * M + q) * H + h) * 2;
      wml[0] = m;
      wml[1] = l;
    }
  }
}

// Merge split partials: one thread per (query, head, d).
template <typename T>
__global__ __launch_bounds__(256) void apb_combine_kernel(const float* __restrict__ ws, T* __restrict__ Og, int64_t M,
                                                         int nsplit) {
  constexpr int H = 4, D = 32;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * H * D) return;
  const int64_t q = idx / (H * D);
  const int hd = (int)(idx % (H * D));
  const int h = hd / D;
  const float* ml = ws + (int64_t)nsplit * M * (H * D) + (q * H + h) * 2;  // split s: + s * M * H * 2
  const float* op = ws + q * (H * D) + hd;                                  // split s: + s * M * H * D
  const int64_t sml = M * H * 2, so = M * (H * D);
  // the loops are unrolled so that several splits' loads are in flight together (a thread's loads
  // are otherwise one dependent round trip per split); same arithmetic and order as a plain loop
  float mx = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ml[s * sml]);
  const float mu = mx == -INFINITY ? 0.f : mx;
  float lt = 0.f, ot = 0.f;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) {
    const float w = fast_exp2((ml[s * sml] - mu) * kLog2e);
    lt += w * ml[s * sml + 1];
    ot += w * op[s * so];
  }
  Og[q * (H * D) + hd] = (T)(ot / lt);
}

// Split merge fused with the gate and output projection of attention_pair_bias
// (attn_pair_bias/module.py:69-70: out = ((Og * sigmoid(X . Wg^T + bg)) -> io) . Wo^T + bo), C = 128:
// one block per 16 queries, 4 waves (the kernel is bound by the latency of its loads, so more,
// smaller blocks finish sooner).  Thread t merges the split partials of query t / 16, channels
// 32 g + 8 (t % 4) + e (e < 8) of head g = (t % 16) / 4, in apb_combine_kernel's arithmetic and
// order, so the merged Og has the same bits, and stages it in LDS beside the block's 16 rows of X;
// then wave w computes features [32 w, +32) of both GEMMs exactly as gate_out_kernel does (weight
// rows in registers, permuted so each lane holds 16 consecutive features of one query; the 32
// MFMA columns hold the 16 queries twice; the gated values overwrite Og in LDS; the output goes
// through a query-major LDS tile to whole-row stores).
// RES: out = res + result, the single-representation residual of a Pairformer block, rounded once.
constexpr int kApbMergeTok = 16;  // queries per block of apb_merge_gate_kernel

template <typename T, bool RES>
__global__ __launch_bounds__(256) void apb_merge_gate_kernel(const float* __restrict__ ws, const T* __restrict__ X,
                                                            const T* __restrict__ Wg, const T* __restrict__ bg,
                                                            const T* __restrict__ Wo, const T* __restrict__ bo,
                                                            const T* __restrict__ res, T* __restrict__ out,
                                                            int64_t M, int nsplit) {
  constexpr int C = 128, H = 4, TOK = kApbMergeTok, ROW = C * 2, KS = C / 16;
  using V8 = vec<T, 8>;
  __shared__ __attribute__((aligned(16))) char og_s[TOK * ROW];  // merged Og, then the gated values
  __shared__ __attribute__((aligned(16))) char x_s[TOK * ROW];   // gate input X
  __shared__ __attribute__((aligned(16))) T o_s[TOK * C];         // output tile, query-major

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int64_t q0 = (int64_t)blockIdx.x * TOK;
  auto swz = [](int t, int chunk) { return (chunk ^ row_key<C>(t)) << 4; };

  // X rows of the block's queries (rows past M repeat row M - 1; their results are not stored)
  {
    const int t = tid >> 4, c = tid & 15;
    const int64_t q = q0 + t < M ? q0 + t : M - 1;
    *reinterpret_cast<V8*>(&x_s[t * ROW + swz(t, c)]) = ldg<V8>(X + q * C + 8 * c);
  }
  // weight rows as MFMA A operands: row col of wave w is feature 32 w + prow
  const int prow = 16 * ((col >> 2) & 1) + 4 * (col >> 3) + (col & 3);
  // G's rows times -log2(e) and its bias -log2(e) bg as one more MFMA k-step, and bo as W_o's, as
  // in the triangle gate kernel (the accumulator is the gate's exp2 argument; same bits as that
  // kernel)
  V8 wg[KS], wo[KS], gb_a, one_b, ob_a;
  {
    const int64_t frow = (int64_t)(32 * wave + prow) * C;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const V8 g = ldg<V8>(Wg + frow + 16 * s + 8 * hl);
#pragma unroll
      for (int e = 0; e < 8; ++e) wg[s][e] = (T)((float)g[e] * -kLog2e);
      wo[s] = ldg<V8>(Wo + frow + 16 * s + 8 * hl);
    }
    // (clamped: exp2 saturates long before, and the 16-bit parts of a larger value could overflow)
    const float cb = fminf(fmaxf(bg ? -kLog2e * (float)bg[32 * wave + prow] : 0.f, -3e4f), 3e4f);
    const T bhi = (T)cb, blo = (T)(cb - (float)bhi);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gb_a[e] = hl == 0 && e == 0 ? bhi : (hl == 0 && e == 1 ? blo : (T)0.f);
      one_b[e] = (T)((hl == 0 && e < 2) ? 1.f : 0.f);
      ob_a[e] = hl == 0 && e == 0 && bo ? bo[32 * wave + prow] : (T)0.f;  // bo (16-bit) as W_o's bias k-step
    }
  }
  // ---- merge the split partials ----
  // thread t: query t / 16, head g = (t % 16) / 4, channels 32 g + 8 (t % 4) + e: each thread reads
  // its head's (m, l) pair and 32 contiguous bytes of O per split
  {
    const int t = tid >> 4, j = tid & 15, g = j >> 2;
    const int64_t q = q0 + t < M ? q0 + t : M - 1;
    const float* ml = ws + (int64_t)nsplit * M * C + (q * H + g) * 2;  // split s: + s * M * H * 2
    const float* op = ws + q * C + 32 * g + 8 * (j & 3);                // split s: + s * M * C
    const int64_t sml = M * H * 2, so = M * C;
    // batches of 16 splits with every load of a batch issued before its first use; per element the
    // sums run in split order with apb_combine_kernel's arithmetic, so Og gets the same bits
    constexpr int SB = 16;
    using F2 = vec<float, 2>;
    float mx = -INFINITY;
    F2 mb[SB];
    f32x4 ob[SB][2];
    auto batch = [&](int s0, bool with_o) {
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int s = s0 + i < nsplit ? s0 + i : s0;  // past the batch: split s0 again (unused)
        mb[i] = ldg<F2>(ml + s * sml);
        if (with_o) {
          ob[i][0] = ldg<f32x4>(op + s * so);
          ob[i][1] = ldg<f32x4>(op + s * so + 4);
        }
      }
    };
    // up to SB splits (every M from 2 * SB * 32 CUs' worth of query blocks on): one batch of loads
    // serves the maximum and the sums; more splits take a first pass for the maximum
    const bool one = nsplit <= SB;
    if (one) batch(0, true);
    for (int s0 = 0; s0 < nsplit; s0 += SB) {
      if (!one) batch(s0, false);
#pragma unroll
      for (int i = 0; i < SB; ++i)
        if (s0 + i < nsplit) mx = fmaxf(mx, mb[i][0]);
    }
    const float mu = mx == -INFINITY ? 0.f : mx;
    float lt = 0.f, ot[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ot[e] = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += SB) {
      if (!one) batch(s0, true);
#pragma unroll
      for (int i = 0; i < SB; ++i)
        if (s0 + i < nsplit) {
          const float w = fast_exp2((mb[i][0] - mu) * kLog2e);
          lt += w * mb[i][1];
#pragma unroll
          for (int e = 0; e < 8; ++e) ot[e] += w * ob[i][e >> 2][e & 3];
        }
    }
    V8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (T)(ot[e] / lt);
    *reinterpret_cast<V8*>(&og_s[t * ROW + swz(t, 4 * g + (j & 3))]) = r;
  }
  __syncthreads();  // X and Og staged

  // MFMA column col holds query col % TOK (the block's queries twice; both copies write the same
  // values to the same LDS locations)
  const int tok = col % TOK, f0 = 32 * wave + 16 * hl;
  {  // GEMM 1, sigmoid gate, Og * gate -> in place over the Og tile
    const char* grow = &x_s[tok * ROW];
    char* orow = &og_s[tok * ROW];
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
  }
  __syncthreads();  // gated tile complete
  {  // GEMM 2 on the gated tile -> query-major output tile
    const char* trow = &og_s[tok * ROW];
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
      *reinterpret_cast<V8*>(&o_s[tok * C + ((c ^ row_key<C>(tok)) << 3)]) = r;
    }
  }
  __syncthreads();  // output tile complete
  {
    const int t = tid >> 4, c = tid & 15;
    const int64_t q = q0 + t;
    if (q < M) {
      V8 v = *reinterpret_cast<const V8*>(&o_s[t * C + ((c ^ row_key<C>(t)) << 3)]);
      if constexpr (RES) {
        const V8 rr = ldg<V8>(res + q * C + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (T)((float)rr[e] + (float)v[e]);
      }
      stg<V8>(out + q * C + 8 * c, v);
    }
  }
}

// Q / K / V pre-pass at the tuned shape (C = H*D = 128, H = 4, D = 32): 32 tokens per block,
// wave h computes head h's 32 channels (8 MFMA k-steps each; lane col holds 16 of the 32 channels
// of token q0 + col, the other 16 in lane col + 32).  Without QKN each block computes one of q, k,
// v (blockIdx.x % 3) for its 32 tokens: three times the blocks, each with a third of the weight
// loads and MFMA chain, so the latency-bound pass finishes sooner.  With QKN a block computes all
// three, and the per-token LayerNorm over all 128 channels of q and k takes its sums from the four
// head waves through LDS (two passes: mean, then centred squares).  q is scaled by qscale last.
template <typename T, bool QKN>
__global__ __launch_bounds__(256) void apb_qkv_kernel(const T* __restrict__ X, const T* __restrict__ wqkv,
                                                     const T* __restrict__ bq, const T* __restrict__ gq,
                                                     const T* __restrict__ bqn, const T* __restrict__ gk,
                                                     const T* __restrict__ bkn, T* __restrict__ qo,
                                                     T* __restrict__ ko, T* __restrict__ vo, int64_t M, float qscale,
                                                     float eps) {
  constexpr int C = 128, D = 32, H = 4, HD = H * D;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;
  __shared__ float red[2][4][32];  // [q / k][head][token]: per-head partial sums
  const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int64_t q0 = (int64_t)(QKN ? blockIdx.x : blockIdx.x / 3) * 32;
  int64_t tok = q0 + col;
  tok = tok < M ? tok : M - 1;
  V8 xs[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) xs[s] = ldg<V8>(X + tok * C + 16 * s + 8 * hl);
  const T* wh = wqkv + (int64_t)h * 3 * D * C;
  // slot v of acc[t]: channel h*D + dch(v) of token q0 + col
  auto dch = [&](int v) { return 8 * (v >> 2) + 4 * hl + (v & 3); };
  if constexpr (!QKN) {  // one of q, k, v: t = blockIdx.x % 3
    const int t = (int)(blockIdx.x % 3);
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = Mma<T>::m32(ldg<V8>(wh + (int64_t)(t * D + col) * C + 16 * s + 8 * hl), xs[s], acc);
    if (t == 0 && bq) {
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] += (float)bq[h * D + dch(v)];
    }
    if (q0 + col >= M) return;
    T* dst = (t == 0 ? qo : t == 1 ? ko : vo) + (q0 + col) * HD + h * D;
    const float f = t == 0 ? qscale : 1.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      V4 r = {(T)(acc[4 * g] * f), (T)(acc[4 * g + 1] * f), (T)(acc[4 * g + 2] * f), (T)(acc[4 * g + 3] * f)};
      stg<V4>(dst + 8 * g + 4 * hl, r);
    }
    return;
  }
  f32x16 acc[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    acc[t] = f32x16{};
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[t] = Mma<T>::m32(ldg<V8>(wh + (int64_t)(t * D + col) * C + 16 * s + 8 * hl), xs[s], acc[t]);
  }
  if (bq) {
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[0][v] += (float)bq[h * D + dch(v)];
  }
  if constexpr (QKN) {
    float mean[2], rstd[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float s1 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) s1 += acc[t][v];
      s1 += __shfl_xor(s1, 32);
      if (hl == 0) red[t][h][col] = s1;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t) mean[t] = (red[t][0][col] + red[t][1][col] + red[t][2][col] + red[t][3][col]) * (1.0f / HD);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float s2 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float d = acc[t][v] - mean[t];
        s2 += d * d;
      }
      s2 += __shfl_xor(s2, 32);
      if (hl == 0) red[t][h][col] = s2;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t)
      rstd[t] = rsqrtf((red[t][0][col] + red[t][1][col] + red[t][2][col] + red[t][3][col]) * (1.0f / HD) + eps);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const T* g = t == 0 ? gq : gk;
      const T* b = t == 0 ? bqn : bkn;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int c = h * D + dch(v);
        float y = (acc[t][v] - mean[t]) * rstd[t];
        if (g) y *= (float)g[c];
        if (b) y += (float)b[c];
        acc[t][v] = y;
      }
    }
  }
  if (q0 + col >= M) return;
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    T* dst = (t == 0 ? qo : t == 1 ? ko : vo) + (q0 + col) * HD + h * D;
    const float f = t == 0 ? qscale : 1.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      V4 r = {(T)(acc[t][4 * g] * f), (T)(acc[t][4 * g + 1] * f), (T)(acc[t][4 * g + 2] * f),
              (T)(acc[t][4 * g + 3] * f)};
      stg<V4>(dst + 8 * g + 4 * hl, r);
    }
  }
}

// Bytes of the Q / K / V region at the head of the apb workspace (16-bit I/O, 256-byte aligned).
static int64_t apb_qkv_bytes(int64_t M) { return ((3 * M * 128 * 2) + 255) / 256 * 256; }

template <typename T>
static int apb_qkv_t(const void* X, const void* wqkv, const void* bq, int qkn, const void* gq, const void* bqn,
                     const void* gk, const void* bkn, void* q, void* k, void* v, int64_t M, float qscale, float eps,
                     hipStream_t st) {
  const int64_t blocks = (M + 31) / 32;
  if (blocks == 0) return TOPS_OK;
  if (qkn)
    hipLaunchKernelGGL((apb_qkv_kernel<T, true>), dim3((unsigned)blocks), dim3(256), 0, st, (const T*)X,
                       (const T*)wqkv, (const T*)bq, (const T*)gq, (const T*)bqn, (const T*)gk, (const T*)bkn, (T*)q,
                       (T*)k, (T*)v, M, qscale, eps);
  else
    hipLaunchKernelGGL((apb_qkv_kernel<T, false>), dim3((unsigned)(3 * blocks)), dim3(256), 0, st, (const T*)X,
                       (const T*)wqkv, (const T*)bq, (const T*)gq, (const T*)bqn, (const T*)gk, (const T*)bkn, (T*)q,
                       (T*)k, (T*)v, M, qscale, eps);
  return launched("apb_qkv_kernel");
}

// The attention kernel alone: Og when the keys are not split, else the split partials in `part`.
template <typename T>
static int apb_attention_core_t(const void* Q, const void* K, const void* V, const void* Z, int64_t sz0, int64_t sz1,
                                const float* Wc, const float* sWc, const float* Bc, const void* mask, void* Og,
                                void* part, int64_t M, float scale, float eps, hipStream_t st) {
  if (M == 0) return TOPS_OK;
  const ApbSplit sp = apb_split(M);
  const int64_t qblocks = (M + 31) / 32;
  const int64_t grid = qblocks * sp.nsplit;
  hipLaunchKernelGGL((apb_attn_kernel<T>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)Q, (const T*)K,
                     (const T*)V, (const T*)Z, sz0, sz1, Wc, sWc, Bc, (const int8_t*)mask, (T*)Og, (float*)part, M,
                     sp.nsplit, sp.keys_per_split, scale, eps);
  return launched("apb_attn_kernel");
}

template <typename T>
static int apb_attention_t(const void* Q, const void* K, const void* V, const void* Z, int64_t sz0, int64_t sz1,
                           const float* Wc, const float* sWc, const float* Bc, const void* mask, void* Og, void* part,
                           int64_t M, float scale, float eps, hipStream_t st) {
  if (M == 0) return TOPS_OK;
  const ApbSplit sp = apb_split(M);
  int rc = apb_attention_core_t<T>(Q, K, V, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, part, M, scale, eps, st);
  if (rc != TOPS_OK || sp.nsplit == 1) return rc;
  const int64_t n = M * 128;
  hipLaunchKernelGGL((apb_combine_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const float*)part, (T*)Og, M, sp.nsplit);
  return launched("apb_combine_kernel");
}

// ---------------------------------------------------------------------------------------------
// qk-norm pre-pass (benchmarks/references.py:258-264), any C, H, D: per token m
//   q = X[m] . Wq^T + b_q,  k = X[m] . Wk^T,  v = X[m] . Wv^T          (fp32 accumulation)
//   with qkn: q <- LN(q) * g_q + b_q', k <- LN(k) * g_k + b_k' over the full H*D channel
// written as (M, H*D) rows in the I/O type.  kQknTok tokens per block: the weight rows are read
// once per block, the token rows are LDS broadcasts.
// ---------------------------------------------------------------------------------------------
constexpr int kQknTok = 8;

template <typename T>
__global__ __launch_bounds__(256) void apb_qkn_prep_kernel(const T* __restrict__ X, const T* __restrict__ wqkv,
                                                          const T* __restrict__ bq, int qkn, const T* __restrict__ gq,
                                                          const T* __restrict__ bqn, const T* __restrict__ gk,
                                                          const T* __restrict__ bkn,
                                                          T* __restrict__ qo, T* __restrict__ ko, T* __restrict__ vo,
                                                          int64_t M, int C, int H, int D, float qscale, float eps) {
  extern __shared__ float sm[];
  const int HD = H * D, F = 3 * HD;
  float* xs = sm;                    // [kQknTok][C]
  float* raw = xs + kQknTok * C;     // [kQknTok][3][HD]: q, k, v
  float* stat = raw + kQknTok * F;   // [kQknTok][2][2]: (mean, rstd) of q and k
  const int tid = threadIdx.x;
  const int64_t m0 = (int64_t)blockIdx.x * kQknTok;
  for (int e = tid; e < kQknTok * C; e += 256) {
    const int64_t m = m0 + e / C;
    xs[e] = m < M ? (float)X[m * C + e % C] : 0.f;
  }
  __syncthreads();
  for (int f = tid; f < F; f += 256) {  // f: row of the (H, 3, D, C) weight
    const int h = f / (3 * D), which = (f / D) % 3, d = f % D;
    const T* w = wqkv + (int64_t)f * C;
    float acc[kQknTok];
#pragma unroll
    for (int t = 0; t < kQknTok; ++t) acc[t] = 0.f;
    for (int c = 0; c < C; ++c) {
      const float wc = (float)w[c];
#pragma unroll
      for (int t = 0; t < kQknTok; ++t) acc[t] = fmaf(xs[t * C + c], wc, acc[t]);
    }
    const int ch = h * D + d;
    const float add = (which == 0 && bq) ? (float)bq[ch] : 0.f;
#pragma unroll
    for (int t = 0; t < kQknTok; ++t) raw[(t * 3 + which) * HD + ch] = acc[t] + add;
  }
  __syncthreads();
  if (qkn) {
    // one wave per (token, q / k) row: two-pass mean and variance over H*D
    const int lane = tid & 63, wave = tid >> 6;
    for (int r = wave; r < 2 * kQknTok; r += 4) {
      const float* row = raw + ((r >> 1) * 3 + (r & 1)) * HD;
      float sum = 0.f;
      for (int c = lane; c < HD; c += 64) sum += row[c];
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
      const float mean = sum / (float)HD;
      float sq = 0.f;
      for (int c = lane; c < HD; c += 64) {
        const float dv = row[c] - mean;
        sq += dv * dv;
      }
      for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o);
      if (lane == 0) {
        stat[r * 2] = mean;
        stat[r * 2 + 1] = rsqrtf(sq / (float)HD + eps);
      }
    }
    __syncthreads();
  }
  for (int e = tid; e < kQknTok * F; e += 256) {
    const int t = e / F, which = (e / HD) % 3, ch = e % HD;
    const int64_t m = m0 + t;
    if (m >= M) continue;
    float val = raw[e];
    if (qkn && which < 2) {
      const int r = t * 2 + which;
      val = (val - stat[r * 2]) * stat[r * 2 + 1];
      const T* g = which == 0 ? gq : gk;
      const T* b = which == 0 ? bqn : bkn;
      if (g) val *= (float)g[ch];
      if (b) val += (float)b[ch];
    }
    T* dst = which == 0 ? qo : which == 1 ? ko : vo;
    dst[m * HD + ch] = (T)(which == 0 ? val * qscale : val);
  }
}

template <typename T>
static int apb_qkn_prep_t(const void* X, const void* wqkv, const void* bq, int qkn, const void* gq, const void* bqn,
                          const void* gk, const void* bkn, void* q, void* k, void* v, int64_t M, int C, int H, int D,
                          float qscale, float eps, hipStream_t st) {
  if constexpr (!std::is_same_v<T, float>) {
    if (C == 128 && H == 4 && D == 32) return apb_qkv_t<T>(X, wqkv, bq, qkn, gq, bqn, gk, bkn, q, k, v, M, qscale, eps, st);
  }
  const int64_t blocks = (M + kQknTok - 1) / kQknTok;
  if (blocks == 0) return TOPS_OK;
  const size_t lds = ((size_t)kQknTok * C + (size_t)kQknTok * 3 * H * D + 4 * kQknTok) * sizeof(float);
  hipLaunchKernelGGL((apb_qkn_prep_kernel<T>), dim3((unsigned)blocks), dim3(256), lds, st, (const T*)X,
                     (const T*)wqkv, (const T*)bq, qkn, (const T*)gq, (const T*)bqn, (const T*)gk, (const T*)bkn,
                     (T*)q, (T*)k, (T*)v, M, C, H, D, qscale, eps);
  return launched("tops_apb_qkn_prep");
}

}  // namespace tops

using namespace tops;

extern "C" int64_t tops_apb_workspace_bytes(int64_t M, int64_t H, int64_t D) {
  if (M <= 0) return 0;
  const ApbSplit sp = apb_split(M);
  const int64_t part = sp.nsplit == 1 ? 0 : (int64_t)sp.nsplit * M * H * (D + 2) * 4;
  return apb_qkv_bytes(M) + part;
}

extern "C" int64_t tops_apb_gated_workspace_bytes(int64_t M, int64_t H, int64_t D) {
  if (M <= 0) return 0;
  const ApbSplit sp = apb_split(M);
  // without a key split the attention writes Og (M x H*D io values) after Q / K / V instead
  return sp.nsplit == 1 ? apb_qkv_bytes(M) + (M * H * D * 2 + 255) / 256 * 256 : tops_apb_workspace_bytes(M, H, D);
}

template <typename T>
static int apb_merge_gate_t(const float* part, const void* X, const void* Wg, const void* bg, const void* Wo,
                            const void* bo, const void* res, void* out, int64_t M, int nsplit, hipStream_t st) {
  const int64_t blocks = (M + kApbMergeTok - 1) / kApbMergeTok;
  if (res)
    hipLaunchKernelGGL((apb_merge_gate_kernel<T, true>), dim3((unsigned)blocks), dim3(256), 0, st, part, (const T*)X,
                       (const T*)Wg, (const T*)bg, (const T*)Wo, (const T*)bo, (const T*)res, (T*)out, M, nsplit);
  else
    hipLaunchKernelGGL((apb_merge_gate_kernel<T, false>), dim3((unsigned)blocks), dim3(256), 0, st, part, (const T*)X,
                       (const T*)Wg, (const T*)bg, (const T*)Wo, (const T*)bo, (const T*)res, (T*)out, M, nsplit);
  return launched("apb_merge_gate_kernel");
}

extern "C" int tops_apb_forward_gated(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                                      const float* Wc, const float* sWc, const float* Bc, const void* mask,
                                      const void* Wg, const void* bg, const void* Wo, const void* bo, const void* res,
                                      void* out, void* work, int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D,
                                      int64_t Cout, float scale, float eps, int dtype, void* stream) {
  TOPS_REQUIRE(X && wqkv && Z && Wc && sWc && Bc && Wg && Wo && out, "tops_apb_forward_gated: null pointer argument");
  TOPS_REQUIRE(C == 128 && Cz == 128 && H == 4 && D == 32 && Cout == 128,
               "tops_apb_forward_gated: supports C == Cz == C_out == 128, H == 4, D == 32 (got C=%lld Cz=%lld H=%lld "
               "D=%lld C_out=%lld)", (long long)C, (long long)Cz, (long long)H, (long long)D, (long long)Cout);
  TOPS_REQUIRE(M >= 0 && M < (1LL << 31), "tops_apb_forward_gated: bad M");
  TOPS_REQUIRE(work || M == 0, "tops_apb_forward_gated: workspace of tops_apb_gated_workspace_bytes(M, H, D) bytes required");
  TOPS_REQUIRE(sz0 % 8 == 0 && sz1 % 8 == 0 && (uintptr_t)Z % 16 == 0 && (uintptr_t)X % 16 == 0 &&
                   (uintptr_t)work % 16 == 0 && (uintptr_t)out % 16 == 0 && (uintptr_t)res % 16 == 0,
               "tops_apb_forward_gated: Z needs token strides that are multiples of 8, and Z, X, res, out and the "
               "workspace 16-byte aligned base pointers");
  TOPS_REQUIRE(dtype == TOPS_DTYPE_BF16 || dtype == TOPS_DTYPE_F16,
               "tops_apb_forward_gated: unsupported dtype code %d", dtype);
  if (M == 0) return TOPS_OK;
  hipStream_t st = (hipStream_t)stream;
  const ApbSplit sp = apb_split(M);
  char* w = (char*)work;
  char *q = w, *k = w + M * 128 * 2, *v = w + 2 * M * 128 * 2, *part = w + apb_qkv_bytes(M);
  int rc;
  if (sp.nsplit == 1) {  // no split partials: Og in the workspace, then the gate kernel
    rc = tops_apb_forward(X, wqkv, Z, sz0, sz1, Wc, sWc, Bc, mask, part, work, M, C, Cz, H, D, scale, eps, dtype,
                          stream);
    if (rc != TOPS_OK) return rc;
    if (res)
      return tops_gate_out_residual(part, 128, 128, X, 128, 128, nullptr, nullptr, 1e-5f, 0, Wg, bg, Wo, bo, res, 128,
                                    128, out, 128, 128, M, 1, 128, dtype, stream);
    return tops_gate_out(part, 128, 128, X, 128, 128, nullptr, nullptr, 1e-5f, 0, Wg, bg, Wo, bo, out, M, 1, 128,
                         dtype, stream);
  }
  if (dtype == TOPS_DTYPE_BF16) {
    rc = apb_qkv_t<__bf16>(X, wqkv, nullptr, 0, nullptr, nullptr, nullptr, nullptr, q, k, v, M, scale, eps, st);
    if (rc == TOPS_OK)  // Og unused with a split: the partials go to `part`
      rc = apb_attention_core_t<__bf16>(q, k, v, Z, sz0, sz1, Wc, sWc, Bc, mask, nullptr, part, M, 1.0f, eps, st);
    return rc != TOPS_OK ? rc : apb_merge_gate_t<__bf16>((const float*)part, X, Wg, bg, Wo, bo, res, out, M, sp.nsplit, st);
  }
  rc = apb_qkv_t<_Float16>(X, wqkv, nullptr, 0, nullptr, nullptr, nullptr, nullptr, q, k, v, M, scale, eps, st);
  if (rc == TOPS_OK)
    rc = apb_attention_core_t<_Float16>(q, k, v, Z, sz0, sz1, Wc, sWc, Bc, mask, nullptr, part, M, 1.0f, eps, st);
  return rc != TOPS_OK ? rc : apb_merge_gate_t<_Float16>((const float*)part, X, Wg, bg, Wo, bo, res, out, M, sp.nsplit, st);
}

extern "C" int tops_apb_merge_gate(const float* part, const void* X, const void* Wg, const void* bg, const void* Wo,
                                   const void* bo, const void* res, void* out, int64_t M, int64_t H, int64_t D,
                                   int dtype, void* stream) {
  TOPS_REQUIRE(part && X && Wg && Wo && out, "tops_apb_merge_gate: null pointer argument");
  TOPS_REQUIRE(H == 4 && D == 32, "tops_apb_merge_gate: supports H == 4, D == 32 (got H=%lld D=%lld)", (long long)H,
               (long long)D);
  TOPS_REQUIRE(M >= 0 && M < (1LL << 31), "tops_apb_merge_gate: bad M");
  TOPS_REQUIRE(M == 0 || apb_split(M).nsplit > 1, "tops_apb_merge_gate: M = %lld leaves the keys unsplit (no partials)",
               (long long)M);
  TOPS_REQUIRE((uintptr_t)part % 16 == 0 && (uintptr_t)X % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                   (uintptr_t)res % 16 == 0,
               "tops_apb_merge_gate: part, X, res and out must be 16-byte aligned");
  if (M == 0) return TOPS_OK;
  hipStream_t st = (hipStream_t)stream;
  const int ns = apb_split(M).nsplit;
  if (dtype == TOPS_DTYPE_BF16) return apb_merge_gate_t<__bf16>(part, X, Wg, bg, Wo, bo, res, out, M, ns, st);
  if (dtype == TOPS_DTYPE_F16) return apb_merge_gate_t<_Float16>(part, X, Wg, bg, Wo, bo, res, out, M, ns, st);
  return fail(TOPS_EUNSUPPORTED, "tops_apb_merge_gate: unsupported dtype code %d", dtype);
}

// The workspace of tops_apb_forward_noalloc: a library-owned array in device memory (one copy per
// GPU the library runs on, held until the process ends).  Host code never uses the array's name
// as an address: its device address comes from hipGetSymbolAddress, once per device.
constexpr int64_t kApbScratchBytes = 16LL << 20;
static __device__ __align__(256) char scratch[kApbScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};
}  // namespace

static int apb_forward_impl(const char* who, const void* X, const void* wqkv, const void* Z, int64_t sz0,
                            int64_t sz1, const float* Wc, const float* sWc, const float* Bc, const void* mask,
                            void* Og, void* work, int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D, float scale,
                            float eps, int dtype, void* stream);

extern "C" int tops_apb_forward_noalloc(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                                        const float* Wc, const float* sWc, const float* Bc, const void* mask,
                                        void* Og, int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D, float scale,
                                        float eps, int dtype, void* stream) {
  TOPS_REQUIRE(X && wqkv && Z && Wc && sWc && Bc && Og, "tops_apb_forward_noalloc: null pointer argument");
  TOPS_REQUIRE(C == 128 && Cz == 128 && H == 4 && D == 32,
               "tops_apb_forward_noalloc: supports C == Cz == 128, H == 4, D == 32 (got C=%lld Cz=%lld H=%lld D=%lld)",
               (long long)C, (long long)Cz, (long long)H, (long long)D);
  TOPS_REQUIRE(M >= 0, "tops_apb_forward_noalloc: bad M");
  const int64_t need = tops_apb_workspace_bytes(M, H, D);
  TOPS_REQUIRE(need <= kApbScratchBytes,
               "tops_apb_forward_noalloc: M = %lld needs %lld workspace bytes, more than the library's %lld-byte "
               "static workspace; use tops_apb_forward with a caller-allocated workspace",
               (long long)M, (long long)need, (long long)kApbScratchBytes);
  if (M == 0) return TOPS_OK;
  int dev = 0;
  TOPS_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64,
               "tops_apb_forward_noalloc: no current HIP device");
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(TOPS_ELAUNCH, "tops_apb_forward_noalloc: hipGetSymbolAddress of the workspace failed: %s",
                    hipGetErrorString(e));
      g_scratch_ptr[dev] = p;
    }
    ws = g_scratch_ptr[dev];
  }
  return apb_forward_impl("tops_apb_forward_noalloc", X, wqkv, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, ws, M, C, Cz, H,
                          D, scale, eps, dtype, stream);
}

extern "C" int tops_apb_forward(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                                const float* Wc, const float* sWc, const float* Bc, const void* mask, void* Og,
                                void* work, int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D, float scale,
                                float eps, int dtype, void* stream) {
  return apb_forward_impl("tops_apb_forward", X, wqkv, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, work, M, C, Cz, H, D,
                          scale, eps, dtype, stream);
}

static int apb_forward_impl(const char* who, const void* X, const void* wqkv, const void* Z, int64_t sz0,
                            int64_t sz1, const float* Wc, const float* sWc, const float* Bc, const void* mask,
                            void* Og, void* work, int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D, float scale,
                            float eps, int dtype, void* stream) {
  TOPS_REQUIRE(X && wqkv && Z && Wc && sWc && Bc, "%s: null pointer argument", who);
  TOPS_REQUIRE(Og || M == 0 || apb_split(M).nsplit > 1,
               "%s: Og may be NULL only when the keys are split (the partials stay in work)", who);
  TOPS_REQUIRE(C == 128 && Cz == 128 && H == 4 && D == 32,
               "%s: supports C == Cz == 128, H == 4, D == 32 (got C=%lld Cz=%lld H=%lld D=%lld)", who, (long long)C,
               (long long)Cz, (long long)H, (long long)D);
  TOPS_REQUIRE(M >= 0, "%s: bad M", who);
  TOPS_REQUIRE(work || M == 0, "%s: workspace of tops_apb_workspace_bytes(M, H, D) bytes required", who);
  TOPS_REQUIRE(sz0 % 8 == 0 && sz1 % 8 == 0 && (uintptr_t)Z % 16 == 0 && (uintptr_t)X % 16 == 0 &&
                   (uintptr_t)work % 16 == 0,
               "%s: Z needs token strides that are multiples of 8, and Z, X and the workspace 16-byte aligned base "
               "pointers", who);
  if (M == 0) return TOPS_OK;
  hipStream_t st = (hipStream_t)stream;
  char* w = (char*)work;
  char *q = w, *k = w + M * 128 * 2, *v = w + 2 * M * 128 * 2, *part = w + apb_qkv_bytes(M);
  int rc;
  // Og == NULL: the attention's split partials stay in `part` (tops_apb_merge_gate reads them)
  if (dtype == TOPS_DTYPE_BF16) {
    rc = apb_qkv_t<__bf16>(X, wqkv, nullptr, 0, nullptr, nullptr, nullptr, nullptr, q, k, v, M, scale, eps, st);
    if (rc != TOPS_OK) return rc;
    return Og ? apb_attention_t<__bf16>(q, k, v, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, part, M, 1.0f, eps, st)
              : apb_attention_core_t<__bf16>(q, k, v, Z, sz0, sz1, Wc, sWc, Bc, mask, nullptr, part, M, 1.0f, eps, st);
  }
  if (dtype == TOPS_DTYPE_F16) {
    rc = apb_qkv_t<_Float16>(X, wqkv, nullptr, 0, nullptr, nullptr, nullptr, nullptr, q, k, v, M, scale, eps, st);
    if (rc != TOPS_OK) return rc;
    return Og ? apb_attention_t<_Float16>(q, k, v, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, part, M, 1.0f, eps, st)
              : apb_attention_core_t<_Float16>(q, k, v, Z, sz0, sz1, Wc, sWc, Bc, mask, nullptr, part, M, 1.0f, eps,
                                               st);
  }
  return fail(TOPS_EUNSUPPORTED, "%s: unsupported dtype code %d", who, dtype);
}

extern "C" int tops_apb_forward_qkv(const void* Q, const void* K, const void* V, const void* Z, int64_t sz0,
                                    int64_t sz1, const float* Wc, const float* sWc, const float* Bc, const void* mask,
                                    void* Og, void* work, int64_t M, int64_t HD, int64_t Cz, int64_t H, int64_t D,
                                    float scale, float eps, int dtype, void* stream) {
  TOPS_REQUIRE(Q && K && V && Z && Wc && sWc && Bc, "tops_apb_forward_qkv: null pointer argument");
  TOPS_REQUIRE(Og || M == 0 || apb_split(M).nsplit > 1,
               "tops_apb_forward_qkv: Og may be NULL only when the keys are split (the partials stay in work)");
  TOPS_REQUIRE(HD == 128 && Cz == 128 && H == 4 && D == 32,
               "tops_apb_forward_qkv: supports H*D == Cz == 128, H == 4, D == 32 (got H*D=%lld Cz=%lld H=%lld D=%lld)",
               (long long)HD, (long long)Cz, (long long)H, (long long)D);
  TOPS_REQUIRE(M >= 0, "tops_apb_forward_qkv: bad M");
  TOPS_REQUIRE(work || M == 0, "tops_apb_forward_qkv: workspace of tops_apb_workspace_bytes(M, H, D) bytes required");
  TOPS_REQUIRE(sz0 % 8 == 0 && sz1 % 8 == 0 && (uintptr_t)Z % 16 == 0 && (uintptr_t)Q % 16 == 0 &&
                   (uintptr_t)K % 16 == 0 && (uintptr_t)V % 16 == 0 && (uintptr_t)work % 16 == 0,
               "tops_apb_forward_qkv: Z needs token strides that are multiples of 8, and Z, Q, K, V and the "
               "workspace 16-byte aligned base pointers");
  if (M == 0) return TOPS_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return Og ? apb_attention_t<__bf16>(Q, K, V, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, work, M, scale, eps, st)
              : apb_attention_core_t<__bf16>(Q, K, V, Z, sz0, sz1, Wc, sWc, Bc, mask, nullptr, work, M, scale, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return Og ? apb_attention_t<_Float16>(Q, K, V, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, work, M, scale, eps, st)
              : apb_attention_core_t<_Float16>(Q, K, V, Z, sz0, sz1, Wc, sWc, Bc, mask, nullptr, work, M, scale, eps,
                                               st);
  return fail(TOPS_EUNSUPPORTED, "tops_apb_forward_qkv: unsupported dtype code %d", dtype);
}

extern "C" int tops_apb_qkn_prep(const void* X, const void* wqkv, const void* bq, int qkn, const void* gq,
                                 const void* bqn, const void* gk, const void* bkn, void* q, void* k, void* v,
                                 int64_t M, int64_t C, int64_t H, int64_t D, float qscale, float eps, int dtype,
                                 void* stream) {
  TOPS_REQUIRE(X && wqkv && q && k && v, "tops_apb_qkn_prep: null pointer argument");
  // generic shapes: LDS of kQknTok rows of C + 3 H D floats (plus the statistics) within 64 KiB
  TOPS_REQUIRE(M >= 0 && M <= (1LL << 31) && C >= 1 && H >= 1 && D >= 1 && C + 3 * H * D <= 2040,
               "tops_apb_qkn_prep: supports C + 3 * H * D <= 2040 (got M=%lld C=%lld H=%lld D=%lld)", (long long)M,
               (long long)C, (long long)H, (long long)D);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return apb_qkn_prep_t<__bf16>(X, wqkv, bq, qkn, gq, bqn, gk, bkn, q, k, v, M, (int)C, (int)H, (int)D, qscale, eps,
                                  st);
  if (dtype == TOPS_DTYPE_F16)
    return apb_qkn_prep_t<_Float16>(X, wqkv, bq, qkn, gq, bqn, gk, bkn, q, k, v, M, (int)C, (int)H, (int)D, qscale,
                                    eps, st);
  if (dtype == TOPS_DTYPE_F32)
    return apb_qkn_prep_t<float>(X, wqkv, bq, qkn, gq, bqn, gk, bkn, q, k, v, M, (int)C, (int)H, (int)D, qscale, eps,
                                 st);
  return fail(TOPS_EUNSUPPORTED, "tops_apb_qkn_prep: unsupported dtype code %d", dtype);
}
