// attention_pair_bias core on gfx950.
//
// One block per (32-query block, key split).  Z is the dominant HBM stream (M^2 * Cz * 2
// bytes); every block reads its Z[q-block, key-range, :] exactly once for ALL heads:
//   * per (query, 16 keys) the 16 x 128 Z slice is an MFMA A operand loaded straight from HBM;
//     a 16x16x32 MFMA against [Wc_hi; Wc_lo] (the fp32 LN-folded weight split into two
//     io-typed terms, accumulated into the same tile) gives z . Wc_h for the 4 heads, and the
//     LayerNorm statistics are reduced from the same registers (two-pass, fp32);
//   * bias[h,q,k] = rstd * (z . Wc_h - mean * sum(Wc_h)) + Bc_h goes through LDS to the wave
//     of head h, which runs S^T = bias + K . Q^T, the online softmax and O^T += V^T . P^T with
//     K and V projected from X in registers (the D layout of each MFMA is the operand layout of
//     the next, so no LDS traffic for Q/K/V/P).
// Split partials (running max m, sum l, unnormalised O) are merged by apb_combine_kernel.
//
// Reference: attn_pair_bias/kernel.py:24-202 (`_apb_kernel`), :205-257 (`apb_forward`);
// the key mask follows benchmarks/references.py:273-274 (masked keys -> -inf).
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
__global__ __launch_bounds__(256) void apb_attn_kernel(const T* __restrict__ X, const T* __restrict__ wqkv,
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
  const T* wh = wqkv + (int64_t)h * 3 * D * C;

  // ---- Q^T for the block's 32 queries, head h (B operand of S^T = K . Q^T) ----
  const int64_t q0 = (int64_t)qb * 32;
  V8 qop[2];
  {
    int64_t q = q0 + col;
    q = q < M ? q : M - 1;
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < 8; ++s)
      acc = Mma<T>::m32(ldg<V8>(wh + (int64_t)col * C + 16 * s + 8 * hl), ldg<V8>(X + q * C + 16 * s + 8 * hl), acc);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qop[0][e] = (T)(acc[e] * scale);
      qop[1][e] = (T)(acc[8 + e] * scale);
    }
  }
  V8 wk[8], wv[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    wk[s] = ldg<V8>(wh + (int64_t)(D + col) * C + 16 * s + 8 * hl);
    wv[s] = ldg<V8>(wh + (int64_t)(2 * D + col) * C + 16 * s + 8 * hl);
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

  const int64_t kbeg = (int64_t)sp * keys_per_split;
  const int64_t kend = kbeg + keys_per_split < M ? kbeg + keys_per_split : M;
  for (int64_t k0 = kbeg; k0 < kend; k0 += 32) {
    // key validity of this 32-key block (same in every wave)
    unsigned int kbits;
    {
      const int64_t k = k0 + (lane & 31);
      bool ok = k < kend;
      if (ok && mask) ok = mask[k] != 0;
      kbits = (unsigned int)__ballot(ok && lane < 32);
    }
    if (kbits == 0) continue;  // block-uniform

    // ---- pair bias for the 32 x 32 (query, key) tile: wave w -> queries 8w .. 8w+7 ----
#pragma unroll 1
    for (int u = 0; u < 16; ++u) {
      const int lq = 8 * wave + (u >> 1), kh = u & 1;
      int64_t q = q0 + lq;
      q = q < M ? q : M - 1;
      int64_t key = k0 + 16 * kh + l16;
      key = key < M ? key : M - 1;
      const T* zr = Z + q * sz0 + key * sz1 + 8 * g16;
      V8 za[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) za[s] = ldg<V8>(zr + 32 * s);
      float sum = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += (float)za[s][e];
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      const float mean = sum * (1.0f / C);
      float sq = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = (float)za[s][e] - mean;
          sq += d * d;
        }
      sq += __shfl_xor(sq, 16);
      sq += __shfl_xor(sq, 32);
      const float rstd = rsqrtf(sq * (1.0f / C) + eps);
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
    }

    // ---- K^T and V of the 32 keys for head h (registers only) ----
    V8 kop[2], vop[2];
    {
      int64_t key = k0 + col;
      key = key < M ? key : M - 1;
      f32x16 ka = {}, va = {};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const V8 xk = ldg<V8>(X + key * C + 16 * s + 8 * hl);
        ka = Mma<T>::m32(wk[s], xk, ka);
        va = Mma<T>::m32(xk, wv[s], va);
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
  const float* ml = ws + (int64_t)nsplit * M * (H * D);
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ml[(((int64_t)s * M + q) * H + h) * 2]);
  const float mu = mx == -INFINITY ? 0.f : mx;
  float lt = 0.f, ot = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float ms = ml[(((int64_t)s * M + q) * H + h) * 2];
    const float w = fast_exp2((ms - mu) * kLog2e);
    lt += w * ml[(((int64_t)s * M + q) * H + h) * 2 + 1];
    ot += w * ws[((int64_t)s * M + q) * (H * D) + hd];
  }
  Og[q * (H * D) + hd] = (T)(ot / lt);
}

template <typename T>
static int apb_forward_t(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1, const float* Wc,
                         const float* sWc, const float* Bc, const void* mask, void* Og, void* work, int64_t M,
                         float scale, float eps, hipStream_t st) {
  if (M == 0) return TOPS_OK;
  const ApbSplit sp = apb_split(M);
  const int64_t qblocks = (M + 31) / 32;
  const int64_t grid = qblocks * sp.nsplit;
  hipLaunchKernelGGL((apb_attn_kernel<T>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)X, (const T*)wqkv,
                     (const T*)Z, sz0, sz1, Wc, sWc, Bc, (const int8_t*)mask, (T*)Og, (float*)work, M, sp.nsplit,
                     sp.keys_per_split, scale, eps);
  int rc = launched("tops_apb_forward");
  if (rc != TOPS_OK || sp.nsplit == 1) return rc;
  const int64_t n = M * 128;
  hipLaunchKernelGGL((apb_combine_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const float*)work, (T*)Og, M, sp.nsplit);
  return launched("tops_apb_forward(combine)");
}

}  // namespace tops

using namespace tops;

extern "C" int64_t tops_apb_workspace_bytes(int64_t M, int64_t H, int64_t D) {
  if (M <= 0) return 0;
  const ApbSplit sp = apb_split(M);
  if (sp.nsplit == 1) return 0;
  return (int64_t)sp.nsplit * M * H * (D + 2) * 4;
}

extern "C" int tops_apb_forward(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                                const float* Wc, const float* sWc, const float* Bc, const void* mask, void* Og,
                                void* work, int64_t M, int64_t C, int64_t Cz, int64_t H, int64_t D, float scale,
                                float eps, int dtype, void* stream) {
  TOPS_REQUIRE(X && wqkv && Z && Wc && sWc && Bc && Og, "tops_apb_forward: null pointer argument");
  TOPS_REQUIRE(C == 128 && Cz == 128 && H == 4 && D == 32,
               "tops_apb_forward: supports C == Cz == 128, H == 4, D == 32 (got C=%lld Cz=%lld H=%lld D=%lld)",
               (long long)C, (long long)Cz, (long long)H, (long long)D);
  TOPS_REQUIRE(M >= 0, "tops_apb_forward: bad M");
  TOPS_REQUIRE(work || tops_apb_workspace_bytes(M, H, D) == 0, "tops_apb_forward: workspace required");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return apb_forward_t<__bf16>(X, wqkv, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, work, M, scale, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return apb_forward_t<_Float16>(X, wqkv, Z, sz0, sz1, Wc, sWc, Bc, mask, Og, work, M, scale, eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_apb_forward: unsupported dtype code %d", dtype);
}
