// triangle_attention (starting node) on gfx950.
//
//   tri_ln_bias_kernel   one pass over x: x_ln = LN(x) (written once, shared by the attention
//                        and the gate epilogue) and the row-shared pair bias
//                        bias[h,q,k] = x_ln[q,k,:] . WZ[h,:] + BZ[h]   (fp32 dot, io store).
//   tri_attn_kernel      one block per (row i, head h, query chunk): projects K/V of row i
//                        once per 64-key block into LDS, each wave streams its queries over
//                        them with an online softmax.  S^T = K . Q^T is accumulated on top of
//                        the bias tile (MFMA C operand), and the D registers of S^T are the
//                        B operand of O^T = V^T . P^T, so scores never leave registers.
//
// Reference: triangle_attn/module.py:57-125 (forward), triangle_attn/kernel.py:36-98 (bias),
// :110-253 (attention), :230-238 and :369 (additive -1e9 pair mask, -inf outside the row).
#include "capi.hpp"
#include "common.hpp"

namespace tops {

// ---------------------------------------------------------------------------------------------
// LayerNorm + bias.  8 threads per token (16 channels each), 32 tokens per 256-thread block.
// ---------------------------------------------------------------------------------------------
template <typename T, int C, int H>
__global__ __launch_bounds__(256) void tri_ln_bias_kernel(const T* __restrict__ x, int64_t sx0, int64_t sx1,
                                                         const T* __restrict__ w_ln, const T* __restrict__ b_ln,
                                                         int apply_ln, const T* __restrict__ WZ,
                                                         const float* __restrict__ BZ, T* __restrict__ x_ln,
                                                         T* __restrict__ bias, int64_t N, float eps) {
  constexpr int TPT = 8, CPT = C / TPT;  // 16 channels per thread
  using V8 = vec<T, 8>;
  const int tid = threadIdx.x;
  const int part = tid % TPT;
  const int64_t t = (int64_t)blockIdx.x * (256 / TPT) + tid / TPT;
  const int64_t NN = N * N;
  const bool valid = t < NN;
  const int64_t q = valid ? t / N : 0, k = valid ? t % N : 0;

  float v[CPT];
  {
    const T* src = x + q * sx0 + k * sx1 + part * CPT;
#pragma unroll
    for (int e = 0; e < CPT / 8; ++e) {
      V8 a = valid ? ldg<V8>(src + 8 * e) : V8{};
#pragma unroll
      for (int j = 0; j < 8; ++j) v[8 * e + j] = (float)a[j];
    }
  }
  if (apply_ln) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) s += v[j];
    const float mean = group_sum<TPT>(s) * (1.0f / C);
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) sq += (v[j] - mean) * (v[j] - mean);
    const float rstd = rsqrtf(group_sum<TPT>(sq) * (1.0f / C) + eps);
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = part * CPT + j;
      v[j] = (v[j] - mean) * rstd * (float)w_ln[c] + (b_ln ? (float)b_ln[c] : 0.f);
    }
    if (x_ln && valid) {
      T* dst = x_ln + t * C + part * CPT;
#pragma unroll
      for (int e = 0; e < CPT / 8; ++e) {
        V8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (T)v[8 * e + j];
        stg<V8>(dst + 8 * e, o);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) d += v[j] * (float)WZ[h * C + part * CPT + j];
    d = group_sum<TPT>(d);
    if (part == 0 && valid) bias[h * NN + t] = (T)(d + (BZ ? BZ[h] : 0.f));
  }
}

// ---------------------------------------------------------------------------------------------
// Attention core.  C = 128, D = 32, 8 waves, 64-key blocks, QT query tiles (32 queries each)
// per wave.  wqkv is (H, 3, D, C): rows of WQ^T, WK^T, WV^T for each head.
//
// Per 64-key block:
//   projection: wave w computes a 16-key x 32-d slice of K (w < 4) or V (w >= 4) with
//     16x16x32 MFMAs straight from x_ln rows in HBM/L2, storing K as [key][d] and V as
//     V^T [d][key] in LDS (rows padded to keep the operand reads bank-conflict free);
//   attention: per 32-key tile and query tile, S^T = bias + K . Q^T (2 MFMAs), masked and
//     folded into the running max / sum, then O^T += V^T . P^T (2 MFMAs).
// Masked keys get probability exactly 0 (exp(-1e9 - m) underflows to 0 in fp32 whenever the
// row has a valid key).  A row without valid keys reproduces the reference's uniform
// average: every score is -1e9 there, so all N keys get weight 1/N.
// ---------------------------------------------------------------------------------------------
constexpr int kTriKRow = 36;  // K  LDS row: 32 d + 4 pad (elements)
constexpr int kTriVRow = 68;  // V^T LDS row: 64 keys + 4 pad (elements)

template <typename T, int QT>
__global__ __launch_bounds__(512) void tri_attn_kernel(const T* __restrict__ xln, const T* __restrict__ wqkv,
                                                      const T* __restrict__ bias, const int8_t* __restrict__ mask,
                                                      int64_t sm0, int64_t sm1, T* __restrict__ out, int64_t so0,
                                                      int64_t so1, int64_t N, int H, int nqc, float scale) {
  constexpr int C = 128, D = 32;
  using V8 = vec<T, 8>;
  using V4 = vec<T, 4>;

  __shared__ __attribute__((aligned(16))) T Ks[64 * kTriKRow];
  __shared__ __attribute__((aligned(16))) T Vs[D * kTriVRow];
  __shared__ unsigned long long kvalid[64];  // N <= 4096 -> at most 64 key blocks
  __shared__ int row_any;

  // ---- block -> (row i, head h, query chunk); XCD-aware: consecutive rows of one head
  // ---- share an XCD so that head's bias stays in that XCD's L2.
  const int64_t total = N * H * nqc;
  int64_t id = blockIdx.x;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  const int64_t i = id % N;
  const int hq = (int)(id / N);
  const int h = hq % H;
  const int qc = hq / H;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int nkb = (int)((N + 63) / 64);

  // ---- key validity per 64-key block ----
  if (tid == 0) row_any = 0;
  __syncthreads();
  for (int kb = wave; kb < nkb; kb += 8) {
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
  const bool uniform = row_any == 0;  // no valid key in this row: every score is -1e9
  if (uniform) {
    for (int kb = wave; kb < nkb; kb += 8) {
      const int64_t k = (int64_t)kb * 64 + lane;
      const unsigned long long bits = __ballot(k < N);
      if (lane == 0) kvalid[kb] = bits;
    }
    __syncthreads();
  }

  const T* xrow = xln + i * N * C;
  const T* wh = wqkv + (int64_t)h * 3 * D * C;

  // ---- Q^T tiles for this wave's queries: B operand of S^T = K . Q^T ----
  const int64_t qbase = (int64_t)qc * (8 * 32 * QT) + (int64_t)wave * 32 * QT;
  V8 qop[QT][2];
  {
    V8 wq[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) wq[s] = ldg<V8>(wh + (int64_t)col * C + 16 * s + 8 * hl);
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      int64_t q = qbase + 32 * t + col;
      q = q < N ? q : N - 1;
      f32x16 acc = {};
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = Mma<T>::m32(wq[s], ldg<V8>(xrow + q * C + 16 * s + 8 * hl), acc);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qop[t][0][e] = (T)(acc[e] * scale);
        qop[t][1][e] = (T)(acc[8 + e] * scale);
      }
    }
  }

  // ---- projection role: rows of WK^T (waves 0-3) or WV^T (waves 4-7), 16x16x32 layout ----
  const bool is_v = wave >= 4;
  const int kq = wave & 3;  // 16-key quarter of the block
  V8 wr[2][4];
  {
    const T* wsrc = wh + (is_v ? 2 : 1) * D * C;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        wr[dt][s] = ldg<V8>(wsrc + (int64_t)(16 * dt + (lane & 15)) * C + 32 * s + 8 * (lane >> 4));
  }

  f32x16 o[QT];
  float m[QT], l[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    o[t] = f32x16{};
    m[t] = -INFINITY;
    l[t] = 0.f;
  }
  const bool bias_vec = (N % 4) == 0;

  for (int kb = 0; kb < nkb; ++kb) {
    const unsigned long long kbits = kvalid[kb];
    if (kbits == 0) continue;  // block-uniform
    // ---- projection of this block's K / V into LDS ----
    {
      int64_t key = (int64_t)kb * 64 + 16 * kq + (lane & 15);
      key = key < N ? key : N - 1;
      V8 xa[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) xa[s] = ldg<V8>(xrow + key * C + 32 * s + 8 * (lane >> 4));
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        f32x4 acc = {};
        if (!is_v) {
#pragma unroll
          for (int s = 0; s < 4; ++s) acc = Mma<T>::m16(wr[dt][s], xa[s], acc);
          // D = K^T tile: lane -> key (lane & 15), d = 16 dt + 4 (lane >> 4) + v
          V4 kv = {(T)acc[0], (T)acc[1], (T)acc[2], (T)acc[3]};
          *reinterpret_cast<V4*>(&Ks[(16 * kq + (lane & 15)) * kTriKRow + 16 * dt + 4 * (lane >> 4)]) = kv;
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) acc = Mma<T>::m16(xa[s], wr[dt][s], acc);
          // D = V tile: lane -> d = 16 dt + (lane & 15), keys 4 (lane >> 4) + v
          V4 vv = {(T)acc[0], (T)acc[1], (T)acc[2], (T)acc[3]};
          *reinterpret_cast<V4*>(&Vs[(16 * dt + (lane & 15)) * kTriVRow + 16 * kq + 4 * (lane >> 4)]) = vv;
        }
      }
    }
    __syncthreads();

    // ---- attention over the two 32-key tiles ----
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const unsigned int tbits = (unsigned int)(kbits >> (32 * kt));
      if (tbits == 0) continue;
      const bool full = tbits == 0xffffffffu;
      V8 kop[2], vop[2];
      {
        const T* kr = &Ks[(32 * kt + col) * kTriKRow];
        const V4 a0 = *reinterpret_cast<const V4*>(kr + 4 * hl);
        const V4 a1 = *reinterpret_cast<const V4*>(kr + 8 + 4 * hl);
        const V4 a2 = *reinterpret_cast<const V4*>(kr + 16 + 4 * hl);
        const V4 a3 = *reinterpret_cast<const V4*>(kr + 24 + 4 * hl);
        kop[0] = V8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        kop[1] = V8{a2[0], a2[1], a2[2], a2[3], a3[0], a3[1], a3[2], a3[3]};
        const T* vr = &Vs[col * kTriVRow + 32 * kt];
        const V4 b0 = *reinterpret_cast<const V4*>(vr + 4 * hl);
        const V4 b1 = *reinterpret_cast<const V4*>(vr + 8 + 4 * hl);
        const V4 b2 = *reinterpret_cast<const V4*>(vr + 16 + 4 * hl);
        const V4 b3 = *reinterpret_cast<const V4*>(vr + 24 + 4 * hl);
        vop[0] = V8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        vop[1] = V8{b2[0], b2[1], b2[2], b2[3], b3[0], b3[1], b3[2], b3[3]};
      }
      const int64_t k0 = (int64_t)kb * 64 + 32 * kt;
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        int64_t q = qbase + 32 * t + col;
        q = q < N ? q : N - 1;
        f32x16 s;
        if (uniform) {
          s = f32x16{};
        } else {
          const T* brow = bias + ((int64_t)h * N + q) * N + k0;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int kk = 8 * g + 4 * hl;
            if (bias_vec && k0 + kk + 3 < N) {
              const V4 b = ldg<V4>(brow + kk);
#pragma unroll
              for (int e = 0; e < 4; ++e) s[4 * g + e] = (float)b[e];
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) s[4 * g + e] = (k0 + kk + e < N) ? (float)brow[kk + e] : 0.f;
            }
          }
          s = Mma<T>::m32(kop[0], qop[t][0], s);
          s = Mma<T>::m32(kop[1], qop[t][1], s);
        }
        if (!full) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int kk = 8 * (v / 4) + 4 * hl + (v % 4);
            if (!((tbits >> kk) & 1u)) s[v] = -INFINITY;
          }
        }
        float mt = s[0];
#pragma unroll
        for (int v = 1; v < 16; ++v) mt = fmaxf(mt, s[v]);
        mt = halves_max(mt);
        const float mnew = fmaxf(m[t], mt);
        const float muse = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = fast_exp2((m[t] - muse) * kLog2e);
        const float nb = -muse * kLog2e;
        float ps = 0.f;
        V8 pop0, pop1;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = fast_exp2(fmaf(s[v], kLog2e, nb));
          ps += p;
          if (v < 8)
            pop0[v] = (T)p;
          else
            pop1[v - 8] = (T)p;
        }
        l[t] = l[t] * alpha + ps;
        m[t] = mnew;
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] *= alpha;
        o[t] = Mma<T>::m32(vop[0], pop0, o[t]);
        o[t] = Mma<T>::m32(vop[1], pop1, o[t]);
      }
    }
    __syncthreads();
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
static int tri_ln_bias_t(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln, int apply_ln,
                         const void* WZ, const float* BZ, void* x_ln, void* bias, int64_t N, int64_t H, float eps,
                         hipStream_t st) {
  const int64_t NN = N * N;
  const int64_t grid = (NN + 31) / 32;
  if (grid == 0) return TOPS_OK;
#define TOPS_LNB(HH)                                                                                          \
  hipLaunchKernelGGL((tri_ln_bias_kernel<T, 128, HH>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)x, sx0, \
                     sx1, (const T*)w_ln, (const T*)b_ln, apply_ln, (const T*)WZ, BZ, (T*)x_ln, (T*)bias, N, eps)
  switch (H) {
    case 1: TOPS_LNB(1); break;
    case 2: TOPS_LNB(2); break;
    case 4: TOPS_LNB(4); break;
    case 8: TOPS_LNB(8); break;
    default: return fail(TOPS_EUNSUPPORTED, "tops_tri_ln_bias: H must be 1, 2, 4 or 8 (got %lld)", (long long)H);
  }
#undef TOPS_LNB
  return launched("tops_tri_ln_bias");
}

template <typename T>
static int tri_attention_t(const void* xln, const void* wqkv, const void* bias, const void* mask, int64_t sm0,
                           int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t H, float scale,
                           hipStream_t st) {
  const int qt = N <= 256 ? 1 : (N <= 512 ? 2 : 4);
  const int64_t per_block = 8 * 32 * qt;
  const int nqc = (int)((N + per_block - 1) / per_block);
  const int64_t grid = N * H * nqc;
  if (grid == 0) return TOPS_OK;
#define TOPS_TRI(QTV)                                                                                        \
  hipLaunchKernelGGL((tri_attn_kernel<T, QTV>), dim3((unsigned)grid), dim3(512), 0, st, (const T*)xln,        \
                     (const T*)wqkv, (const T*)bias, (const int8_t*)mask, sm0, sm1, (T*)out, so0, so1, N, (int)H, \
                     nqc, scale)
  if (qt == 1)
    TOPS_TRI(1);
  else if (qt == 2)
    TOPS_TRI(2);
  else
    TOPS_TRI(4);
#undef TOPS_TRI
  return launched("tops_tri_attention");
}

}  // namespace tops

using namespace tops;

extern "C" int tops_tri_ln_bias(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln,
                                int apply_ln, const void* WZ, const float* BZ, void* x_ln, void* bias, int64_t N,
                                int64_t C, int64_t H, float eps, int dtype, void* stream) {
  TOPS_REQUIRE(x && WZ && bias, "tops_tri_ln_bias: null pointer argument");
  TOPS_REQUIRE(!apply_ln || w_ln, "tops_tri_ln_bias: w_ln is required when apply_ln != 0");
  TOPS_REQUIRE(apply_ln || !x_ln, "tops_tri_ln_bias: x_ln must be NULL when apply_ln == 0");
  TOPS_REQUIRE(C == 128, "tops_tri_ln_bias: C must be 128 (got %lld)", (long long)C);
  TOPS_REQUIRE(N >= 0, "tops_tri_ln_bias: bad N");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_ln_bias_t<__bf16>(x, sx0, sx1, w_ln, b_ln, apply_ln, WZ, BZ, x_ln, bias, N, H, eps, st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_ln_bias_t<_Float16>(x, sx0, sx1, w_ln, b_ln, apply_ln, WZ, BZ, x_ln, bias, N, H, eps, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_ln_bias: unsupported dtype code %d", dtype);
}

extern "C" int tops_tri_attention(const void* x_ln, const void* wqkv, const void* bias, const void* mask, int64_t sm0,
                                  int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t C, int64_t H,
                                  int64_t D, float scale, int dtype, void* stream) {
  TOPS_REQUIRE(x_ln && wqkv && bias && out, "tops_tri_attention: null pointer argument");
  TOPS_REQUIRE(C == 128 && D == 32, "tops_tri_attention: supports C == 128, D == 32 (got C=%lld D=%lld)",
               (long long)C, (long long)D);
  TOPS_REQUIRE(N >= 0 && N <= 4096, "tops_tri_attention: N must be in [0, 4096] (got %lld)", (long long)N);
  TOPS_REQUIRE(H >= 1 && H <= 64, "tops_tri_attention: bad H %lld", (long long)H);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TOPS_DTYPE_BF16)
    return tri_attention_t<__bf16>(x_ln, wqkv, bias, mask, sm0, sm1, out, so0, so1, N, H, scale, st);
  if (dtype == TOPS_DTYPE_F16)
    return tri_attention_t<_Float16>(x_ln, wqkv, bias, mask, sm0, sm1, out, so0, so1, N, H, scale, st);
  return fail(TOPS_EUNSUPPORTED, "tops_tri_attention: unsupported dtype code %d", dtype);
}
