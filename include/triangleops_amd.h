/*
 * triangleops_amd — C ABI of the MI355X (gfx950) kernels behind the triangle_ops Python API.
 *
 * Plain C: raw device pointers, element counts/strides (in elements, not bytes), scalars and
 * an opaque HIP stream handle (`hipStream_t` passed as `void*`; NULL = default stream).
 * Every function enqueues work on `stream` and returns immediately; none allocates, frees or
 * synchronizes.  Return value: TOPS_OK (0) or a TOPS_E* code; the message for the calling
 * thread is then available from tops_last_error().
 *
 * Each entry point names the reference function it replaces (paths relative to the
 * youngchan2/TriangleOps repository root).  Dtype codes select the I/O type of the io-typed
 * pointers ("io" below); the LayerNorm-fold vectors are always fp32.
 */
#ifndef TRIANGLEOPS_AMD_H
#define TRIANGLEOPS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TOPS_DTYPE_F16 = 1, TOPS_DTYPE_BF16 = 2, TOPS_DTYPE_F32 = 3 };
enum { TOPS_OK = 0, TOPS_EINVAL = 1, TOPS_EUNSUPPORTED = 2, TOPS_ELAUNCH = 3 };

/* Message describing the last error returned on the calling thread ("" if none). */
const char* tops_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int tops_abi_version(void);

/*
 * triangle_multiplicative_update, input phase.
 * Replaces `input_phase` + its Triton kernel (triangle_mul/kernel.py:235-279, :54-162).
 *   x      io   (B, L, L, C) contiguous
 *   mask   int8 (B, L, L) contiguous (bool storage is accepted: 0/1), or NULL; multiplies the output
 *   Wp, Wg io   (C_out, C) LN-folded weights (out, in);  sWp, sWg, Bp, Bg fp32 (C_out,)
 *   ab     io   out[f * B*L*ld + (b*L + r)*ld + c] for f < C_out, r < L, c < ld (ld >= L, ld % 64 == 0)
 *               = sigmoid(G) * P * mask of token (b, i, j) with (i, j) = (r, c), or (c, r) when
 *               transpose != 0; positions c >= L are written as 0.
 * C == 128, C_out in {128, 256} with bf16 / fp16 I/O runs the tuned kernel; any other C <= 1024,
 * C_out <= 4096, or fp32 I/O runs the any-shape kernel (every value fp32 with fp32 I/O).
 */
int tops_tmu_input_phase(const void* x, const void* mask, const void* Wp, const void* Wg, const float* sWp,
                         const float* sWg, const float* Bp, const float* Bg, void* ab, int64_t B, int64_t L,
                         int64_t C, int64_t C_out, int64_t ld, int transpose, float eps, int dtype, void* stream);

/*
 * triangle_multiplicative_update, triangle einsum (replaces the torch.einsum calls at
 * triangle_mul/module.py:80-84).  For every channel-batch slab s < nslab:
 *   y[s*L*ldy + i*ldy + j] = sum_{k < L} a[s*L*ld + i*ld + k] * b[s*L*ld + j*ld + k]
 * with a = ab, b = ab + nslab*L*ld, for i, j < L.  ld and ldy must be multiples of 64 and
 * the columns k in [L, ld) must hold zeros (tops_tmu_input_phase writes them; the product
 * reads k < round_up(L, 64) only, so ld may exceed that as a row padding); columns [L, ldy) of
 * y receive unspecified finite values.  Outgoing feeds the natural token grid,
 * incoming the transposed one (transpose=1 above).  fp32 I/O runs an fp32 VALU product.
 */
int tops_tmu_einsum(const void* ab, void* y, int64_t nslab, int64_t L, int64_t ld, int64_t ldy, int dtype,
                    void* stream);

/*
 * triangle_multiplicative_update, output phase.
 * Replaces `output_phase` + its Triton kernel (triangle_mul/kernel.py:282-326).
 *   y      io   channel-major: y[c * B*L*ldy + (b*L + i)*ldy + j], c < C (ldy >= L, ldy % 64 == 0)
 *   x      io   (B, L, L, C) contiguous
 *   Wp, Wg io   (C_out, C);  sWp, sWg, Bp, Bg fp32 (C_out,)
 *   out    io   (B, L, L, C_out) contiguous = p_out(LN_out(y)) * sigmoid(g_out(LN_in(x)))
 * C == C_out == 128 with bf16 / fp16 I/O runs the tuned kernel; other C <= 512 or fp32 I/O the
 * any-shape kernel.
 */
int tops_tmu_output_phase(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                          const float* sWg, const float* Bp, const float* Bg, void* out, int64_t B, int64_t L,
                          int64_t C, int64_t C_out, int64_t ldy, float eps, int dtype, void* stream);

/*
 * triangle_attention pre-pass: LayerNorm, row-shared pair bias and the Q/K/V projections of all
 * heads in one pass over x.  Replaces F.layer_norm (triangle_attn/module.py:77-83),
 * `bias_proj_kernel` (triangle_attn/kernel.py:36-98) and the Q/K/V projections inside
 * `triangle_attn_kernel` (triangle_attn/kernel.py:181-219).
 *   x      io   element (i, k, c) at x[i*sx0 + k*sx1 + c], c < C (channel stride 1); read as
 *               already normalized when apply_ln == 0 (w_ln, b_ln ignored)
 *   w_ln, b_ln  io (C,) LayerNorm affine (b_ln may be NULL)
 *   wqkv   io   (H, 3, D, C): per head the rows of WQ^T, WK^T, WV^T
 *   WZ     io   (H, C);  BZ fp32 (H,) or NULL
 *   ldn         max(64, N rounded up to a multiple of 64); any other value is rejected (TOPS_EINVAL)
 *   Qp     io   (N, H, ldn, 32): scale * log2(e) * Q, d permuted within each 32 as
 *               [0-3, 8-11, 4-7, 12-15, 16-19, 24-27, 20-23, 28-31]; zero for d >= D
 *   KV     io   (N, H, ldn/64, 4096): per 64-key block K (64 keys x 32, d permuted) then
 *               V^T (32 x 64 keys, keys permuted the same way within each 32); zero for d >= D
 *   bias   io   (H, ceil(N/32), ldn/32, 1024): log2(e) * (LN(x)[q,k,:] . WZ[h,:] + BZ[h]) per
 *               32 x 32 (query, key) tile; (q, k) = (32 qt + c, 32 kt + 16 j + 8 u + 4 hl + e)
 *               (u < 2, e < 4) at element (64 j + 32 hl + c) * 8 + 4 u + e of tile (qt, kt),
 *               i.e. the keys permuted within each 32 as Q's d are; zeros for k >= N
 * C in {128, 64}, H == 4, D in {32, 16} (the default shape and the C_in = 64, D = 16 "Apo" shape
 * of tests/test_triangle_attn.py:137-192, which the reference runs on its tensor-core kernel:
 * triangle_attn/kernel.py:211-213), N <= 16384 (tops_tri_generic_prep serves other shapes).
 */
int tops_tri_prep(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln, int apply_ln,
                  const void* wqkv, const void* WZ, const float* BZ, void* Qp, void* KV, void* bias, int64_t N,
                  int64_t ldn, int64_t C, int64_t H, int64_t D, float eps, float scale, int dtype, void* stream);

/*
 * triangle_attention core (starting node) over the pre-pass outputs.  Replaces the attention
 * of `triangle_attn_kernel` (triangle_attn/kernel.py:197-253, launched at :335-373).
 *   mask   int8 (N, N) with strides (sm0, sm1), nonzero = valid key, or NULL
 *   out    io   O[i, q, h*D + d] at out[i*so0 + q*so1 + h*D + d], d < D (so0, so1 multiples of 4)
 * out[i,q,h] = softmax_k(scale * Q.K + bias[h,q,k] - 1e9 * (mask[i,k] == 0)) V; a row with no
 * valid key is the uniform average of V over all N keys (what the -1e9 add gives).  Qp and KV
 * always hold 32-wide heads (tops_tri_prep / tops_tri_repack layouts); D in {8, 16, 24, 32} is
 * the head width written (Q, K, V zero for d >= D), H <= 64, N <= 16384, ldn as in
 * tops_tri_prep (any other value is rejected).
 */
int tops_tri_attention(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0, int64_t sm1,
                       void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H, int64_t D, int dtype,
                       void* stream);

/*
 * The same attention with two rows per wave (bf16, D = 32 only; other arguments as
 * tops_tri_attention): each wave takes one 32-query tile of rows i and i + 1, so one bias operand
 * load serves both rows, and K / V^T are copied into LDS three 64-key blocks ahead.  Replaces the
 * same reference code as tops_tri_attention (triangle_attn/kernel.py:197-253); its results agree
 * with tops_tri_attention's to bf16 rounding (the weights of the two kernels round at the same
 * points).
 */
int tops_tri_attention_two_row(const void* Qp, const void* KV, const void* bias, const void* mask, int64_t sm0,
                               int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t ldn, int64_t H,
                               int64_t D, int dtype, void* stream);

/*
 * Repack for triangle attention at shapes the pre-pass does not cover (any H <= 64, D <= 32; e.g.
 * the D = 16, C_in = 64 "Apo" shape of tests/test_triangle_attn.py:137-192, which the reference runs
 * on its tensor-core kernel: triangle_attn/kernel.py:211-213, :282): the any-shape pre-pass's
 *   q, k, v io (N, N, H, D) contiguous and bias fp32 (H, N, N) (tops_tri_generic_prep)
 * rewritten into tops_tri_attention's layouts with D zero-padded to 32:
 *   Qp     io   (N, H, ldn, 32): scale * log2(e) * q, d permuted as in tops_tri_prep, zero for d >= D
 *   KV     io   (N, H, ldn/64, 4096): K and V^T as in tops_tri_prep, zero for d >= D or keys >= N
 *   btiles io   (H, ceil(N/32), ldn/32, 1024): log2(e) * bias in tops_tri_prep's tile order
 * tops_tri_attention then writes O with D columns per head (D in {8, 16, 24, 32}), or with 32 of
 * which the first D are the result.
 * N <= 16384, ldn = max(64, round_up(N, 64)); bf16 / fp16.
 */
int tops_tri_repack(const void* q, const void* k, const void* v, const float* bias, void* Qp, void* KV, void* btiles,
                    int64_t N, int64_t ldn, int64_t H, int64_t D, float scale, int dtype, void* stream);

/*
 * Gate + output projection over M1*M2 tokens.  Replaces `fused_gate_forward` /
 * `fused_gate_kernel` (triangle_attn/kernel.py:387-470) and the apb epilogue
 * (attn_pair_bias/module.py:69-70):
 *   out[t] = ((o[t] * sigmoid(g[t] Wg^T + bg)) -> io) Wo^T + bo,  g = LN(gin) if apply_ln else gin
 *   o      io   token (m1, m2) at o[m1*so0 + m2*so1 + c], c < C (strides multiples of 8,
 *               16-byte aligned base)
 *   gin    io   token (m1, m2) at gin[m1*sg0 + m2*sg1 + c], same constraints;  w_ln, b_ln io (C,)
 *   Wg, Wo io   (C, C) in (out, in) layout;  bg, bo io (C,) or NULL
 *   out    io   (M1*M2, C) contiguous.  C (= C_in = H*D = C_out) in {128, 64}.
 */
int tops_gate_out(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                  const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg, const void* bg,
                  const void* Wo, const void* bo, void* out, int64_t M1, int64_t M2, int64_t C, int dtype,
                  void* stream);

/*
 * Residual-fused output kernels for composing a Pairformer block (z <- z + op(z)); the
 * reference has no block composition, these serve the step after each of its ops (no
 * counterpart in the reference):
 * tops_tmu_output_phase_residual: as tops_tmu_output_phase with out = res + result, res io
 *   (B, L, L, C_out) contiguous (16-byte aligned at the tuned shape).
 * tops_gate_out_residual / tops_gate_out_generic_residual: as tops_gate_out /
 *   tops_gate_out_generic with out[m1, m2] = res[m1, m2] + result, token (m1, m2) of res at
 *   res[m1*sr0 + m2*sr1 + c] and of out at out[m1*sd0 + m2*sd1 + c] (the ending node writes
 *   straight into the untransposed pair tensor); the tuned kernel needs strides that are
 *   multiples of 8 and 16-byte aligned bases.
 * Each sum is rounded once to the I/O type, from the result already rounded, as a separate
 * `res + result` in the I/O type would be.
 */
int tops_tmu_output_phase_residual(const void* y, const void* x, const void* Wp, const void* Wg, const float* sWp,
                                   const float* sWg, const float* Bp, const float* Bg, const void* res, void* out,
                                   int64_t B, int64_t L, int64_t C, int64_t C_out, int64_t ldy, float eps, int dtype,
                                   void* stream);
int tops_gate_out_residual(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                           const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg,
                           const void* bg, const void* Wo, const void* bo, const void* res, int64_t sr0, int64_t sr1,
                           void* out, int64_t sd0, int64_t sd1, int64_t M1, int64_t M2, int64_t C, int dtype,
                           void* stream);
int tops_gate_out_generic_residual(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0,
                                   int64_t sg1, const void* w_ln, const void* b_ln, float ln_eps, int apply_ln,
                                   const void* Wg, const void* bg, const void* Wo, const void* bo, const void* res,
                                   int64_t sr0, int64_t sr1, void* out, int64_t sd0, int64_t sd1, int64_t M1,
                                   int64_t M2, int64_t Cin, int64_t HD, int64_t Cout, int dtype, void* stream);

/*
 * attention_pair_bias core.  Replaces `apb_forward` + `_apb_kernel`
 * (attn_pair_bias/kernel.py:205-257, :24-202).
 *   X      io   (M, C) contiguous, C == 128
 *   wqkv   io   (H, 3, D, C): per head the rows of WQ^T, WK^T, WV^T (feature-major)
 *   Z      io   element (q, k, c) at Z[q*sz0 + k*sz1 + c], c < Cz, Cz == 128
 *   Wc     fp32 (H, Cz) LN-folded bias weight;  sWc, Bc fp32 (H,)
 *   mask   int8 (M,) key mask (nonzero = valid) or NULL; masked keys get -inf
 *   Og     io   (M, H*D) contiguous: softmax_k(scale * Q.K + LN(Z[q,k]) . W + b) V
 *   work   device scratch of tops_apb_workspace_bytes(M, H, D) bytes (caller-owned): the
 *          projected Q / K / V (3 * M * 128 * 2 bytes, rounded up to 256) and the split partials
 * Og may be NULL when the keys are split (tops_apb_workspace_bytes exceeds the Q / K / V region):
 * the attention's fp32 split partials then stay in `work` right after Q / K / V, the input of
 * tops_apb_merge_gate.
 */
int64_t tops_apb_workspace_bytes(int64_t M, int64_t H, int64_t D);
int tops_apb_forward(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1, const float* Wc,
                     const float* sWc, const float* Bc, const void* mask, void* Og, void* work, int64_t M, int64_t C,
                     int64_t Cz, int64_t H, int64_t D, float scale, float eps, int dtype, void* stream);

/*
 * attention_pair_bias forward with the gate and output projection fused after the attention:
 * replaces `apb_forward` followed by attn_pair_bias/module.py:69-70
 *   out = ((Og * sigmoid(X . Wg^T + bg)) -> io) . Wo^T + bo   (+ res when res != NULL)
 * with Og as tops_apb_forward computes it (same bits).  Same arguments as tops_apb_forward plus
 *   Wg, Wo io (128, 128) nn.Linear (out, in) weights;  bg, bo io (128,) or NULL (zero)
 *   res    io (M, 128) contiguous or NULL: the residual added before the single rounding
 *   out    io (M, 128) contiguous
 *   work   tops_apb_gated_workspace_bytes(M, H, D) bytes (Q / K / V, then the split partials,
 *          or Og when the keys are not split)
 * C == Cz == C_out == 128, H == 4, D == 32, 16-bit I/O.  With split keys the split merge, gate and
 * output projection are one kernel (apb_merge_gate_kernel), otherwise tops_gate_out runs.
 */
int64_t tops_apb_gated_workspace_bytes(int64_t M, int64_t H, int64_t D);
int tops_apb_forward_gated(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1, const float* Wc,
                           const float* sWc, const float* Bc, const void* mask, const void* Wg, const void* bg,
                           const void* Wo, const void* bo, const void* res, void* out, void* work, int64_t M,
                           int64_t C, int64_t Cz, int64_t H, int64_t D, int64_t Cout, float scale, float eps,
                           int dtype, void* stream);

/*
 * The last launch of tops_apb_forward_gated on its own (no separate counterpart in the reference:
 * the split merge of the attention's partials, then attn_pair_bias/module.py:69-70's gate and W_o):
 * part = the fp32 split partials as the attention left them (tops_apb_forward_qkv with Og == NULL
 * leaves them at the head of its `work`), X / Wg / bg / Wo / bo / res / out as in
 * tops_apb_forward_gated.  Only for M whose keys are split (TOPS_EINVAL otherwise).
 */
int tops_apb_merge_gate(const float* part, const void* X, const void* Wg, const void* bg, const void* Wo,
                        const void* bo, const void* res, void* out, int64_t M, int64_t H, int64_t D, int dtype,
                        void* stream);

/*
 * tops_apb_forward without allocation: no counterpart in the reference.  For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same computation and arguments as tops_apb_forward minus `work`; the workspace is
 * a library-owned static device array of 16 MiB per GPU (held until the process ends), so calls
 * with tops_apb_workspace_bytes(M, H, D) > 16 MiB return TOPS_EINVAL (on a 256-CU MI355X every M up
 * to 6990 fits, and M in 8161..9039 or 16353..21845, where the keys are split into fewer parts;
 * other M up to 16352 need the split partials of tops_apb_forward's workspace).  The entry point
 * allocates nothing and calls no allocating routine; the array's device
 * address is looked up once per device on the first call made with that device current.  Every
 * call on one GPU shares that GPU's array: calls that overlap in time on one GPU (other streams,
 * other threads) race; calls ordered on one stream do not.  Nothing in the array needs to start
 * at zero (each call writes every byte it reads).
 */
int tops_apb_forward_noalloc(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1,
                             const float* Wc, const float* sWc, const float* Bc, const void* mask, void* Og, int64_t M,
                             int64_t C, int64_t Cz, int64_t H, int64_t D, float scale, float eps, int dtype,
                             void* stream);

/*
 * Q / K / V pre-pass and the attention with given Q / K / V.  tops_apb_forward is the two run
 * back to back (Q scaled by `scale` in the pre-pass, Q / K / V at the head of `work`).  They also
 * serve the qk-norm variant of attention_pair_bias (the K-Fold formulation the reference states
 * in benchmarks/references.py:230-277 as `torch_attn_pair_bias_qknorm`; the reference has no
 * kernel for it, so these entry points replace that torch function).
 * tops_apb_qkn_prep, any C, H, D with C + 3*H*D <= 2040, io bf16 / fp16 / fp32:
 *   X      io   (M, C) contiguous;  wqkv io (H, 3, D, C) as in tops_apb_forward
 *   bq     io   (H*D,) Q bias or NULL
 *   qkn    1: q and k are LayerNormed over the full H*D channel (eps) with affine
 *           gq / bqn (for q) and gk / bkn (for k), io (H*D,) each or NULL (= 1 / 0)
 *   q,k,v  io   (M, H*D) contiguous: qscale * LN(X.Wq + bq), LN(X.Wk), X.Wv (fp32 accumulation,
 *               one rounding)
 * tops_apb_forward_qkv, the tuned shape (H*D == Cz == 128, H == 4, D == 32), bf16 / fp16: as
 *   tops_apb_forward with Q, K, V (M, H*D) contiguous taken as they are: Og = softmax_k(scale *
 *   q.k + LN(Z[q,k]) . W + b, masked keys -inf) v;  work as for tops_apb_forward.  With Og == NULL
 *   (only for M whose keys are split) the attention kernel runs alone and leaves its fp32 split
 *   partials at the head of `work` (the input of tops_apb_merge_gate).
 */
int tops_apb_qkn_prep(const void* X, const void* wqkv, const void* bq, int qkn, const void* gq, const void* bqn,
                      const void* gk, const void* bkn, void* q, void* k, void* v, int64_t M, int64_t C, int64_t H,
                      int64_t D, float qscale, float eps, int dtype, void* stream);
int tops_apb_forward_qkv(const void* Q, const void* K, const void* V, const void* Z, int64_t sz0, int64_t sz1,
                         const float* Wc, const float* sWc, const float* Bc, const void* mask, void* Og, void* work,
                         int64_t M, int64_t HD, int64_t Cz, int64_t H, int64_t D, float scale, float eps, int dtype,
                         void* stream);

/*
 * Any-shape triangle attention (C_in, H, D other than 128, 4, 32; e.g. the D = 16, C_in = 64
 * "Apo" shape of tests/test_triangle_attn.py:137-192).  The same three phases as above with
 * plain layouts; they replace the reference's Triton path for those shapes
 * (triangle_attn/kernel.py:256-340 with `separate_kv = D == 16`, :282).
 *
 * tops_tri_generic_prep: per token (a, b) of x (token at x[a*sx0 + b*sx1 + c], c < C):
 *   xln    io   (N*N, C) contiguous: LN(x) (or x when apply_ln == 0)
 *   q,k,v  io   (N, N, H, D) contiguous: LN(x) . W^T per head, wqkv as in tops_tri_prep
 *   bias   fp32 (H, N, N): LN(x[a, b]) . WZ[h] + BZ[h] (unrounded LN), WZ io (H, C), BZ fp32 or NULL
 *   C <= 1024, H <= 64, D <= 64.
 * tops_tri_generic_attention: out[i*so0 + q*so1 + h*D + d] =
 *   softmax_k(scale * q[i,q,h] . k[i,k,h] + bias[h,q,k] (+ -1e9 where mask[i*sm0 + k*sm1] == 0)) v
 *   (fp32 scores; mask int8 or NULL).
 * tops_gate_out_generic: tops_gate_out for any (C_in, H*D, C_out) with C_in + H*D <= 1024:
 *   Wg io (H*D, C_in), Wo io (C_out, H*D) in (out, in) layout, o / gin at any token strides.
 */
int tops_tri_generic_prep(const void* x, int64_t sx0, int64_t sx1, const void* w_ln, const void* b_ln, int apply_ln,
                          const void* wqkv, const void* WZ, const float* BZ, void* xln, void* q, void* k, void* v,
                          float* bias, int64_t N, int64_t C, int64_t H, int64_t D, float eps, int dtype,
                          void* stream);
int tops_tri_generic_attention(const void* q, const void* k, const void* v, const float* bias, const void* mask,
                               int64_t sm0, int64_t sm1, void* out, int64_t so0, int64_t so1, int64_t N, int64_t H,
                               int64_t D, float scale, int dtype, void* stream);
/*
 * Any-shape attention_pair_bias (C_s, C_z, H, D other than 128, 128, 4, 32) and its fp32 I/O;
 * replaces attn_pair_bias/kernel.py:205-257 for those shapes.
 * tops_apb_generic_prep: q, k, v io (M, H, D) = X . W per head (wqkv as in tops_apb_forward);
 *   bias fp32 (H, M, M) = LN(Z[q, k, :]) . W + b in the folded form (Wc fp32 (H, Cz), Bc fp32 (H,)).
 * tops_apb_generic_attention: Og io (M, H*D) = softmax_k(scale q . k + bias, masked keys -inf) v;
 *   mask int8 (M,) or NULL.
 * The gate + output projection is tops_gate_out / tops_gate_out_generic.
 */
int tops_apb_generic_prep(const void* X, const void* wqkv, const void* Z, int64_t sz0, int64_t sz1, const float* Wc,
                          const float* Bc, void* q, void* k, void* v, float* bias, int64_t M, int64_t C, int64_t Cz,
                          int64_t H, int64_t D, float eps, int dtype, void* stream);
int tops_apb_generic_attention(const void* q, const void* k, const void* v, const float* bias, const void* mask,
                               void* Og, int64_t M, int64_t H, int64_t D, float scale, int dtype, void* stream);
int tops_gate_out_generic(const void* o, int64_t so0, int64_t so1, const void* gin, int64_t sg0, int64_t sg1,
                          const void* w_ln, const void* b_ln, float ln_eps, int apply_ln, const void* Wg,
                          const void* bg, const void* Wo, const void* bo, void* out, int64_t M1, int64_t M2,
                          int64_t Cin, int64_t HD, int64_t Cout, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIANGLEOPS_AMD_H */
