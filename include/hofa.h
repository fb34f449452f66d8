/*
 * hofa.h - C ABI of the MI355X (gfx950) HOFA hybrid-attention library.
 *
 * Plain pointers, sizes and element strides only: no framework types cross
 * this boundary.  Every entry point enqueues work on the HIP stream passed as
 * `stream` (a hipStream_t; NULL = the legacy default stream), returns 0 on
 * success and a negative code on a rejected argument or a launch error;
 * hofa_last_error() then describes the failure (thread-local string).
 *
 * Paths in comments are relative to the reference repository root.
 */
#ifndef HOFA_H
#define HOFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum { HOFA_F32 = 0, HOFA_BF16 = 1, HOFA_F16 = 2 };

/* Error codes. */
enum { HOFA_OK = 0, HOFA_EINVAL = -1, HOFA_EUNSUPPORTED = -2, HOFA_ELAUNCH = -3, HOFA_EWORKSPACE = -4 };

/*
 * A strided tensor view: base pointer, element type and element strides of
 * up to four dimensions (unused trailing strides are ignored).  Sizes come
 * from the scalar fields of the argument struct that holds the view.
 */
typedef struct {
    const void *data;
    int32_t dtype;
    int32_t reserved;
    int64_t stride[4];
} hofa_view_t;

/* ------------------------------------------------------------------------
 * Split-K decode of one token.
 *
 * Replaces fused_hofa_decode(q, k, v, cache_k, cache_v, state_I_in,
 * state_I_out, log_gamma, mix_g, norm_w, R, seq_len, sm_scale, split_k,
 * log_alpha) (src/hofa_decode_triton.py:342-476) and the three Triton kernels
 * behind it (:48-159, :173-239, :242-340).
 *
 *   outlier:  y_O = softmax(q[:R] . cache_k[0:seq_len]^T * sm_scale) cache_v[0:seq_len]
 *   inlier:   S'  = gamma (.) S_in + k[R:]^T v ;  y_I = q[R:] S'
 *             gamma_j = exp(log_gamma * exp(log_alpha[h, j]))  (exp(log_gamma) without alpha)
 *   output:   y = mix * y_O + (1 - mix) * RMSNorm(y_I; eps) * norm_w[h]
 *
 * Views (element strides; q/k/v/cache/y share one dtype, f32 | bf16 | f16):
 *   q, k, v    [B,H,1,D]       stride[0..3] = b, h, n, d
 *   cache_k    [B,H,L,R]       stride[3] must be 1, rows 16-byte aligned
 *   cache_v    [B,H,L,D]       stride[3] must be 1, rows 16-byte aligned
 *   state_in   [B,H,J,D] f32   contiguous  (J = D - R)
 *   state_out  [B,H,J,D] f32   contiguous, must not alias state_in
 *   log_gamma  [B,H,1]         stride[0..1] = b, h  (f32 | bf16 | f16)
 *   mix        [B,H,1]         stride[0..1] = b, h  (0 strides allowed)
 *   norm_w     [H,D]           stride[0..1] = h, d
 *   log_alpha  [H,J]           stride[0..1] = h, j; data NULL = no alpha
 *   y          [B,H,1,D]       output
 * seq_len rows of the caches are read (the new token already written at row
 * seq_len-1).  When seq_len_dev is non-NULL the count is read on the device
 * at run time (graph replay with an advancing position) and cache_len bounds
 * it.  split_k = 0 chooses the split count from the CU count (at most 64).
 * Supported: D in {64, 128}, R in {16, 32, 64}, 8*R >= D, R < D; one head's
 * cache must span less than 2 GiB.  The call enqueues two kernels (cache
 * streaming, then the per-head state update and merge).
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, H, D, R;
    int32_t seq_len;
    int32_t cache_len;
    const int32_t *seq_len_dev;
    float sm_scale;
    float eps;
    int32_t split_k;
    int32_t reserved;
    hofa_view_t q, k, v;
    hofa_view_t cache_k, cache_v;
    hofa_view_t state_in, state_out;
    hofa_view_t log_gamma, mix, norm_w, log_alpha;
    hofa_view_t y;
} hofa_decode_args_t;

/* Bytes of scratch the call needs (depends on B, H, D and the split plan):
 * one partial (m, l, acc[D]) per stream block.  No initialisation is needed;
 * calls that share a buffer must be stream-ordered.  Returns 0 for rejected
 * arguments. */
size_t hofa_decode_workspace_bytes(const hofa_decode_args_t *args);

/* No reference counterpart beyond the split choice at
 * src/hofa_decode_triton.py:374-383: reports the split count and tokens per
 * split the call would use. */
int hofa_decode_plan(const hofa_decode_args_t *args, int32_t *split_k, int32_t *tokens_per_split);

int hofa_decode(const hofa_decode_args_t *args, void *workspace, size_t workspace_bytes, void *stream);

/*
 * hofa_decode_static: hofa_decode without a caller workspace and without any
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The split-K partials go to a file-scope
 * device array of HOFA_DECODE_STATIC_SCRATCH_BYTES per GPU, which the library
 * holds until the process ends; a call whose plan needs more (see
 * hofa_decode_workspace_bytes) is rejected with HOFA_EWORKSPACE.  At cfg3
 * (B=4, H=16, d_h=64) a call uses about 0.8 MiB.  Same kernels, split plan and
 * results as hofa_decode.  Every call on one GPU shares that GPU's array:
 * calls that may overlap on one GPU (different streams, concurrent threads)
 * race and must be serialised by the caller.  Nothing in the array needs
 * initialisation; the caller still passes inputs and outputs.
 */
#define HOFA_DECODE_STATIC_SCRATCH_BYTES (8u << 20)
int hofa_decode_static(const hofa_decode_args_t *args, void *stream);

/* ------------------------------------------------------------------------
 * Outlier pathway of the prefill: causal softmax attention on the first R
 * channels of Q/K against full-width V, mixed into the output.
 *
 * Replaces exact_attention_triton(q, k, v, r, sm_scale, mix_g, out, split_k)
 * (src/exact_attention.py:163-188) and its kernel _fwd_kernel (:46-161):
 *
 *   O = softmax(Q[..., :R] K[..., :R]^T * sm_scale + causal mask) V
 *   y = (accumulate ? y : 0) + mix * O        (mix = 1 when mix.data is NULL)
 *
 * Views (element strides b, h, t, d; q/k/v/y/o share one dtype f32|bf16|f16;
 * the last stride must be 1 and rows 16-byte aligned):
 *   q, k, v, y    [B,H,T,D]
 *   mix           [B,H,T]   strides b, h, t (f32|bf16|f16)
 *   o             optional [B,H,T,D]: O itself (data NULL = not written)
 *   acc           optional float32 [B,H,T,D] (strides b, h, t; unit last
 *                 stride, 16-byte aligned rows): y = acc + mix * O, rounded
 *                 once to the dtype of y (accumulate is then ignored).  With
 *                 hofa_gla_fwd writing its float32 result to acc, the two
 *                 pathways meet with a single rounding of the output.
 * lse (optional, float32 [B*H*T], NULL = not written) receives the base-2
 * log-sum-exp of the scaled logits per query row (log2 of the softmax
 * denominator, with logits multiplied by sm_scale*log2(e)).
 * Supported: D in {64, 128}, R in {16, 32, 64}, R <= D.  bf16 and f32 use
 * bf16 matrix cores (f32 logits from split hi/lo bf16 operands), f16 uses
 * f16 matrix cores; accumulation is f32.
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, H, T, D, R;
    float sm_scale;
    int32_t accumulate;
    int32_t reserved;
    hofa_view_t q, k, v;
    hofa_view_t mix;
    hofa_view_t y;
    hofa_view_t o;
    float *lse;
    hofa_view_t acc;
} hofa_attn_fwd_args_t;

int hofa_attn_fwd(const hofa_attn_fwd_args_t *args, void *stream);

/* ------------------------------------------------------------------------
 * Inlier pathway of the prefill: chunked gated linear attention over the
 * channels [R, D) of Q/K with full-width V, 64-token chunks.
 *
 * Replaces chunk_gla_inlier_fwd(Q, K, V, log_gamma, r, chunk_size, log_alpha,
 * mix_g, gla_scale, out, states_in, requires_grad) (src/chunk_gla_inlier.py:153-237)
 * and chunk_gla_fwd_kernel (:6-150):
 *
 *   S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,   Y_I[t] = q_t S_t     (S_0 = 0)
 *   g_{t,c} = log_gamma_t * exp(log_alpha[h, c])     (or the general g[t, c])
 *   y = fuse_norm_gate ? (1 - mix) * gla_scale * RMSNorm(Y_I; eps) : Y_I
 *   state_out = S_T
 *
 * Views (element strides; q/k/v share one dtype f32|bf16|f16, unit last
 * stride, 16-byte aligned rows):
 *   q, k, v, y     [B,H,T,D]      strides b, h, t, d; y has the dtype of q or
 *                                 is float32 (the result unrounded, e.g. the
 *                                 acc input of hofa_attn_fwd)
 *   log_gamma      [B,H,T]        strides b, h, t (f32|bf16|f16); used when g.data is NULL
 *   log_alpha      [H,J]          strides h, j; optional
 *   g              [B,H,T,J] f32  strides b, h, t, j; optional general decay (wins over log_gamma)
 *   mix            [B,H,T]        strides b, h, t (needed when fuse_norm_gate)
 *   gla_scale      [H,D]          strides h, d (needed when fuse_norm_gate)
 *   state_out      [B,H,J,D] f32  strides b, h, j, d; with state_pad_rows = P > 0
 *                  rows J .. J+P-1 (same strides, P <= J) are written with zeros:
 *                  the reference returns the state zero-padded to [B,H,j_pad,d_pad]
 *   chunk_states   optional 16-bit [B*H][ceil(T/64)][4][D*J] receiving the
 *                  state that enters each chunk as bf16 hi/lo operand pairs
 *                  (hi + lo ~ the fp32 state): planes 0/1 transposed [D][J],
 *                  planes 2/3 as [J][D] (written for D = 128 only: for D = 64 the
 *                  backward reads S from the S^T planes); saved for hofa_gla_bwd
 *   n_out          optional [B,H,T,D] (dtype of y): RMSNorm(Y_I) before the
 *                  gate, saved for hofa_gla_bwd (needs fuse_norm_gate)
 *   rstd           float32 [B*H*T] receiving 1/sqrt(mean(Y_I^2) + eps) when
 *                  n_out is given
 *   round_operands 0: matrix-core operands are split hi/lo bf16 pairs for
 *                  every input dtype, so the result tracks an fp32
 *                  computation.  1 (bf16/f16 inputs, no chunk_states): each
 *                  operand of the in-chunk and inter-chunk products and the
 *                  entering state are rounded to bf16 once, as the reference
 *                  kernel rounds its dot operands (src/chunk_gla_inlier.py:96-121);
 *                  ignored for f32 inputs.
 * Supported: D in {64, 128}, J = D - R a multiple of 16.  Decay per token
 * must be <= 0 (log of a factor in (0, 1]).
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, H, T, D, R;
    float eps;
    int32_t fuse_norm_gate;
    int32_t state_pad_rows;
    hofa_view_t q, k, v;
    hofa_view_t log_gamma, log_alpha, g;
    hofa_view_t mix, gla_scale;
    hofa_view_t y;
    hofa_view_t state_out;
    void *chunk_states;
    hofa_view_t n_out;
    float *rstd;
    int32_t round_operands;
    int32_t reserved;
} hofa_gla_fwd_args_t;

size_t hofa_gla_fwd_workspace_bytes(const hofa_gla_fwd_args_t *args);
int hofa_gla_fwd(const hofa_gla_fwd_args_t *args, void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------
 * Backward of the outlier pathway (causal softmax attention, QK width R,
 * value width D).
 *
 * No reference kernel: the reference trains through autograd of torch SDPA
 * (src/HybridOutlierFactorizedAttentionTrain.py:258-259).  Given the
 * upstream gradient dout of O = softmax(Q K^T sm_scale) V, the base-2 lse
 * written by hofa_attn_fwd and delta = rowsum(dout (.) O):
 *   dv = P^T dout (+ dv when dv_accumulate), dq = sm_scale dS K,
 *   dk = sm_scale dS^T Q,  dS = P (.) (dout V^T - delta)
 * Views (element strides b, h, t, d; one dtype f32|bf16|f16; unit last
 * stride, 16-byte aligned rows): q, k, dq, dk [B,H,T,>=R] (columns [0,R)
 * used / written); v, dout, dv [B,H,T,D].  lse, delta float32 [B*H*T].
 * Supported: D in {64, 128}, R in {16, 32, 64}, R <= D.  Matrix-core
 * operands are 16-bit (bf16 for bf16/f32 inputs, f16 for f16), f32 accumulate.
 * Two kernels (dk/dv per key block, dq per query block), no atomics.
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, H, T, D, R;
    float sm_scale;
    int32_t dv_accumulate;
    int32_t reserved;
    hofa_view_t q, k, v, dout;
    const float *lse;
    const float *delta;
    hofa_view_t dq, dk, dv;
} hofa_attn_bwd_args_t;

int hofa_attn_bwd(const hofa_attn_bwd_args_t *args, void *stream);

/* ------------------------------------------------------------------------
 * Backward of the inlier pathway and of the fused norm/gate epilogue.
 *
 * No reference kernel: the reference trains through autograd of fla's
 * chunk_gla, nn.RMSNorm, the gla_scale product and torch.lerp
 * (src/HybridOutlierFactorizedAttentionTrain.py:263-294).  For
 *   Y = (1 - mix) * gla_scale * N + mix * O,   N = RMSNorm(Y_I; eps),
 *   Y_I = GLA(q[..., R:], k[..., R:], v, g)
 * and the upstream gradient dy, writes
 *   dq, dk          columns [R, D) (columns [0, R) are not touched)
 *   dv              the GLA part of dv (overwritten)
 *   d_log_gamma     [B,H,T] (scalar decay) or d_g [B,H,T,J] f32 (general g)
 *   d_log_alpha     [H,J] (when log_alpha is given; optional)
 *   d_mix           [B,H,T] (optional; mix.data NULL means mix = 0)
 *   d_gla_scale     [H,D]
 *   dout_attn       optional [B,H,T,D] = mix * dy, and delta float32 [B*H*T]
 *                   = rowsum(dout_attn (.) O): the inputs of hofa_attn_bwd
 * Saved from the forward: n = RMSNorm(Y_I) and rstd (hofa_gla_fwd n_out /
 * rstd), chunk_states (four planes), o = the attention output O
 * (hofa_attn_fwd o; needed for d_mix and delta).
 * Views as in hofa_gla_fwd; dq, dk, dv, dy, n, o, dout_attn share the dtype
 * of q.  Small per-head / per-token outputs take any dtype.  Matrix-core
 * operands are hi/lo bf16 pairs (fp32-like products), like the forward.
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, H, T, D, R;
    int32_t reserved;
    hofa_view_t q, k, v;
    hofa_view_t log_gamma, log_alpha, g;
    hofa_view_t mix, gla_scale;
    hofa_view_t n, o;
    const float *rstd;
    const void *chunk_states;
    hofa_view_t dy;
    hofa_view_t dq, dk, dv;
    hofa_view_t d_log_gamma, d_g, d_log_alpha, d_mix, d_gla_scale;
    hofa_view_t dout_attn;
    float *delta;
} hofa_gla_bwd_args_t;

size_t hofa_gla_bwd_workspace_bytes(const hofa_gla_bwd_args_t *args);
int hofa_gla_bwd(const hofa_gla_bwd_args_t *args, void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------
 * Single-token decode of a TransformerBlock: the work around hofa_decode.
 *
 * hofa_rows_linear: a row-batched linear for decode (B <= 4 rows),
 *   xn      = LayerNorm(x; ln_w, ln_b, ln_eps) when ln_w is non-NULL, else x,
 *             rounded to dtype (the output of nn.LayerNorm)
 *   t       = round(xn[b] . w[n] + bias[n])            bias optional
 *   t       = round(GELU_erf(t))                       act = 1
 *   t       = round(t * scale)                         n < scale_cols
 *   y[b, n] = round(res[b, n] + t)                     res optional, may alias y
 * With argmax non-NULL it also writes, for every batch row b and every block
 * i of 16 output rows, the block's greatest key of y[b, n] (order-preserving
 * value bits << 32 | 0xffffffff - n, so ties go to the first index) to
 * argmax[b * ceil(N/16) + i]; argmax holds B * ceil(N/16) entries and needs
 * no initialisation.  Replaces, for one token, nn.LayerNorm +
 * nn.Linear (+ nn.GELU) + the residual add of TransformerBlock.forward_step
 * (src/HybridOutlierFactorizedAttention.py:447-451), the scaled W_q/W_k/W_v
 * projections of forward_step (:223-235), out_proj, and SubwordLM.lm_head
 * (:471) with the greedy argmax of src/inference.py:220-221.
 * Rows are contiguous; x, ln_w, ln_b, w, bias, res and y share dtype
 * (bf16 | f16).  w is [N, K] (nn.Linear layout), 16-byte aligned.
 * Supported: 1 <= B <= 4, K a multiple of 8 and at most 4096.
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, K, N, dtype;
    int32_t act;
    int32_t scale_cols;
    float scale;
    float ln_eps;
    const void *x;
    int64_t x_stride;
    const void *ln_w, *ln_b;
    const void *w;
    const void *bias;
    const void *res;
    int64_t res_stride;
    void *y;
    int64_t y_stride;
    unsigned long long *argmax;
} hofa_rows_linear_args_t;

int hofa_rows_linear(const hofa_rows_linear_args_t *args, void *stream);

/*
 * hofa_decode_prologue: per (b, h), from qkv = [B, 3*H*D] (Q | K | V of one
 * token, Q and K already scaled by d_h^-1/4):
 *   gate = round(Q . gate_w[h, :D] + K . gate_w[h, D:] + gate_b[h])
 *   log_gamma[b, h] = round(logsigmoid(-gate))                       (f32 out)
 *   mix[b, h] = round(sigmoid(round(Q . mix_w[h, :D] + K . mix_w[h, D:] + mix_b[h])))
 *               or round(sigmoid(fixed_mix[h]))                      (f32 out)
 *   Q[:R], K[:R] <- RoPE at row *pos of cos/sin [rope_rows, R] (in place in
 *                   qkv; skipped when cos is NULL).  Tables are f32 (one
 *                   rounding) or of the qkv dtype (rope_dtype; each product
 *                   rounded, as a 16-bit module computes it)
 *   cache_k[b, h, *pos, :] = K[:R],  cache_v[b, h, *pos, :] = V
 * Replaces the gates, RoPE and cache append of forward_step
 * (src/HybridOutlierFactorizedAttention.py:67-95, :365-387) with the
 * position read on the device.  Caches are contiguous [B,H,cache_len,R] and
 * [B,H,cache_len,D]; gate_w/mix_w [H, 2D]; everything shares dtype
 * (bf16 | f16) except cos/sin, log_gamma/mix (f32) and pos (int64).
 * Supported: D in {64, 128}, R even, 0 < R <= 64, R < D.
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, H, D, R;
    int32_t dtype;
    int32_t cache_len;
    int32_t rope_rows;
    int32_t rope_dtype;
    void *qkv;
    int64_t qkv_stride;
    const void *gate_w, *gate_b;
    const void *mix_w, *mix_b;
    const void *fixed_mix;
    const void *cos, *sin;
    const int64_t *pos;
    void *cache_k, *cache_v;
    float *log_gamma, *mix;
} hofa_decode_prologue_args_t;

int hofa_decode_prologue(const hofa_decode_prologue_args_t *args, void *stream);

/*
 * hofa_decode_fused: hofa_decode with hofa_decode_prologue folded into its
 * launch, for a caller (the greedy graph decoder) that would run the two back
 * to back.  q, k, v are the pre-RoPE scaled projections (as handed to
 * hofa_decode_prologue); the position is pos = seq_len - 1 (seq_len_dev or
 * seq_len); the log_gamma and mix views are not read (they come from the
 * gates).  The state block of each head computes the gates, rotates the
 * outlier channels, appends cache row pos, adds the token's own softmax term
 * as one more split partial and updates the GLA state; the stream blocks
 * rotate q themselves and read rows [0, pos).  Same results as the two calls
 * (up to the summation order of the token's score).  Supported: bf16 | f16;
 * the prologue's B, H, D, R and dtype must match.  Replaces, per token, the
 * same reference code as the two calls it fuses.
 * ---------------------------------------------------------------------- */
size_t hofa_decode_fused_workspace_bytes(const hofa_decode_args_t *args);
int hofa_decode_fused(const hofa_decode_args_t *args, const hofa_decode_prologue_args_t *prologue,
                      void *workspace, size_t workspace_bytes, void *stream);

/*
 * hofa_decode_advance: ends one greedy step.  For each batch row b the token
 * idx = the index in the greatest of argmax[b * ceil(vocab/16) + i] (the LM
 * head's per-block keys, see hofa_rows_linear) is written to tok[b]
 * and out[b, *col] (when *col < out_cols), and emb[idx, :] (the tied
 * embedding, [vocab, d_model]) becomes x[b, :], the next step's input; then
 * *col, *pos and *seq_len advance by one.  Replaces
 * the greedy feedback of the generation loop (src/inference.py:220-239).
 * Supported: 1 <= B <= 4; emb and x share dtype (bf16 | f16).
 * ---------------------------------------------------------------------- */
typedef struct {
    int32_t B, d_model, vocab, dtype;
    int32_t out_cols;
    int32_t reserved;
    const unsigned long long *argmax;
    const void *emb;
    void *x;
    int64_t x_stride;
    int64_t *tok;
    int64_t *out;
    int64_t out_stride;
    int64_t *col, *pos;
    int32_t *seq_len;
} hofa_decode_advance_args_t;

int hofa_decode_advance(const hofa_decode_advance_args_t *args, void *stream);

/* Library-wide helpers. */
const char *hofa_last_error(void);
int hofa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HOFA_H */
