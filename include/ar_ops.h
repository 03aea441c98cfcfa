/*
 * ar_ops.h -- C ABI of the MI355X (gfx950) kernel library for the
 * autoresearch GPT training step (libautoresearch_amd.so).
 *
 * One entry point per GPU kernel of the Mojo reference
 * (sergeytimoshin/autoresearch: kernels/ops.mojo, optimizer.mojo,
 * model.mojo), with the reference kernel's argument order and meaning.
 * Each entry point replaces one `ctx.enqueue_function[kernel, kernel](...)`
 * launch site: the library, not the caller, chooses the launch geometry.
 *
 * Conventions
 *   - Pointers are device pointers.  Sizes are int64_t element counts.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Calls are
 *     asynchronous on that stream, like enqueue_function.
 *   - Return AR_OK (0) or a negative ar_status; ar_last_error() returns the
 *     message of the last failure on the calling thread.
 *   - Accumulate vs overwrite follows the reference: linear_bwd_dw,
 *     embedding_bwd, ve_gate_bwd and scalar_grad_reduce accumulate (+=);
 *     every other kernel overwrites its outputs.
 *   - In-place aliasing the reference's callers rely on is supported:
 *     rmsnorm_fwd(x, rms, x), rope_fwd(q, q), softcap_fwd(l, l),
 *     add_residual_fwd/scaled_add_fwd with out == a, rmsnorm_bwd(g, g, ...),
 *     scaled_add_bwd(g, gx0, g), scale_add(X, X, G), and linear_bwd_dx with
 *     grad_input == grad_output (model.mojo:906), which reads all of dY before
 *     writing dX.
 *   - `_bf16` variants take the same fp32 buffers and compute on the bf16
 *     matrix cores (operands rounded to bf16, fp32 accumulation, fp32 out).
 *   - No entry point allocates, frees or synchronises device memory.  The
 *     ones that need scratch (split-K partials, the in-place linear_bwd_dx
 *     copy, the embedding scatter's sort and chunk sums, reduction partials,
 *     Muon temporaries, the bf16 operand copies of the attention _bf16
 *     variants) take it from the workspace the caller bound to `stream`
 *     (ar_workspace_*, below); with none bound, or one too small, they return
 *     AR_ENOMEM and ar_last_error() names the bytes needed.
 *   - Thread safety: entry points may be called from several host threads.
 *     Calls that share a workspace must not overlap in time (bind one
 *     workspace per stream, and keep each stream's calls in order, as the
 *     reference's single in-order DeviceContext does).
 */
#ifndef AR_OPS_H
#define AR_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ar_stream_t;

enum ar_status {
    AR_OK = 0,
    AR_EINVAL = -1,      /* bad pointer / shape / alias the kernel cannot honour */
    AR_EUNSUPPORTED = -2, /* e.g. head_dim > 128 (ops.mojo:267 returns silently) */
    AR_EHIP = -3,        /* HIP runtime error (launch, copy, ...) */
    AR_ENOMEM = -4
};

enum ar_precision { AR_PREC_FP32 = 0, AR_PREC_BF16 = 1 };

const char* ar_last_error(void);
int32_t ar_version(void);

/* ---------------- workspaces ----------------
 * Device scratch created by the caller, the counterpart of the DeviceBuffers
 * the reference's host code allocates for its kernels (model.mojo:263-335,
 * optimizer.mojo:86-101, 242-253): the library's entry points choose their own
 * launch geometry and scratch layout, so the scratch is one caller-owned
 * buffer instead of per-kernel buffers. */
typedef struct ar_workspace ar_workspace;
/* hipMalloc of `bytes` on the current device (the only allocation the per-op
 * entry points depend on).  Create it before a stream capture, not during. */
int32_t ar_workspace_create(ar_workspace** out, size_t bytes);
/* Per-op calls on `stream` (on the current device) use `ws` from now on; NULL
 * unbinds.  One workspace may serve several streams whose calls never overlap.
 * Bindings are keyed by the stream handle: unbind a stream
 * (ar_workspace_bind(stream, NULL)) before hipStreamDestroy, or a later stream
 * that reuses the handle inherits the binding. */
int32_t ar_workspace_bind(ar_stream_t stream, ar_workspace* ws);
/* Unbinds it everywhere, waits for its device to finish queued work, frees it. */
int32_t ar_workspace_destroy(ar_workspace* ws);
size_t ar_workspace_bytes(const ar_workspace* ws);

/* ---------------- kernels/ops.mojo ---------------- */

/* ops.mojo:41-55  output[i,d] = weight[indices[i], d] */
int32_t ar_embedding_fwd(ar_stream_t stream, float* output, const float* weight, const int64_t* indices,
                         int64_t num_tokens, int64_t embd_dim);
/* ops.mojo:61-104  y = x / sqrt(mean(x^2) + 1e-5); rms saved.  output may alias input. */
int32_t ar_rmsnorm_fwd(ar_stream_t stream, float* output, float* rms_out, const float* input,
                       int64_t num_rows, int64_t dim);
/* ops.mojo:110-203  Y[m,n] = sum_k X[m,k] W[n,k]  (NT, overwrite) */
int32_t ar_linear_fwd(ar_stream_t stream, float* output, const float* input, const float* weight,
                      int64_t M, int64_t N, int64_t K);
int32_t ar_linear_fwd_bf16(ar_stream_t stream, float* output, const float* input, const float* weight,
                           int64_t M, int64_t N, int64_t K);
/* ops.mojo:209-238  rotate halves; cos/sin row = flat token index */
int32_t ar_rope_fwd(ar_stream_t stream, float* output, const float* input, const float* cos_buf,
                    const float* sin_buf, int64_t num_tokens, int64_t num_heads, int64_t head_dim);
/* ops.mojo:244-323  causal / sliding-window softmax attention + LSE.
 * q,k,v,output: [B*T*num_heads, head_dim]; lse_out: [B*T*num_heads].
 * Key kp visible from qp iff kp <= qp and (window_size <= 0 or kp >= qp - window_size).
 * Any head_dim in [1, 128] (AR_EUNSUPPORTED above, where ops.mojo:267 returns
 * silently; AR_EINVAL for head_dim <= 0 or a negative B, T or num_heads; an
 * empty shape is AR_OK).  head_dim 32, 64 and 128 run the tiled kernels directly; any
 * other runs them at the next of those sizes on zero-padded copies of the rows
 * in the workspace (softmax scale 1/sqrt(head_dim)).  The same holds for the
 * dq and dkv entries below. */
int32_t ar_flash_attn_fwd(ar_stream_t stream, float* output, float* lse_out, const float* q, const float* k,
                          const float* v, int64_t B, int64_t T, int64_t num_heads, int64_t head_dim,
                          int64_t window_size);
int32_t ar_flash_attn_fwd_bf16(ar_stream_t stream, float* output, float* lse_out, const float* q,
                               const float* k, const float* v, int64_t B, int64_t T, int64_t num_heads,
                               int64_t head_dim, int64_t window_size);
/* ops.mojo:329-346  D[bth] = sum_d O[bth,d] dO[bth,d] */
int32_t ar_flash_attn_bwd_precompute_d(ar_stream_t stream, float* d_out, const float* output,
                                       const float* grad_output, int64_t B, int64_t T, int64_t num_heads,
                                       int64_t head_dim);
/* D for the _bf16 backward kernels: dO is rounded to bf16 exactly as those
 * kernels round it for dP = dO V^T, so that D = sum_j P_j dP_j holds and
 * dS = P (dP - D) is unbiased (pair with ar_flash_attn_fwd_bf16's O). */
int32_t ar_flash_attn_bwd_precompute_d_bf16(ar_stream_t stream, float* d_out, const float* output,
                                            const float* grad_output, int64_t B, int64_t T, int64_t num_heads,
                                            int64_t head_dim);
/* ops.mojo:349-411  dQ = scale * sum_kp P (dP - D) K */
int32_t ar_flash_attn_bwd_dq(ar_stream_t stream, float* grad_q, const float* q, const float* k, const float* v,
                             const float* grad_output, const float* lse, const float* d_buf, int64_t B, int64_t T,
                             int64_t num_heads, int64_t head_dim, int64_t window_size);
int32_t ar_flash_attn_bwd_dq_bf16(ar_stream_t stream, float* grad_q, const float* q, const float* k,
                                  const float* v, const float* grad_output, const float* lse, const float* d_buf,
                                  int64_t B, int64_t T, int64_t num_heads, int64_t head_dim,
                                  int64_t window_size);
/* ops.mojo:414-480  dK = scale * sum_qp dS Q, dV = sum_qp P dO */
int32_t ar_flash_attn_bwd_dkv(ar_stream_t stream, float* grad_k, float* grad_v, const float* q, const float* k,
                              const float* v, const float* grad_output, const float* lse, const float* d_buf,
                              int64_t B, int64_t T, int64_t num_heads, int64_t head_dim, int64_t window_size);
int32_t ar_flash_attn_bwd_dkv_bf16(ar_stream_t stream, float* grad_k, float* grad_v, const float* q,
                                   const float* k, const float* v, const float* grad_output, const float* lse,
                                   const float* d_buf, int64_t B, int64_t T, int64_t num_heads,
                                   int64_t head_dim, int64_t window_size);
/* ops.mojo:486-497  relu(x)^2 */
int32_t ar_relu_squared_fwd(ar_stream_t stream, float* output, const float* input, int64_t size);
/* ops.mojo:500-510  cap * tanh(x / cap); output may alias input */
int32_t ar_softcap_fwd(ar_stream_t stream, float* output, const float* input, float cap, int64_t size);
/* ops.mojo:516-541  gate[t,h] = 2 sigmoid(sum_{c<gate_channels} W[h,c] x[t,c]) */
int32_t ar_ve_gate_fwd(ar_stream_t stream, float* gate_out, const float* x_norm, const float* gate_weight,
                       int64_t num_tokens, int64_t n_kv_head, int64_t gate_channels, int64_t embd_dim);
/* ops.mojo:544-560  v[t,h,d] += gate[t,h] ve[t,h,d] (in place) */
int32_t ar_ve_apply_fwd(ar_stream_t stream, float* v, const float* gate, const float* ve, int64_t num_tokens,
                        int64_t n_kv_head, int64_t head_dim);
/* ops.mojo:566-576  output = residual + input */
int32_t ar_add_residual_fwd(ar_stream_t stream, float* output, const float* residual, const float* input,
                            int64_t size);
/* ops.mojo:579-594  output = scale_a[idx] a + scale_b[idx] b (device scalars) */
int32_t ar_scaled_add_fwd(ar_stream_t stream, float* output, const float* a, const float* b,
                          const float* scale_a, const float* scale_b, int64_t idx, int64_t size);
/* ops.mojo:600-666  row softmax (used only by the reference's kernel tests) */
int32_t ar_softmax_fwd(ar_stream_t stream, float* output, const float* input, int64_t num_rows, int64_t cols);
/* ops.mojo:672-740  loss[t] = lse(row) - row[target]; target < 0 gives 0 */
int32_t ar_cross_entropy_fwd(ar_stream_t stream, float* loss_out, const float* logits, const int64_t* targets,
                             int64_t num_tokens, int64_t vocab_size);
/* ops.mojo:746-772  output[0] = mean(input[0:size]) */
int32_t ar_mean_reduce(ar_stream_t stream, float* output, const float* input, int64_t size);
/* ops.mojo:778-864  grad = (softmax(capped) - onehot) * loss_scale (no softcap derivative) */
int32_t ar_cross_entropy_softcap_bwd(ar_stream_t stream, float* grad_logits, const float* logits,
                                     const int64_t* targets, float cap, int64_t num_tokens, int64_t vocab_size,
                                     float loss_scale);
/* ops.mojo:870-950  dX[m,k] = sum_n dY[m,n] W[n,k] (NN, overwrite; dX may alias dY) */
int32_t ar_linear_bwd_dx(ar_stream_t stream, float* grad_input, const float* grad_output, const float* weight,
                         int64_t M, int64_t N, int64_t K);
int32_t ar_linear_bwd_dx_bf16(ar_stream_t stream, float* grad_input, const float* grad_output,
                              const float* weight, int64_t M, int64_t N, int64_t K);
/* ops.mojo:953-1033  dW[n,k] += sum_m dY[m,n] X[m,k] (TN, accumulate, deterministic) */
int32_t ar_linear_bwd_dw(ar_stream_t stream, float* grad_weight, const float* grad_output, const float* input,
                         int64_t M, int64_t N, int64_t K);
int32_t ar_linear_bwd_dw_bf16(ar_stream_t stream, float* grad_weight, const float* grad_output,
                              const float* input, int64_t M, int64_t N, int64_t K);
/* ar_linear_bwd_dw_bf16 that needs no workspace and allocates nothing.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory or bind a workspace (code under stream capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results
 * (bit-identical); its scratch (split-K partials, zero-padded copies of
 * unaligned operands) is a fixed 64 MiB device array per device, held until
 * the process ends.  A shape that needs more returns AR_EINVAL and
 * ar_last_error() names the bytes.  All calls on one device share that array:
 * calls that overlap in time on one device race.  The first call on a device
 * looks the array's address up (hipGetSymbolAddress); make it before any
 * stream capture. */
int32_t ar_linear_bwd_dw_bf16_noalloc(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                      const float* input, int64_t M, int64_t N, int64_t K);
/* Storage-typed GEMM (no counterpart in the reference, which is fp32 only):
 * layout 0/1/2 = linear_fwd / linear_bwd_dx / linear_bwd_dw semantics with
 * X, W and C each stored as bf16 (flag 1) or fp32 (flag 0); bf16 matrix
 * cores with fp32 accumulation.  accumulate: C += result. */
int32_t ar_gemm_mixed(ar_stream_t stream, int32_t layout, void* C, int32_t c_bf16, const void* X, int32_t x_bf16,
                      const void* W, int32_t w_bf16, int64_t M, int64_t N, int64_t K, int32_t accumulate);
/* The bf16 step's fused LM-head loss.  The reference runs it as five
 * launches: linear_fwd (ops.mojo:110-203) of the final normed x by lm_head,
 * softcap_fwd (ops.mojo:500-510), cross_entropy_fwd (ops.mojo:672-740) in the
 * forward (model.mojo:745-764) and cross_entropy_softcap_bwd (ops.mojo:
 * 778-864) in the backward (model.mojo:845-850).  Here: one GEMM whose
 * epilogue applies cap * tanh(z / cap) and stores the logits as bf16, then one
 * pass per row that writes the per-token loss (lse - logit[target]; 0 for a
 * target outside [0, vocab_size)) and grad_logits = (softmax - onehot) *
 * loss_scale as bf16 (no softcap derivative, as the reference).
 * input: bf16 [num_tokens, embd_dim]; weight: bf16 [vocab_size, embd_dim];
 * logits, grad_logits: bf16 [num_tokens, vocab_size]; loss_out: fp32
 * [num_tokens] (may be NULL).  Sizes multiples of 8, pointers 16-byte aligned. */
int32_t ar_lm_head_softcap_ce_bf16(ar_stream_t stream, float* loss_out, void* grad_logits, void* logits,
                                   const void* input, const void* weight, const int64_t* targets,
                                   int64_t num_tokens, int64_t vocab_size, int64_t embd_dim, float cap,
                                   float loss_scale);
/* ops.mojo:1039-1085  dx = (dy - x <dy,x> / (dim rms^2)) / rms; grad_input may alias grad_output */
int32_t ar_rmsnorm_bwd(ar_stream_t stream, float* grad_input, const float* grad_output, const float* input,
                       const float* rms_saved, int64_t num_rows, int64_t dim);
/* ops.mojo:1091-1120  inverse rotation */
int32_t ar_rope_bwd(ar_stream_t stream, float* grad_input, const float* grad_output, const float* cos_buf,
                    const float* sin_buf, int64_t num_tokens, int64_t num_heads, int64_t head_dim);
/* ops.mojo:1126-1140  2 x dy [x > 0] */
int32_t ar_relu_squared_bwd(ar_stream_t stream, float* grad_input, const float* grad_output, const float* input,
                            int64_t size);
/* ops.mojo:1146-1164  grad_weight[idx[i], :] += dY[i, :]; summed in token order
 * (deterministic, bit-identical to a sequential CPU loop) */
int32_t ar_embedding_bwd(ar_stream_t stream, float* grad_weight, const float* grad_output,
                         const int64_t* indices, int64_t num_tokens, int64_t embd_dim);
/* ops.mojo:1170-1190  grad_a = sa[idx] g, grad_b = sb[idx] g (assign) */
int32_t ar_scaled_add_bwd(ar_stream_t stream, float* grad_a, float* grad_b, const float* grad_output,
                          const float* scale_a, const float* scale_b, int64_t idx, int64_t size);
/* ops.mojo:1193-1237  gve = gate gv; ggate = sum_d ve gv */
int32_t ar_ve_apply_bwd(ar_stream_t stream, float* grad_ve, float* grad_gate, const float* grad_v,
                        const float* gate, const float* ve, int64_t num_tokens, int64_t n_kv_head,
                        int64_t head_dim);
/* ops.mojo:1240-1274  dz = gg g (1 - g/2); gW += sum_t dz x; gx[:, :gc] += sum_h dz W (accumulate) */
int32_t ar_ve_gate_bwd(ar_stream_t stream, float* grad_x_norm_out, float* grad_gate_weight,
                       const float* grad_gate, const float* gate, const float* x_norm, const float* gate_weight,
                       int64_t num_tokens, int64_t n_kv_head, int64_t gate_channels, int64_t embd_dim);
/* ops.mojo:1277-1308  grad_scalar[idx] += sum(g x) */
int32_t ar_scalar_grad_reduce(ar_stream_t stream, float* grad_scalar, const float* grad_output,
                              const float* input, int64_t idx, int64_t size);
/* ops.mojo:1314-1322 */
int32_t ar_zero_buffer(ar_stream_t stream, float* buf, int64_t size);

/* ---------------- optimizer.mojo ---------------- */

/* optimizer.mojo:27-57 */
int32_t ar_adamw(ar_stream_t stream, float* params, const float* grads, float* exp_avg, float* exp_avg_sq,
                 float lr, float beta1, float beta2, float eps, float weight_decay, float bias_corr1,
                 float bias_corr2, int64_t size);
/* optimizer.mojo:103-127  AdamWState.step_group: lr = f32(lr_group * lrm), bias
 * corrections by `step` repeated f32 multiplications. */
int32_t ar_adamw_step_group(ar_stream_t stream, float* params, const float* grads, float* exp_avg,
                            float* exp_avg_sq, int64_t size, double lr_group, double beta1, double beta2,
                            double eps, double weight_decay, double lr_multiplier, int64_t step);
/* optimizer.mojo:132-146 */
int32_t ar_nesterov_momentum(ar_stream_t stream, float* output, const float* grads, float* momentum_buf,
                             float momentum, int64_t size);
/* optimizer.mojo:149-180  data /= (||data||_F * 1.02 + 1e-6) */
int32_t ar_normalize_frobenius(ar_stream_t stream, float* data, int64_t size);
/* optimizer.mojo:183-194  output = sa a + sb b */
int32_t ar_scale_add(ar_stream_t stream, float* output, const float* a, const float* b, float sa, float sb,
                     int64_t size);
/* optimizer.mojo:197-210  p -= lr (g + wd p [g p >= 0]) */
int32_t ar_muon_update(ar_stream_t stream, float* params, const float* grads, float lr, float wd, int64_t size);
/* optimizer.mojo:255-342  MuonState.step for one [rows, cols] matrix of any
 * shape: Nesterov -> Frobenius normalise -> 5 Polar Express iterations ->
 * cautious update.  The products run on the matrix zero-padded to multiples
 * of 8 rows and columns (zero rows / columns stay zero through the
 * iterations).  `grads` is read only (the reference uses it as scratch after its
 * last read, optimizer.mojo:317-332; its contents are not used afterwards).
 * precision selects the GEMM path (AR_PREC_FP32 / AR_PREC_BF16). */
int32_t ar_muon_step(ar_stream_t stream, float* params, float* grads, float* momentum_buf, int64_t rows,
                     int64_t cols, double initial_lr, double lr_multiplier, double momentum,
                     double weight_decay, int32_t precision);

/* ---------------- model.mojo init ---------------- */

/* model.mojo:86-115  xorshift + Box-Muller N(0, std) */
int32_t ar_fill_normal(ar_stream_t stream, float* output, uint64_t seed_base, float std_, int64_t size);
/* model.mojo:118-134  xorshift U(low, high) (bit-exact: no FMA contraction) */
int32_t ar_fill_uniform(ar_stream_t stream, float* output, uint64_t seed_base, float low, float high,
                        int64_t size);
/* model.mojo:137-145 */
int32_t ar_fill_zeros(ar_stream_t stream, float* output, int64_t size);
/* model.mojo:148-157 */
int32_t ar_fill_value(ar_stream_t stream, float* output, float value, int64_t size);
/* model.mojo:57-81  cos/sin(t / base^(2d/hd)) in f64, stored f32, [seq_len, head_dim/2];
 * computed on the host and copied (synchronously) to the device buffers. */
int32_t ar_precompute_rope(ar_stream_t stream, float* cos_buf, float* sin_buf, int64_t seq_len,
                           int64_t head_dim, double base);

/* ---------------- whole training step (model.mojo / optimizer.mojo / train.mojo) ---------------- */

typedef struct ar_gpt_config {
    int64_t sequence_len, vocab_size, n_layer, n_head, n_kv_head, n_embd, head_dim, kv_dim;
} ar_gpt_config; /* config.mojo:9-24 */

typedef struct ar_gpt ar_gpt;

/* Allocates weights, gradients, optimizer state and activation buffers
 * (ModelWeights, ForwardBuffers, AdamWState, MuonState).  rope_period: 0 =
 * reference table indexing (row = flat token b*T+t; needs B*T <= 2048 like
 * the reference's table), T = per-sequence positions.  precision: AR_PREC_*.
 * Every call on the model is ordered on `stream`; the optimizer step also
 * forks work onto two library-owned streams (default priority) and joins
 * them back into `stream` before it returns control of the ordering, so a
 * caller sees stream-ordered semantics (and a graph capture of `stream`
 * records the fork and join). */
int32_t ar_gpt_create(ar_gpt** out, const ar_gpt_config* cfg, int64_t B, int64_t T, int32_t precision,
                      int64_t rope_period, ar_stream_t stream);
int32_t ar_gpt_destroy(ar_gpt* model);
/* model.mojo:337-427 (seed0 = 42 in the reference) */
int32_t ar_gpt_init_weights(ar_gpt* model, uint64_t seed0);
/* Flat parameter / gradient arenas, tensor order = train.mojo's optimizer
 * registration order: wte, lm_head, resid_lambdas, x0_lambdas, then per layer
 * c_q, c_k, c_v, c_proj, c_fc, mlp_proj[, value_embeds, ve_gate].  With a
 * null model the counts are 0, tensor_info is -1 and the pointers are NULL;
 * the ar_gpt_* entries returning a status answer AR_EINVAL for it
 * (ar_gpt_destroy: AR_OK, nothing to do). */
int64_t ar_gpt_num_tensors(const ar_gpt* model);
int64_t ar_gpt_tensor_info(const ar_gpt* model, int64_t i, int64_t* offset, const char** name);
int64_t ar_gpt_num_params(const ar_gpt* model);
float* ar_gpt_params(ar_gpt* model);
float* ar_gpt_grads(ar_gpt* model);
/* per-token loss [B*T] and mean loss [1] of the last forward (device) */
float* ar_gpt_token_loss(ar_gpt* model);
float* ar_gpt_mean_loss(ar_gpt* model);
/* model.mojo:777-814 */
int32_t ar_gpt_zero_grads(ar_gpt* model);
/* model.mojo:576-772.  inputs/targets: device int64 [B*T].  If loss_host is
 * non-NULL the call synchronises and stores the mean loss there. */
int32_t ar_gpt_forward(ar_gpt* model, const int64_t* inputs, const int64_t* targets, float* loss_host);
/* model.mojo:819-1037 (quirks of the reference backward reproduced) */
int32_t ar_gpt_backward(ar_gpt* model, const int64_t* inputs, const int64_t* targets, float loss_scale);
/* train.mojo:246-281: AdamW groups then Muon on all 2-D matrices */
int32_t ar_gpt_optimizer_step(ar_gpt* model, double progress);
/* train.mojo:231-282: zero_grads -> forward -> backward(1.0) -> optimizer */
int32_t ar_gpt_train_step(ar_gpt* model, const int64_t* inputs, const int64_t* targets, double progress,
                          float* loss_host);
/* ar_gpt_train_step replayed from a HIP graph (the "HIP-graph capture of the
 * whole step" of the training driver; no counterpart in the reference, whose
 * step is ~1,700 separate launches).  Same results as ar_gpt_train_step,
 * bit for bit.  The graph records inputs / targets: pass the same device
 * buffers every call (new pointers re-record it); the token-id sort of the
 * embedding backward is part of the graph.  The model's stream
 * must not be the null stream, and profiling (ar_gpt_profile) must be off.
 * loss_host as in ar_gpt_train_step. */
int32_t ar_gpt_train_step_graph(ar_gpt* model, const int64_t* inputs, const int64_t* targets, double progress,
                                float* loss_host);

/* Per-kernel-class timing of the step (no counterpart in the reference: the
 * measurement hook behind bench.py's roofline figure).  When enabled, every
 * GEMM / attention launch of the step is bracketed by HIP events on the
 * model's stream.  Classes: 0 linear_fwd, 1 linear_bwd_dx, 2 linear_bwd_dw,
 * 3 flash_attn_fwd, 4 flash_attn_bwd_dq, 5 flash_attn_bwd_dkv, 6 muon GEMMs. */
enum ar_prof_class { AR_PROF_NCLASS = 7 };
int32_t ar_gpt_profile(ar_gpt* model, int32_t enable);
/* Synchronises; sums elapsed time (ms), launch count and algorithmic FLOPs of
 * class `cls` since profiling was enabled. */
int32_t ar_gpt_profile_read(ar_gpt* model, int32_t cls, double* ms, int64_t* launches, double* flops);

#ifdef __cplusplus
}
#endif
#endif /* AR_OPS_H */
