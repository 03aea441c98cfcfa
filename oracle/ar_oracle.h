/*
 * ar_oracle.h -- CPU restatement of the autoresearch GPT training step.
 *
 * TEST INFRASTRUCTURE ONLY.  This oracle is the parity checker for the HIP
 * library in autoresearch_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function restates one kernel or host routine of the Mojo reference
 * (sergeytimoshin/autoresearch) and cites the file:line it follows.  Argument
 * order is the reference kernel's argument order.  Element arithmetic is
 * fp32 at the points where the reference stores fp32; long sums (GEMM inner
 * products, row reductions, attention dot products) accumulate in double and
 * round once, so the oracle sits within fp32 rounding of every summation
 * order the GPU may choose.  Built with -ffp-contract=off: no FMA contraction.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   embedding fwd/bwd      KAT test_kernels.mojo:20-64, brute force
 *   rmsnorm fwd/bwd        KAT test_kernels.mojo:140-181, torch fp64 autograd
 *   linear fwd/dx/dw       numpy fp64 matmul
 *   rope fwd/bwd           closed form, bwd∘fwd = id, norm preservation
 *   flash attention        torch fp64 masked softmax attention + autograd
 *   relu², softcap         KAT test_kernels.mojo:67-137, torch autograd
 *   cross entropy          KAT test_kernels.mojo:227-267, torch fp64
 *   ce+softcap bwd         code text only (Q4: not an autograd gradient) plus
 *                          torch softmax − onehot of the capped logits
 *   ve gate/apply fwd/bwd  torch fp64 autograd
 *   residual kernels       closed forms
 *   adamw                  torch.optim.AdamW (fp64)
 *   muon                   polar-express singular-value invariant, fp64 numpy
 *   init kernels           integer restatement; uniform checked bit-exact
 *                          against an independent numpy uint64 restatement
 *   whole step             behavioural invariants of test_forward.mojo and
 *                          test_backward.mojo, finite differences of the loss
 */
#ifndef AR_ORACLE_H
#define AR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernels/ops.mojo ---------------------------------------------------- */
void orc_embedding_fwd(float* out, const float* weight, const int64_t* idx, int64_t num_tokens, int64_t dim);
void orc_rmsnorm_fwd(float* out, float* rms_out, const float* in, int64_t rows, int64_t dim);
void orc_linear_fwd(float* out, const float* in, const float* w, int64_t M, int64_t N, int64_t K);
void orc_rope_fwd(float* out, const float* in, const float* cos_t, const float* sin_t,
                  int64_t num_tokens, int64_t num_heads, int64_t head_dim);
void orc_flash_attn_fwd(float* out, float* lse, const float* q, const float* k, const float* v,
                        int64_t B, int64_t T, int64_t H, int64_t hd, int64_t window);
void orc_flash_attn_bwd_precompute_d(float* d, const float* out, const float* dout,
                                     int64_t B, int64_t T, int64_t H, int64_t hd);
void orc_flash_attn_bwd_dq(float* dq, const float* q, const float* k, const float* v,
                           const float* dout, const float* lse, const float* d,
                           int64_t B, int64_t T, int64_t H, int64_t hd, int64_t window);
void orc_flash_attn_bwd_dkv(float* dk, float* dv, const float* q, const float* k, const float* v,
                            const float* dout, const float* lse, const float* d,
                            int64_t B, int64_t T, int64_t H, int64_t hd, int64_t window);
void orc_relu_squared_fwd(float* out, const float* in, int64_t size);
void orc_softcap_fwd(float* out, const float* in, float cap, int64_t size);
void orc_ve_gate_fwd(float* gate, const float* xn, const float* w, int64_t num_tokens,
                     int64_t n_kv_head, int64_t gate_channels, int64_t embd_dim);
void orc_ve_apply_fwd(float* v, const float* gate, const float* ve, int64_t num_tokens,
                      int64_t n_kv_head, int64_t head_dim);
void orc_add_residual_fwd(float* out, const float* res, const float* in, int64_t size);
void orc_scaled_add_fwd(float* out, const float* a, const float* b, const float* sa,
                        const float* sb, int64_t idx, int64_t size);
void orc_cross_entropy_fwd(float* loss, const float* logits, const int64_t* targets,
                           int64_t num_tokens, int64_t V);
void orc_mean_reduce(float* out, const float* in, int64_t size);
void orc_cross_entropy_softcap_bwd(float* grad, const float* logits, const int64_t* targets,
                                   float cap, int64_t num_tokens, int64_t V, float loss_scale);
void orc_linear_bwd_dx(float* dx, const float* dy, const float* w, int64_t M, int64_t N, int64_t K);
void orc_linear_bwd_dw(float* dw, const float* dy, const float* x, int64_t M, int64_t N, int64_t K);
void orc_rmsnorm_bwd(float* dx, const float* dy, const float* x, const float* rms, int64_t rows, int64_t dim);
void orc_rope_bwd(float* dx, const float* dy, const float* cos_t, const float* sin_t,
                  int64_t num_tokens, int64_t num_heads, int64_t head_dim);
void orc_relu_squared_bwd(float* dx, const float* dy, const float* x, int64_t size);
void orc_embedding_bwd(float* gw, const float* dy, const int64_t* idx, int64_t num_tokens, int64_t dim);
void orc_scaled_add_bwd(float* ga, float* gb, const float* g, const float* sa, const float* sb,
                        int64_t idx, int64_t size);
void orc_ve_apply_bwd(float* gve, float* ggate, const float* gv, const float* gate, const float* ve,
                      int64_t num_tokens, int64_t n_kv_head, int64_t head_dim);
void orc_ve_gate_bwd(float* gxn, float* gw, const float* ggate, const float* gate, const float* xn,
                     const float* w, int64_t num_tokens, int64_t n_kv_head, int64_t gate_channels,
                     int64_t embd_dim);
void orc_scalar_grad_reduce(float* gs, const float* g, const float* x, int64_t idx, int64_t size);
void orc_zero_buffer(float* buf, int64_t size);

/* ---- optimizer.mojo ------------------------------------------------------ */
void orc_adamw(float* p, const float* g, float* m, float* v, float lr, float b1, float b2, float eps,
               float wd, float bc1, float bc2, int64_t size);
void orc_nesterov_momentum(float* out, const float* g, float* buf, float mu, int64_t size);
void orc_normalize_frobenius(float* x, int64_t size);
void orc_scale_add(float* out, const float* a, const float* b, float sa, float sb, int64_t size);
void orc_muon_update(float* p, const float* g, float lr, float wd, int64_t size);
/* MuonState.step for one matrix; grads is clobbered like the reference's. */
void orc_muon_step(float* param, float* grads, float* momentum_buf, int64_t rows, int64_t cols,
                   double initial_lr, double lrm, double momentum, double wd);

/* ---- model.mojo init ----------------------------------------------------- */
void orc_fill_normal(float* out, uint64_t seed, float std_, int64_t size);
void orc_fill_uniform(float* out, uint64_t seed, float lo, float hi, int64_t size);
void orc_fill_zeros(float* out, int64_t size);
void orc_fill_value(float* out, float value, int64_t size);
void orc_precompute_rope(float* cos_t, float* sin_t, int64_t seq_len, int64_t head_dim, double base);

/* ---- whole model (model.mojo, optimizer.mojo, train.mojo) ---------------- */
typedef struct orc_config {
    int64_t sequence_len, vocab_size, n_layer, n_head, n_kv_head, n_embd, head_dim, kv_dim;
} orc_config;

typedef struct orc_model orc_model;

/* rope_period: 0 = reference table indexing (row = flat token b*T+t, needs
 * B*T <= table rows), otherwise row = flat token % rope_period. */
orc_model* orc_model_create(const orc_config* cfg, int64_t B, int64_t T, int64_t rope_period);
void orc_model_destroy(orc_model* m);
void orc_model_init_weights(orc_model* m, uint64_t seed0);
/* Parameters/gradients/optimizer state are one flat arena each, in the
 * tensor order listed by orc_model_tensor_info(). */
int64_t orc_model_num_tensors(const orc_model* m);
int64_t orc_model_tensor_info(const orc_model* m, int64_t i, int64_t* offset, const char** name);
int64_t orc_model_num_params(const orc_model* m);
float* orc_model_params(orc_model* m);
float* orc_model_grads(orc_model* m);
void orc_model_zero_grads(orc_model* m);
float orc_model_forward(orc_model* m, const int64_t* inputs, const int64_t* targets);
void orc_model_backward(orc_model* m, const int64_t* inputs, const int64_t* targets, float loss_scale);
/* AdamW groups then Muon, as train.mojo:246-281 (progress given by caller). */
void orc_model_optimizer_step(orc_model* m, double progress);
/* zero_grads -> forward -> backward(loss_scale 1) -> optimizer; returns loss */
float orc_model_train_step(orc_model* m, const int64_t* inputs, const int64_t* targets, double progress);
/* per-token loss of the last forward, [B*T] */
const float* orc_model_token_loss(const orc_model* m);
int64_t orc_model_adam_step(const orc_model* m);
/* sum_i |g_i x_i| of each layer's resid_lambdas / x0_lambdas gradient sum in
 * the last backward: the scale of their rounding sensitivity */
void orc_model_scalar_grad_l1(const orc_model* m, double* res, double* x0);
/* Saved activations by name ("q","k","v","attn_out","lse" per layer;
 * "grad_attn_out","grad_q" = last layer processed by backward). */
float* orc_model_buffer(orc_model* m, const char* name, int64_t layer);

int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
