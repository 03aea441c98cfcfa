// ar_model.hip -- the whole training step: a C++ restatement of the Mojo
// host code (model.mojo ModelWeights / ForwardBuffers / forward / backward /
// zero_grads, optimizer.mojo AdamWState / MuonState, train.mojo's step body)
// sequencing the gfx950 kernels of this library.
//
// Differences from the reference's host code, none of which change results:
//   * activations are produced directly into their per-layer saved buffers,
//     so the reference's device-to-device "save" copies disappear
//     (model.mojo:618, 632, 640, 659-660, 689-691, 700-701, 717, 721, 727,
//     738, 743, 873, 903);
//   * c_proj dX is written to its own buffer instead of in place
//     (model.mojo:906), which is the read-all-then-write semantics;
//   * the token-id sort used by the deterministic embedding scatter is done
//     once per backward and shared by the wte and value-embedding scatters;
//   * all reductions are deterministic (fixed order, no float atomics).
//
// Precision AR_PREC_BF16 runs the bf16 step (forward_bf16 / backward_bf16):
// GEMM and attention operands are stored as bf16 (a bf16 shadow of the
// weights is refreshed at every forward), c_q / c_k / c_v run as one
// [3C, C] GEMM (they are adjacent in the parameter arena), the residual add,
// ReLU^2 and softcap are GEMM epilogues and the remaining element-wise steps
// are the fused row kernels of ar_fused.hip.  The reference's operation order
// and quirks are kept; only where each bf16 rounding happens moves (to the
// producer instead of each consumer).
#include <math.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "ar_internal.hpp"

using namespace ar;

namespace {

constexpr int64_t kGateChannels = 32;  // config.mojo:64
constexpr int64_t kMlpExpansion = 4;   // config.mojo:63
constexpr float kSoftcap = 15.0f;      // config.mojo:86

struct Tensor {
    int64_t offset, size, rows, cols;
    std::string name;
};

struct LayerBufs {
    float *x, *xn_attn, *q, *k, *v, *lse, *attn_out, *xn_mlp, *mlp_hidden, *mlp_act, *rms_attn, *rms_mlp, *ve, *gate;
};

// Saved activations of one layer in the bf16 step.
struct LayerBufsB {
    float *x, *lse, *attn_out, *rms_attn, *rms_mlp, *gate, *xg;
    ar::bf16 *xn, *q, *k, *v, *attn_out_b, *xn_mlp, *act;
};

}  // namespace

struct ar_gpt {
    ar_gpt_config c;
    int64_t B, T, BT, period;
    bool bf16;
    hipStream_t st;
    std::vector<Tensor> t;
    int64_t nparams = 0;
    float *params = nullptr, *grads = nullptr, *adam_m = nullptr, *adam_v = nullptr, *muon_buf = nullptr;
    int64_t i_wte, i_lm, i_res, i_x0;
    std::vector<int64_t> i_q, i_k, i_v, i_proj, i_fc, i_mlpp, i_ve, i_gate;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    int64_t rope_rows = 0;
    // activations
    float *x0, *x, *rms_qk, *logits, *loss, *mean_loss, *x_final, *rms_final, *d_buf;
    std::vector<LayerBufs> L;
    // gradients of activations
    float *grad_x, *grad_x0, *grad_logits, *grad_attn_out, *grad_q, *grad_k, *grad_v, *grad_x_norm, *grad_tmp,
        *grad_mlp, *grad_ve, *grad_gate;
    // bf16 step
    ar::bf16* wb = nullptr;  // bf16 shadow of the parameter arena (same offsets)
    // bf16 transposes of the matrices the backward multiplies by (W^T at W's
    // offset): dX = dY . W runs as an NT product with both operands K-major.
    ar::bf16* wbt = nullptr;
    ar::TransposeEntry* wbt_tab = nullptr;
    int wbt_n = 0;
    int64_t wbt_tiles = 0;
    std::vector<LayerBufsB> LB;
    ar::bf16* qkv = nullptr;  // [BT, 3C] q | k | v GEMM output
    ar::bf16 *x_final_b = nullptr, *grad_logits_b = nullptr, *grad_xb = nullptr, *grad_x_norm_b = nullptr,
             *grad_h = nullptr, *grad_attn_out_b = nullptr, *grad_qkv = nullptr;
    // bf16 dS tiles of one layer's attention backward (written by the dK / dV
    // kernel, read by the dQ product)
    ar::bf16* ds_buf = nullptr;
    // qkv_post fused into the q|k|v product and D = rowsum(dO O) into the
    // c_proj dX product (head-aligned persistent GEMM), when the shape allows
    bool fuse_heads = false;
    // the forward's residual products (c_proj, mlp_proj) as row-complete
    // GEMMs that also run the following resid_norm pass (C = 512)
    bool fuse_rows = false;
    float grad_logits_scale = 0.f;  // loss_scale baked into grad_logits_b
    bool grad_logits_valid = false;
    // step-dependent optimizer scalars in device memory (StepScalars)
    float* dsc = nullptr;
    // graph replay of the step (ar_gpt_train_step_graph)
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    // Muon's three shape groups (square, c_fc, mlp_proj) are independent:
    // the c_fc and mlp_proj groups run on two side streams (default
    // priority) forked from and joined back into st, each with its own
    // region of scratch starting at muon_off[group].
    hipStream_t side[2] = {nullptr, nullptr};
    hipEvent_t fork_ev = nullptr, join_ev[2] = {nullptr, nullptr};
    int64_t muon_off[3] = {0, 0, 0};
    hipGraphNode_t graph_scalars = nullptr;
    const int64_t *graph_in = nullptr, *graph_tg = nullptr;
    // scratch (sequential users on one stream)
    float* scratch = nullptr;
    int64_t scratch_elems = 0;
    uint32_t* sorted_ids = nullptr;
    int32_t* sorted_tok = nullptr;
    void* sort_scratch = nullptr;
    size_t sort_bytes = 0;
    int32_t sort_bits = 32;
    int64_t adam_step = 0;
    std::vector<void*> allocs;
    // profiling (ar_gpt_profile)
    bool prof = false;
    std::vector<hipEvent_t> ev;
    struct Rec { int cls; double flops; int e0, e1; };
    std::vector<Rec> recs;
    size_t ev_used = 0;
};

namespace {

// Largest attention-backward dS workspace the bf16 step allocates (4 GiB:
// BASELINE config 5 takes 3.2 GB).
constexpr int64_t kDsMaxBytes = int64_t(4) << 30;

bool has_ve(const ar_gpt_config& c, int64_t i) { return (i % 2) == ((c.n_layer - 1) % 2); }  // config.mojo:45-47
int64_t window_size(const ar_gpt_config& c, int64_t i) {                                      // config.mojo:49-55
    if (i == c.n_layer - 1) return c.sequence_len;
    if (i % 4 < 3) return c.sequence_len / 2;
    return c.sequence_len;
}

int32_t dalloc(ar_gpt* m, void** p, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (hipMalloc(p, bytes) != hipSuccess) return set_error(AR_ENOMEM, "gpt: hipMalloc(%zu) failed", bytes);
    m->allocs.push_back(*p);
    return AR_OK;
}
#define AR_TRY(expr)                      \
    do {                                  \
        int32_t _r = (expr);              \
        if (_r != AR_OK) return _r;       \
    } while (0)
#define FALLOC(ptr, n) AR_TRY(dalloc(m, (void**)&(ptr), (size_t)(n) * sizeof(float)))

int64_t add_tensor(ar_gpt* m, int64_t rows, int64_t cols, const std::string& nm) {
    Tensor t{m->nparams, rows * cols, rows, cols, nm};
    m->t.push_back(t);
    m->nparams += (rows * cols + 63) & ~int64_t(63);  // 256-byte aligned tensors
    return (int64_t)m->t.size() - 1;
}

inline float* P(ar_gpt* m, int64_t i) { return m->params + m->t[i].offset; }
inline float* G(ar_gpt* m, int64_t i) { return m->grads + m->t[i].offset; }
inline const bf16* Wb(ar_gpt* m, int64_t i) { return m->wb + m->t[i].offset; }
inline const bf16* WbT(ar_gpt* m, int64_t i) { return m->wbt + m->t[i].offset; }
// the bf16 step's logits: bf16 values in the first half of the fp32 logits buffer
inline bf16* LogitsB(ar_gpt* m) { return reinterpret_cast<bf16*>(m->logits); }

inline ar_stream_t AS(ar_gpt* m) { return reinterpret_cast<ar_stream_t>(m->st); }

// Profiling brackets (no-ops unless ar_gpt_profile enabled them).
int32_t prof_reserve(ar_gpt* m, size_t n) {
    while (m->ev.size() < n) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return set_error(AR_EHIP, "gpt_profile: event create failed");
        m->ev.push_back(e);
    }
    return AR_OK;
}
int prof_begin(ar_gpt* m) {
    if (!m->prof) return -1;
    if (m->ev_used + 2 > m->ev.size() && prof_reserve(m, m->ev.size() + 1024) != AR_OK) return -1;
    const int e0 = (int)m->ev_used;
    m->ev_used += 2;
    hipEventRecord(m->ev[e0], m->st);
    return e0;
}
void prof_end(ar_gpt* m, int e0, int cls, double flops) {
    if (e0 < 0) return;
    hipEventRecord(m->ev[e0 + 1], m->st);
    m->recs.push_back({cls, flops, e0, e0 + 1});
}

int32_t linear(ar_gpt* m, float* out, const float* in, const float* w, int64_t M, int64_t N, int64_t K) {
    const int e = prof_begin(m);
    const int32_t r = gemm_f32(m->st, 0, m->bf16, out, in, w, M, N, K, false, 1, nullptr);
    prof_end(m, e, 0, 2.0 * M * N * K);
    return r;
}
// out = r + in @ w^T (r may alias out): the residual add in the product's epilogue, the same fp32 add
int32_t linear_add(ar_gpt* m, float* out, const float* in, const float* w, const float* r, int64_t M, int64_t N,
                   int64_t K) {
    const int e = prof_begin(m);
    const int32_t rc = gemm_f32_add(m->st, m->bf16, out, in, w, r, M, N, K);
    prof_end(m, e, 0, 2.0 * M * N * K);
    return rc;
}
int32_t linear_dx(ar_gpt* m, float* dx, const float* dy, const float* w, int64_t M, int64_t N, int64_t K) {
    const int e = prof_begin(m);
    const int32_t r = gemm_f32(m->st, 1, m->bf16, dx, dy, w, M, N, K, false, 1, nullptr);
    prof_end(m, e, 1, 2.0 * M * N * K);
    return r;
}
int32_t linear_dw(ar_gpt* m, float* dw, const float* dy, const float* x, int64_t M, int64_t N, int64_t K) {
    const int e = prof_begin(m);
    const int32_t r = gemm_f32(m->st, 2, m->bf16, dw, dy, x, M, N, K, true, 0, m->scratch);
    prof_end(m, e, 2, 2.0 * M * N * K);
    return r;
}
// Algorithmic attention FLOPs of one call: forward 4*B*H*hd*sum_q keys(q),
// dQ 3x that (S, dP, dQ products), dK/dV 4x (S, dP, dV, dK).
double attn_keys(const ar_gpt* m, int64_t ws) {
    const int64_t T = m->T;
    double keys = 0;
    for (int64_t q = 0; q < T; ++q) {
        const int64_t k0 = (ws > 0 && q - ws > 0) ? q - ws : 0;
        keys += (double)(q - k0 + 1);
    }
    return keys;
}
void attn_prof_end(ar_gpt* m, int e, AttnOp op, int64_t ws) {
    if (e < 0) return;
    const ar_gpt_config& c = m->c;
    const double unit = 2.0 * m->B * c.n_head * c.head_dim * attn_keys(m, ws);
    const int cls = op == AttnOp::FWD ? 3 : (op == AttnOp::DQ ? 4 : 5);
    prof_end(m, e, cls, unit * (op == AttnOp::FWD ? 2.0 : (op == AttnOp::DQ ? 3.0 : 4.0)));
}
int32_t attention(ar_gpt* m, AttnOp op, float* o1, float* o2, const float* q, const float* k, const float* v,
                  const float* dout, const float* lse, const float* dbuf, int64_t ws) {
    const int e = prof_begin(m);
    const int32_t r = attn_dispatch<false, float>(m->st, op, o1, o2, q, k, v, dout, lse, dbuf, m->B, m->T,
                                                  m->c.n_head, m->c.head_dim, ws);
    attn_prof_end(m, e, op, ws);
    return r;
}
int32_t attention_b(ar_gpt* m, AttnOp op, float* o1, float* o2, const FlashOut& fo, const bf16* q,
                    const bf16* k, const bf16* v, const bf16* dout, const float* lse, const float* dbuf, int64_t ws) {
    const int e = prof_begin(m);
    const int32_t r = flash_attn_bf16(m->st, op, o1, o2, fo, q, k, v, dout, lse, dbuf, m->B, m->T, m->c.n_head,
                                      m->c.head_dim, ws);
    attn_prof_end(m, e, op, ws);
    return r;
}
// dQ from the dS tiles of the preceding DKV launch (profiling class
// flash_attn_bwd_dq, one product: 2 B H hd keys flops).
int32_t attention_dq_ds(ar_gpt* m, const FlashOut& fo, const bf16* k, int64_t ws) {
    const int e = prof_begin(m);
    const int32_t r = flash_dq_ds_bf16(m->st, fo, k, m->ds_buf, m->B, m->T, m->c.n_head, m->c.head_dim, ws);
    prof_end(m, e, 4, 2.0 * m->B * m->c.n_head * m->c.head_dim * attn_keys(m, ws));
    return r;
}
// bf16-step GEMMs (operand storage per flag; profiling class cls).
int32_t gemm_b(ar_gpt* m, int cls, int layout, void* C, bool cb, const void* X, bool xb, const void* W, bool wb,
               int64_t M, int64_t N, int64_t K, bool accumulate) {
    const int e = prof_begin(m);
    const int32_t r = gemm_bf16io(m->st, layout, C, cb, X, xb, W, wb, M, N, K, accumulate, layout == 2 ? 0 : 1,
                                  m->scratch);
    prof_end(m, e, cls, 2.0 * M * N * K);
    return r;
}
int32_t gemm_e(ar_gpt* m, int cls, int layout, int epi, void* C, bool cb, const void* X, bool xb, const bf16* W,
               int64_t M, int64_t N, int64_t K, const void* aux, void* aux_out, float cap) {
    const int e = prof_begin(m);
    const int32_t r = gemm_epilogue(m->st, layout, epi, C, cb, X, xb, W, 1, M, N, K, aux, aux_out, cap);
    prof_end(m, e, cls, 2.0 * M * N * K);
    return r;
}
int32_t rope_model(ar_gpt* m, float* x, bool inverse) {
    return rope(m->st, x, x, m->rope_cos, m->rope_sin, m->BT, m->c.n_head, m->c.head_dim, m->period, inverse);
}

}  // namespace

// ------------------------------------------------------------------------
// creation (model.mojo:263-335, 495-571; optimizer.mojo:86-101, 242-253)
// ------------------------------------------------------------------------

static int32_t gpt_build(ar_gpt* m) {
    const ar_gpt_config& c = m->c;
    const int64_t C = c.n_embd, V = c.vocab_size, Lr = c.n_layer, kv = c.kv_dim, F = kMlpExpansion * C;
    const int64_t BT = m->BT, H = c.n_head, hd = c.head_dim;
    // Tensor order = train.mojo's optimizer registration order.
    m->i_wte = add_tensor(m, V, C, "wte");
    m->i_lm = add_tensor(m, V, C, "lm_head");
    m->i_res = add_tensor(m, 1, Lr, "resid_lambdas");
    m->i_x0 = add_tensor(m, 1, Lr, "x0_lambdas");
    for (int64_t i = 0; i < Lr; ++i) {
        const std::string p = "h" + std::to_string(i) + ".";
        m->i_q.push_back(add_tensor(m, C, C, p + "c_q"));
        m->i_k.push_back(add_tensor(m, kv, C, p + "c_k"));
        m->i_v.push_back(add_tensor(m, kv, C, p + "c_v"));
        m->i_proj.push_back(add_tensor(m, C, C, p + "c_proj"));
        m->i_fc.push_back(add_tensor(m, F, C, p + "c_fc"));
        m->i_mlpp.push_back(add_tensor(m, C, F, p + "mlp_proj"));
        if (has_ve(c, i)) {
            m->i_ve.push_back(add_tensor(m, V, kv, p + "value_embeds"));
            m->i_gate.push_back(add_tensor(m, c.n_kv_head, kGateChannels, p + "ve_gate"));
        } else {
            m->i_ve.push_back(-1);
            m->i_gate.push_back(-1);
        }
    }
    FALLOC(m->params, m->nparams);
    FALLOC(m->grads, m->nparams);
    FALLOC(m->adam_m, m->nparams);
    FALLOC(m->adam_v, m->nparams);
    FALLOC(m->muon_buf, m->nparams);
    AR_TRY(ar_zero_buffer(AS(m), m->adam_m, m->nparams));
    AR_TRY(ar_zero_buffer(AS(m), m->adam_v, m->nparams));
    AR_TRY(ar_zero_buffer(AS(m), m->muon_buf, m->nparams));
    AR_TRY(ar_zero_buffer(AS(m), m->params, m->nparams));
    AR_TRY(ar_zero_buffer(AS(m), m->grads, m->nparams));

    const int64_t half = hd / 2;
    m->rope_rows = m->period > 2048 ? m->period : 2048;  // MAX_SEQ_LEN rows (model.mojo:307)
    FALLOC(m->rope_cos, m->rope_rows * half);
    FALLOC(m->rope_sin, m->rope_rows * half);

    // shared by both steps
    FALLOC(m->x0, BT * C);
    FALLOC(m->x, BT * C);
    FALLOC(m->logits, BT * V);
    FALLOC(m->loss, BT);
    FALLOC(m->mean_loss, 64);
    FALLOC(m->dsc, 64);
    FALLOC(m->rms_final, BT);
    FALLOC(m->d_buf, BT * H);
    FALLOC(m->grad_x, BT * C);
    FALLOC(m->grad_x_norm, BT * C);
    FALLOC(m->grad_ve, BT * kv);
    FALLOC(m->grad_gate, BT * H);
    auto balloc = [&](bf16** p, int64_t n) { return dalloc(m, (void**)p, (size_t)n * sizeof(bf16)); };
    if (m->bf16) {
        AR_TRY(balloc(&m->wb, m->nparams));
        m->LB.resize(Lr);
        for (int64_t i = 0; i < Lr; ++i) {
            LayerBufsB& b = m->LB[i];
            FALLOC(b.x, BT * C);
            FALLOC(b.lse, BT * H);
            FALLOC(b.attn_out, BT * C);
            FALLOC(b.rms_attn, BT);
            FALLOC(b.rms_mlp, BT);
            AR_TRY(balloc(&b.xn, BT * C));
            AR_TRY(balloc(&b.q, BT * C));
            AR_TRY(balloc(&b.k, BT * kv));
            AR_TRY(balloc(&b.v, BT * kv));
            AR_TRY(balloc(&b.attn_out_b, BT * C));
            AR_TRY(balloc(&b.xn_mlp, BT * C));
            AR_TRY(balloc(&b.act, BT * F));
            if (has_ve(c, i)) {
                FALLOC(b.gate, BT * H);
                FALLOC(b.xg, BT * kGateChannels);
            } else {
                b.gate = b.xg = nullptr;
            }
        }
        // transposed shadows: fused [3C, C] c_q|c_k|c_v, c_proj, c_fc, mlp_proj, lm_head
        AR_TRY(balloc(&m->wbt, m->nparams));
        std::vector<TransposeEntry> tab;
        auto add_t = [&](int64_t idx, int64_t rows, int64_t cols) {
            const int64_t off = m->t[idx].offset;
            const int64_t t0 = tab.empty() ? 0 : tab.back().tile0 + cdiv(tab.back().rows, 64) * cdiv(tab.back().cols, 64);
            tab.push_back(TransposeEntry{off, off, rows, cols, t0});
        };
        for (int64_t i = 0; i < Lr; ++i) {
            add_t(m->i_q[i], 3 * C, C);
            add_t(m->i_proj[i], C, C);
            add_t(m->i_fc[i], F, C);
            add_t(m->i_mlpp[i], C, F);
        }
        add_t(m->i_lm, V, C);
        m->wbt_n = (int)tab.size();
        m->wbt_tiles = tab.back().tile0 + cdiv(tab.back().rows, 64) * cdiv(tab.back().cols, 64);
        AR_TRY(dalloc(m, (void**)&m->wbt_tab, tab.size() * sizeof(TransposeEntry)));
        if (hipMemcpy(m->wbt_tab, tab.data(), tab.size() * sizeof(TransposeEntry), hipMemcpyHostToDevice) !=
            hipSuccess)
            return set_error(AR_EHIP, "gpt: transpose table upload failed");
        AR_TRY(balloc(&m->qkv, BT * 3 * C));
        AR_TRY(balloc(&m->x_final_b, BT * C));
        AR_TRY(balloc(&m->grad_logits_b, BT * V));
        AR_TRY(balloc(&m->grad_xb, BT * C));
        AR_TRY(balloc(&m->grad_x_norm_b, BT * C));
        AR_TRY(balloc(&m->grad_h, BT * F));
        AR_TRY(balloc(&m->grad_attn_out_b, BT * C));
        AR_TRY(balloc(&m->grad_qkv, BT * 3 * C));
        // The dS workspace grows with T^2; past kDsMaxBytes (or the
        // AR_ATTN_DS_MAX_BYTES override) the step keeps the dQ kernel that
        // recomputes S and dP instead.
        // If the allocation fails the step also takes the recomputing path.
        int64_t ds_max = kDsMaxBytes;
        if (const char* e = getenv("AR_ATTN_DS_MAX_BYTES")) {
            char* end = nullptr;
            ds_max = strtoll(e, &end, 10);
            if (end == e || *end != '\0' || ds_max < 0)
                return set_error(AR_EINVAL, "gpt: AR_ATTN_DS_MAX_BYTES='%s' is not a non-negative byte count", e);
        }
        // AR_FUSE_HEADS=0 keeps the separate qkv_post / D kernels (A/B runs, tests)
        const char* fh = getenv("AR_FUSE_HEADS");
        m->fuse_heads = !(fh && strcmp(fh, "0") == 0) && gemm_head_fusable(BT, C, hd);
        // AR_FUSE_ROWS=0 keeps the residual-add GEMMs and separate resid_norm passes
        const char* fr = getenv("AR_FUSE_ROWS");
        m->fuse_rows = !(fr && strcmp(fr, "0") == 0) && gemm_rc_fusable(BT, C, C) && gemm_rc_fusable(BT, C, F) &&
                       kGateChannels == 32;
        const int64_t ds_elems = flash_ds_elems(m->B, m->T, H);
        if (ds_elems * (int64_t)sizeof(bf16) <= ds_max) {
            void* p = nullptr;
            if (hipMalloc(&p, (size_t)ds_elems * sizeof(bf16)) == hipSuccess) {
                m->allocs.push_back(p);
                m->ds_buf = (bf16*)p;
            } else {
                (void)hipGetLastError();  // clear the failed allocation's error; ds_buf stays null
            }
        }
    } else {
        FALLOC(m->rms_qk, BT * H);
        FALLOC(m->x_final, BT * C);
        m->L.resize(Lr);
        for (int64_t i = 0; i < Lr; ++i) {
            LayerBufs& b = m->L[i];
            FALLOC(b.x, BT * C);
            FALLOC(b.xn_attn, BT * C);
            FALLOC(b.q, BT * C);
            FALLOC(b.k, BT * kv);
            FALLOC(b.v, BT * kv);
            FALLOC(b.lse, BT * H);
            FALLOC(b.attn_out, BT * C);
            FALLOC(b.xn_mlp, BT * C);
            FALLOC(b.mlp_hidden, BT * F);
            FALLOC(b.mlp_act, BT * F);
            FALLOC(b.rms_attn, BT);
            FALLOC(b.rms_mlp, BT);
            if (has_ve(c, i)) {
                FALLOC(b.ve, BT * kv);
                FALLOC(b.gate, BT * H);
            } else {
                b.ve = b.gate = nullptr;
            }
        }
        FALLOC(m->grad_q, BT * C);
        FALLOC(m->grad_k, BT * kv);
        FALLOC(m->grad_v, BT * kv);
        FALLOC(m->grad_x0, BT * C);
        FALLOC(m->grad_logits, BT * V);
        FALLOC(m->grad_attn_out, BT * C);
        FALLOC(m->grad_tmp, BT * C);
        FALLOC(m->grad_mlp, BT * F);
    }

    // Scratch: the largest of every sequential user.
    int64_t need = kSumBlocks + 64;
    auto upd = [&](int64_t n) { if (n > need) need = n; };
    const int64_t dw_shapes[][2] = {{C, C}, {kv, C}, {F, C}, {C, F}, {V, C}, {3 * C, C}};
    for (auto& s : dw_shapes)
        upd(gemm_partial_elems(2, BT, s[0], s[1], gemm_auto_splits(2, m->bf16, m->bf16, BT, s[0], s[1])));
    const int64_t groups = (4 * Lr + kMuonMaxGroup - 1) / kMuonMaxGroup;
    const int64_t sq = (4 * Lr + groups - 1) / groups;  // square matrices per launch group
    // the three Muon shape groups run concurrently: disjoint scratch regions
    const int64_t lg = Lr < kMuonMaxGroup ? Lr : kMuonMaxGroup;
    // (each size is a whole number of 64-float blocks)
    m->muon_off[1] = muon_scratch_elems(C, C, m->bf16, sq);
    m->muon_off[2] = m->muon_off[1] + muon_scratch_elems(F, C, m->bf16, lg);
    upd(m->muon_off[2] + muon_scratch_elems(C, F, m->bf16, lg));
    upd(BT * (C > kv ? C : kv));                  // embedding scatter partials
    upd((int64_t)kGateBlocks * H * kGateChannels);  // ve gate partials
    upd(2 * (int64_t)kNormBwdWaves);                // learned-scalar gradient partials
    m->scratch_elems = need;
    FALLOC(m->scratch, need);
    for (int i = 0; i < 2; ++i) {
        if (hipStreamCreateWithFlags(&m->side[i], hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&m->join_ev[i], hipEventDisableTiming) != hipSuccess)
            return set_error(AR_EHIP, "gpt_create: side stream / event");
    }
    if (hipEventCreateWithFlags(&m->fork_ev, hipEventDisableTiming) != hipSuccess)
        return set_error(AR_EHIP, "gpt_create: fork event");
    int bits = 1;
    while ((int64_t(1) << bits) < V) ++bits;
    m->sort_bits = bits;
    AR_TRY(dalloc(m, (void**)&m->sorted_ids, (size_t)BT * sizeof(uint32_t)));
    AR_TRY(dalloc(m, (void**)&m->sorted_tok, (size_t)BT * sizeof(int32_t)));
    AR_TRY(ar_embedding_sort(AS(m), nullptr, nullptr, nullptr, BT, m->sort_bits, nullptr, 0, &m->sort_bytes));
    AR_TRY(dalloc(m, &m->sort_scratch, m->sort_bytes));
    return AR_OK;
}

extern "C" int32_t ar_gpt_create(ar_gpt** out, const ar_gpt_config* cfg, int64_t B, int64_t T, int32_t precision,
                                 int64_t rope_period, ar_stream_t stream) {
    AR_CHECK_ARG(out && cfg, "gpt_create: null pointer");
    const ar_gpt_config& c = *cfg;
    AR_CHECK_ARG(B > 0 && T > 0 && c.n_layer > 0 && c.n_head > 0 && c.head_dim > 0 && c.n_embd > 0 &&
                     c.vocab_size > 0,
                 "gpt_create: bad config");
    AR_CHECK_ARG(c.n_head * c.head_dim == c.n_embd && c.kv_dim == c.n_embd && c.n_kv_head == c.n_head,
                 "gpt_create: the reference model needs n_head*head_dim == n_embd == kv_dim, n_kv_head == n_head");
    AR_CHECK_ARG(c.n_embd % 8 == 0 && c.vocab_size % 8 == 0 && (B * T) % 8 == 0,
                 "gpt_create: n_embd, vocab_size and B*T must be multiples of 8");
    AR_CHECK_ARG(c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128, "gpt_create: head_dim must be 32/64/128");
    AR_CHECK_ARG(c.n_head <= kGateMaxH, "gpt_create: n_head must be <= %d (value-embedding gate)", kGateMaxH);
    AR_CHECK_ARG(c.n_embd <= 4096, "gpt_create: n_embd must be <= 4096");
    AR_CHECK_ARG(precision == AR_PREC_FP32 || precision == AR_PREC_BF16, "gpt_create: bad precision");
    AR_CHECK_ARG(rope_period >= 0, "gpt_create: bad rope_period");
    ar_gpt* m = new ar_gpt();
    m->c = c;
    m->B = B;
    m->T = T;
    m->BT = B * T;
    m->period = rope_period > 0 ? rope_period : B * T;
    m->bf16 = precision == AR_PREC_BF16;
    m->st = S(stream);
    int32_t r = gpt_build(m);
    if (r != AR_OK) {
        ar_gpt_destroy(m);
        return r;
    }
    *out = m;
    return AR_OK;
}

extern "C" int32_t ar_gpt_destroy(ar_gpt* m) {
    if (!m) return AR_OK;
    hipStreamSynchronize(m->st);
    for (int i = 0; i < 2; ++i) {
        if (m->side[i]) hipStreamSynchronize(m->side[i]);
        if (m->side[i]) hipStreamDestroy(m->side[i]);
        if (m->join_ev[i]) hipEventDestroy(m->join_ev[i]);
    }
    if (m->fork_ev) hipEventDestroy(m->fork_ev);
    if (m->graph_exec) hipGraphExecDestroy(m->graph_exec);
    if (m->graph) hipGraphDestroy(m->graph);
    for (hipEvent_t e : m->ev) hipEventDestroy(e);
    for (void* p : m->allocs) hipFree(p);
    delete m;
    return AR_OK;
}

// The accessors answer 0 / -1 / null for a null model.
extern "C" int64_t ar_gpt_num_tensors(const ar_gpt* m) { return m ? (int64_t)m->t.size() : 0; }
extern "C" int64_t ar_gpt_tensor_info(const ar_gpt* m, int64_t i, int64_t* offset, const char** name) {
    if (!m || i < 0 || i >= (int64_t)m->t.size()) return -1;
    if (offset) *offset = m->t[i].offset;
    if (name) *name = m->t[i].name.c_str();
    return m->t[i].size;
}
extern "C" int64_t ar_gpt_num_params(const ar_gpt* m) { return m ? m->nparams : 0; }
extern "C" float* ar_gpt_params(ar_gpt* m) { return m ? m->params : nullptr; }
extern "C" float* ar_gpt_grads(ar_gpt* m) { return m ? m->grads : nullptr; }
extern "C" float* ar_gpt_token_loss(ar_gpt* m) { return m ? m->loss : nullptr; }
extern "C" float* ar_gpt_mean_loss(ar_gpt* m) { return m ? m->mean_loss : nullptr; }

// model.mojo:337-427
extern "C" int32_t ar_gpt_init_weights(ar_gpt* m, uint64_t seed0) {
    AR_CHECK_ARG(m != nullptr, "gpt_init_weights: null model");
    const ar_gpt_config& c = m->c;
    const int64_t C = c.n_embd, V = c.vocab_size, Lr = c.n_layer, kv = c.kv_dim, F = kMlpExpansion * C;
    const float s = (float)(sqrt(3.0) * pow((double)C, -0.5));
    uint64_t seed = seed0;
    ar_stream_t st = AS(m);
    AR_TRY(ar_fill_normal(st, P(m, m->i_wte), seed, 1.0f, V * C)); seed++;
    AR_TRY(ar_fill_normal(st, P(m, m->i_lm), seed, 0.001f, V * C)); seed++;
    AR_TRY(ar_fill_value(st, P(m, m->i_res), 1.0f, Lr));
    AR_TRY(ar_fill_value(st, P(m, m->i_x0), 0.1f, Lr));
    for (int64_t i = 0; i < Lr; ++i) {
        AR_TRY(ar_fill_uniform(st, P(m, m->i_q[i]), seed, -s, s, C * C)); seed++;
        AR_TRY(ar_fill_uniform(st, P(m, m->i_k[i]), seed, -s, s, kv * C)); seed++;
        AR_TRY(ar_fill_uniform(st, P(m, m->i_v[i]), seed, -s, s, kv * C)); seed++;
        AR_TRY(ar_fill_zeros(st, P(m, m->i_proj[i]), C * C));
        AR_TRY(ar_fill_uniform(st, P(m, m->i_fc[i]), seed, -s, s, F * C)); seed++;
        AR_TRY(ar_fill_zeros(st, P(m, m->i_mlpp[i]), C * F));
        if (has_ve(c, i)) {
            AR_TRY(ar_fill_uniform(st, P(m, m->i_ve[i]), seed, -s, s, V * kv)); seed++;
            AR_TRY(ar_fill_zeros(st, P(m, m->i_gate[i]), c.n_kv_head * kGateChannels));
        }
    }
    AR_TRY(ar_precompute_rope(st, m->rope_cos, m->rope_sin, m->rope_rows, c.head_dim, 10000.0));  // config.mojo:87
    if (hipStreamSynchronize(m->st) != hipSuccess) return set_error(AR_EHIP, "gpt_init_weights: sync failed");
    return AR_OK;
}

// model.mojo:777-814
extern "C" int32_t ar_gpt_zero_grads(ar_gpt* m) {
    AR_CHECK_ARG(m != nullptr, "gpt_zero_grads: null model");
    return ar_zero_buffer(AS(m), m->grads, m->nparams);
}

// ------------------------------------------------------------------------
// bf16 step: model.mojo:576-772 / 819-1037 with bf16 operand storage
// ------------------------------------------------------------------------
static int32_t forward_bf16(ar_gpt* m, const int64_t* inputs, const int64_t* targets) {
    const ar_gpt_config& c = m->c;
    const int64_t C = c.n_embd, V = c.vocab_size, BT = m->BT, H = c.n_head, hd = c.head_dim;
    const int64_t F = kMlpExpansion * C;
    hipStream_t st = m->st;
    AR_TRY(to_bf16(st, m->wb, m->params, m->nparams));
    AR_TRY(transpose_bf16(st, m->wbt, m->params, m->wbt_tab, m->wbt_n, m->wbt_tiles));
    for (int64_t i = 0; i < c.n_layer; ++i) {
        LayerBufsB& b = m->LB[i];
        const bool ve = has_ve(c, i);
        // layer 0: x0 = norm(wte[idx]) (model.mojo:605-618); x = res*x_in + x0l*x0; xn = norm(x)
        // (with fuse_rows the previous layer's mlp_proj product produced layer i's input)
        if (i == 0 || !m->fuse_rows)
            AR_TRY(resid_norm(st, i == 0 ? 0 : 1, m->x0, b.x, b.rms_attn, b.xn, ve ? b.xg : nullptr,
                              ve ? b.gate : nullptr, m->x, m->x0, P(m, m->i_wte), inputs, P(m, m->i_res),
                              P(m, m->i_x0), i, ve ? P(m, m->i_gate[i]) : nullptr, H, kGateChannels, BT, C));
        // c_q | c_k | c_v: one [3C, C] weight; rope + head norm of q / k and the
        // value-embedding add of v in its epilogue, or in qkv_post after it
        if (m->fuse_heads) {
            const int e = prof_begin(m);
            const int32_t r = gemm_qkv_fused(st, b.q, b.k, b.v, b.xn, Wb(m, m->i_q[i]), BT, C, hd, m->rope_cos,
                                             m->rope_sin, m->period, ve ? b.gate : nullptr,
                                             ve ? P(m, m->i_ve[i]) : nullptr, inputs);
            prof_end(m, e, 0, 2.0 * BT * 3 * C * C);
            AR_TRY(r);
        } else {
            AR_TRY(gemm_b(m, 0, 0, m->qkv, true, b.xn, true, Wb(m, m->i_q[i]), true, BT, 3 * C, C, false));
            AR_TRY(qkv_post(st, b.q, b.k, b.v, m->qkv, m->rope_cos, m->rope_sin, m->period, b.gate,
                            ve ? P(m, m->i_ve[i]) : nullptr, inputs, BT, C, H, hd));
        }
        FlashOut fo;
        fo.b1 = b.attn_out_b;
        AR_TRY(attention_b(m, AttnOp::FWD, b.attn_out, b.lse, fo, b.q, b.k, b.v, nullptr, nullptr, nullptr,
                           window_size(c, i)));
        // x = x_layer + attn_out @ c_proj^T; rms_mlp, xn_mlp = norm(x)
        if (m->fuse_rows) {
            const int e = prof_begin(m);
            const int32_t r = gemm_rc_norm(st, b.attn_out_b, Wb(m, m->i_proj[i]), BT, C, b.x, m->x, b.rms_mlp,
                                           b.xn_mlp, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0);
            prof_end(m, e, 0, 2.0 * BT * C * C);
            AR_TRY(r);
        } else {
            AR_TRY(gemm_e(m, 0, 0, GEMM_EPI_ADD, m->x, false, b.attn_out_b, true, Wb(m, m->i_proj[i]), BT, C, C, b.x,
                          nullptr, 0.f));
            AR_TRY(resid_norm(st, 2, nullptr, nullptr, b.rms_mlp, b.xn_mlp, nullptr, nullptr, m->x, nullptr, nullptr,
                              nullptr, nullptr, nullptr, 0, nullptr, 0, 0, BT, C));
        }
        // act = relu(xn @ c_fc^T)^2 (the pre-activation is not kept); x += act @ mlp_proj^T
        AR_TRY(gemm_e(m, 0, 0, GEMM_EPI_RELU2, b.act, true, b.xn_mlp, true, Wb(m, m->i_fc[i]), BT, F, C, nullptr,
                      nullptr, 0.f));
        if (m->fuse_rows) {
            // the next layer's input x = res[i+1] (x + act @ mlp_proj^T) + x0l[i+1] x0 and its
            // norm (and VE gate); after the last layer the final norm of x
            const int e = prof_begin(m);
            int32_t r;
            if (i + 1 < c.n_layer) {
                LayerBufsB& nb = m->LB[i + 1];
                const bool nve = has_ve(c, i + 1);
                r = gemm_rc_norm(st, b.act, Wb(m, m->i_mlpp[i]), BT, F, m->x, nb.x, nb.rms_attn, nb.xn, m->x0,
                                 P(m, m->i_res), P(m, m->i_x0), i + 1, nve ? nb.xg : nullptr,
                                 nve ? nb.gate : nullptr, nve ? P(m, m->i_gate[i + 1]) : nullptr, H);
            } else {
                r = gemm_rc_norm(st, b.act, Wb(m, m->i_mlpp[i]), BT, F, m->x, m->x, m->rms_final, m->x_final_b,
                                 nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0);
            }
            prof_end(m, e, 0, 2.0 * BT * C * F);
            AR_TRY(r);
        } else {
            AR_TRY(gemm_e(m, 0, 0, GEMM_EPI_ADD, m->x, false, b.act, true, Wb(m, m->i_mlpp[i]), BT, C, F, m->x,
                          nullptr, 0.f));
        }
    }
    if (!m->fuse_rows)
        AR_TRY(resid_norm(st, 2, nullptr, nullptr, m->rms_final, m->x_final_b, nullptr, nullptr, m->x, nullptr,
                          nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, 0, BT, C));
    // softcapped logits stored as bf16 (in the fp32 logits buffer), as a bf16 lm_head's output is
    AR_TRY(gemm_e(m, 0, 0, GEMM_EPI_SOFTCAP, LogitsB(m), true, m->x_final_b, true, Wb(m, m->i_lm), BT, V, C, nullptr,
                  nullptr, kSoftcap));
    // loss, and the loss gradient for loss_scale 1 while the row is loaded
    AR_TRY(ce_fused(st, m->loss, m->grad_logits_b, LogitsB(m), targets, BT, V, 1.0f));
    m->grad_logits_scale = 1.0f;
    m->grad_logits_valid = true;
    return fixed_sum(st, m->mean_loss, m->loss, nullptr, BT, 0, 0, 0, m->scratch);
}

static int32_t backward_bf16(ar_gpt* m, const int64_t* inputs, const int64_t* targets, float loss_scale) {
    const ar_gpt_config& c = m->c;
    const int64_t C = c.n_embd, V = c.vocab_size, BT = m->BT, H = c.n_head, hd = c.head_dim, kv = c.kv_dim;
    const int64_t F = kMlpExpansion * C;
    hipStream_t st = m->st;
    if (!m->grad_logits_valid || m->grad_logits_scale != loss_scale) {
        AR_TRY(ce_fused(st, nullptr, m->grad_logits_b, LogitsB(m), targets, BT, V, loss_scale));
        m->grad_logits_scale = loss_scale;
        m->grad_logits_valid = true;
    }
    // dX = dY . W as dY . (W^T)^T: NT with both operands K-major
    AR_TRY(gemm_b(m, 1, 0, m->grad_x, false, m->grad_logits_b, true, WbT(m, m->i_lm), true, BT, C, V, false));
    AR_TRY(gemm_b(m, 2, 2, G(m, m->i_lm), false, m->grad_logits_b, true, m->x_final_b, true, BT, V, C, true));
    AR_TRY(norm_bwd(st, 0, m->grad_x, m->grad_xb, nullptr, m->x, m->rms_final, nullptr, nullptr, 0, nullptr, nullptr,
                    nullptr, BT, C));
    for (int64_t r = 0; r < c.n_layer; ++r) {
        const int64_t i = c.n_layer - 1 - r;
        LayerBufsB& b = m->LB[i];
        const bool ve = has_ve(c, i);
        // MLP: dh = relu2_bwd(grad_x @ mlp_proj), 2 h taken as 2 sqrt(act)
        AR_TRY(gemm_e(m, 1, 0, GEMM_EPI_RELU2_BWD, m->grad_h, true, m->grad_xb, true, WbT(m, m->i_mlpp[i]), BT, F, C,
                      b.act, nullptr, 0.f));
        AR_TRY(gemm_b(m, 2, 2, G(m, m->i_mlpp[i]), false, m->grad_xb, true, b.act, true, BT, C, F, true));
        // gradient of the normed MLP input in bf16 (as a bf16 linear's input gradient)
        AR_TRY(gemm_b(m, 1, 0, m->grad_x_norm_b, true, m->grad_h, true, WbT(m, m->i_fc[i]), true, BT, C, F, false));
        AR_TRY(gemm_b(m, 2, 2, G(m, m->i_fc[i]), false, m->grad_h, true, b.xn_mlp, true, BT, F, C, true));
        AR_TRY(norm_bwd(st, 1, m->grad_x, m->grad_xb, nullptr, b.x, b.rms_mlp, nullptr, nullptr, 0, nullptr, nullptr,
                        nullptr, BT, C, m->grad_x_norm_b));  // Q7: saved x of the layer
        // attention output projection (with D = rowsum(dO O) in its epilogue when fused)
        if (m->fuse_heads) {
            const int e = prof_begin(m);
            const int32_t r = gemm_dout_d_fused(st, m->grad_attn_out_b, m->d_buf, m->grad_xb, WbT(m, m->i_proj[i]),
                                                b.attn_out, BT, C, hd);
            prof_end(m, e, 1, 2.0 * BT * C * C);
            AR_TRY(r);
        } else {
            AR_TRY(gemm_b(m, 1, 0, m->grad_attn_out_b, true, m->grad_xb, true, WbT(m, m->i_proj[i]), true, BT, C, C,
                          false));
        }
        AR_TRY(gemm_b(m, 2, 2, G(m, m->i_proj[i]), false, m->grad_xb, true, b.attn_out_b, true, BT, C, C, true));
        const int64_t ws = window_size(c, i);
        // dQ | dK | dV straight into the packed bf16 [BT, 3C] buffer, dQ / dK
        // rotated back by the inverse rope (rope_bwd; Q6: q/k norm backward skipped).
        // D = rowsum(dO * O) (precompute_d) first; the dK / dV kernel stores its
        // bf16 dS tiles and dQ = dS K is formed from them (no S / dP recompute).
        // Without the dS workspace (long sequences) the dQ kernel recomputes S
        // and dP.
        FlashOut fo;
        fo.brs = 3 * C;
        fo.cos_t = m->rope_cos;
        fo.sin_t = m->rope_sin;
        fo.period = m->period;
        fo.b1 = m->grad_qkv + C;
        fo.b2 = m->grad_qkv + 2 * C;
        fo.ds = m->ds_buf;
        if (!m->fuse_heads) AR_TRY(flash_d_bf16(st, m->d_buf, b.attn_out, m->grad_attn_out_b, m->B, m->T, H, hd));
        AR_TRY(attention_b(m, AttnOp::DKV, nullptr, nullptr, fo, b.q, b.k, b.v, m->grad_attn_out_b, b.lse, m->d_buf,
                           ws));
        fo.b1 = m->grad_qkv;
        fo.b2 = nullptr;
        fo.ds = nullptr;
        if (m->ds_buf)
            AR_TRY(attention_dq_ds(m, fo, b.k, ws));
        else
            AR_TRY(attention_b(m, AttnOp::DQ, nullptr, nullptr, fo, b.q, b.k, b.v, m->grad_attn_out_b, b.lse,
                               m->d_buf, ws));
        // ve_apply_bwd from the bf16 dV
        if (ve)
            AR_TRY(ve_bwd(st, m->grad_ve, m->grad_gate, m->grad_qkv + 2 * C, 3 * C, b.gate, P(m, m->i_ve[i]), inputs,
                          BT, C, H, hd));
        if (ve)
            AR_TRY(ar_embedding_bwd_sorted(AS(m), G(m, m->i_ve[i]), m->grad_ve, m->sorted_ids, m->sorted_tok, BT, kv,
                                           m->scratch));
        // gradient of the normed attention input in bf16 (as a bf16 linear's input gradient)
        AR_TRY(gemm_b(m, 1, 0, m->grad_x_norm_b, true, m->grad_qkv, true, WbT(m, m->i_q[i]), true, BT, C, 3 * C,
                      false));
        AR_TRY(gemm_b(m, 2, 2, G(m, m->i_q[i]), false, m->grad_qkv, true, b.xn, true, BT, 3 * C, C, true));
        if (ve)
            AR_TRY(ve_gate_bwd(st, m->grad_x_norm_b, G(m, m->i_gate[i]), m->grad_gate, b.gate, b.xg,
                               P(m, m->i_gate[i]), BT, H, kGateChannels, C, kGateChannels, m->scratch));
        // grad_x = res[i] * (grad_x + rmsnorm_bwd(.)), with the Q8 scalar dots (Q9: grad_x0 unused)
        AR_TRY(norm_bwd(st, 2, m->grad_x, m->grad_xb, nullptr, b.x, b.rms_attn, m->x0, P(m, m->i_res), i,
                        G(m, m->i_res), G(m, m->i_x0), m->scratch, BT, C, m->grad_x_norm_b));
    }
    // Q10: embedding norm backward skipped
    return ar_embedding_bwd_sorted(AS(m), G(m, m->i_wte), m->grad_x, m->sorted_ids, m->sorted_tok, BT, C, m->scratch);
}

// model.mojo:576-772, fp32 step
static int32_t forward_fp32(ar_gpt* m, const int64_t* inputs, const int64_t* targets) {
    const ar_gpt_config& c = m->c;
    const int64_t C = c.n_embd, V = c.vocab_size, BT = m->BT, H = c.n_head, hd = c.head_dim;
    const int64_t kv = c.kv_dim, F = kMlpExpansion * C;
    ar_stream_t st = AS(m);
    AR_TRY(ar_embedding_fwd(st, m->x0, P(m, m->i_wte), inputs, BT, C));
    AR_TRY(ar_rmsnorm_fwd(st, m->x0, m->rms_final, m->x0, BT, C));  // rms discarded, as bufs.rms
    for (int64_t i = 0; i < c.n_layer; ++i) {
        LayerBufs& b = m->L[i];
        const float* xin = i == 0 ? m->x0 : m->x;
        AR_TRY(ar_scaled_add_fwd(st, b.x, xin, m->x0, P(m, m->i_res), P(m, m->i_x0), i, BT * C));
        AR_TRY(ar_rmsnorm_fwd(st, b.xn_attn, b.rms_attn, b.x, BT, C));
        AR_TRY(linear(m, b.q, b.xn_attn, P(m, m->i_q[i]), BT, C, C));
        AR_TRY(linear(m, b.k, b.xn_attn, P(m, m->i_k[i]), BT, kv, C));
        AR_TRY(linear(m, b.v, b.xn_attn, P(m, m->i_v[i]), BT, kv, C));
        if (has_ve(c, i)) {
            AR_TRY(ar_embedding_fwd(st, b.ve, P(m, m->i_ve[i]), inputs, BT, kv));
            AR_TRY(ar_ve_gate_fwd(st, b.gate, b.xn_attn, P(m, m->i_gate[i]), BT, H, kGateChannels, C));
            AR_TRY(ar_ve_apply_fwd(st, b.v, b.gate, b.ve, BT, H, hd));
        }
        AR_TRY(rope_model(m, b.q, false));
        AR_TRY(rope_model(m, b.k, false));
        AR_TRY(ar_rmsnorm_fwd(st, b.q, m->rms_qk, b.q, BT * H, hd));
        AR_TRY(ar_rmsnorm_fwd(st, b.k, m->rms_qk, b.k, BT * H, hd));
        AR_TRY(attention(m, AttnOp::FWD, b.attn_out, b.lse, b.q, b.k, b.v, nullptr, nullptr, nullptr,
                         window_size(c, i)));
        // x = x_layer + attn_out @ c_proj^T (add_residual_fwd in the product's epilogue)
        AR_TRY(linear_add(m, m->x, b.attn_out, P(m, m->i_proj[i]), b.x, BT, C, C));
        AR_TRY(ar_rmsnorm_fwd(st, b.xn_mlp, b.rms_mlp, m->x, BT, C));
        AR_TRY(linear(m, b.mlp_hidden, b.xn_mlp, P(m, m->i_fc[i]), BT, F, C));
        AR_TRY(ar_relu_squared_fwd(st, b.mlp_act, b.mlp_hidden, BT * F));
        AR_TRY(linear_add(m, m->x, b.mlp_act, P(m, m->i_mlpp[i]), m->x, BT, C, F));
    }
    // m->x is the saved pre-final x.
    AR_TRY(ar_rmsnorm_fwd(st, m->x_final, m->rms_final, m->x, BT, C));
    AR_TRY(linear(m, m->logits, m->x_final, P(m, m->i_lm), BT, V, C));
    AR_TRY(ar_softcap_fwd(st, m->logits, m->logits, kSoftcap, BT * V));
    AR_TRY(ar_cross_entropy_fwd(st, m->loss, m->logits, targets, BT, V));
    return fixed_sum(m->st, m->mean_loss, m->loss, nullptr, BT, 0, 0, 0, m->scratch);
}

// model.mojo:576-772
extern "C" int32_t ar_gpt_forward(ar_gpt* m, const int64_t* inputs, const int64_t* targets, float* loss_host) {
    AR_CHECK_ARG(m && inputs && targets, "gpt_forward: null pointer");
    AR_TRY(m->bf16 ? forward_bf16(m, inputs, targets) : forward_fp32(m, inputs, targets));
    if (loss_host) {
        if (hipMemcpyAsync(loss_host, m->mean_loss, sizeof(float), hipMemcpyDeviceToHost, m->st) != hipSuccess ||
            hipStreamSynchronize(m->st) != hipSuccess)
            return set_error(AR_EHIP, "gpt_forward: loss copy failed");
    }
    return AR_OK;
}

// The stable token-id sort shared by the wte and value-embedding scatters
// (depends on the inputs only; run before the rest of the backward).
static int32_t sort_tokens(ar_gpt* m, const int64_t* inputs) {
    return ar_embedding_sort(AS(m), m->sorted_ids, m->sorted_tok, inputs, m->BT, m->sort_bits, m->sort_scratch,
                             m->sort_bytes, nullptr);
}

static int32_t backward_fp32(ar_gpt* m, const int64_t* inputs, const int64_t* targets, float loss_scale) {
    const ar_gpt_config& c = m->c;
    const int64_t C = c.n_embd, V = c.vocab_size, BT = m->BT, H = c.n_head, hd = c.head_dim;
    const int64_t kv = c.kv_dim, F = kMlpExpansion * C;
    ar_stream_t st = AS(m);
    AR_TRY(ar_cross_entropy_softcap_bwd(st, m->grad_logits, m->logits, targets, kSoftcap, BT, V, loss_scale));
    AR_TRY(linear_dx(m, m->grad_x, m->grad_logits, P(m, m->i_lm), BT, V, C));
    AR_TRY(linear_dw(m, G(m, m->i_lm), m->grad_logits, m->x_final, BT, V, C));
    AR_TRY(ar_rmsnorm_bwd(st, m->grad_x, m->grad_x, m->x, m->rms_final, BT, C));
    for (int64_t r = 0; r < c.n_layer; ++r) {
        const int64_t i = c.n_layer - 1 - r;
        LayerBufs& b = m->L[i];
        // MLP block; dY of mlp_proj is grad_x itself (model.mojo:873 copy elided)
        AR_TRY(linear_dx(m, m->grad_mlp, m->grad_x, P(m, m->i_mlpp[i]), BT, C, F));
        AR_TRY(linear_dw(m, G(m, m->i_mlpp[i]), m->grad_x, b.mlp_act, BT, C, F));
        AR_TRY(ar_relu_squared_bwd(st, m->grad_mlp, m->grad_mlp, b.mlp_hidden, BT * F));
        AR_TRY(linear_dx(m, m->grad_x_norm, m->grad_mlp, P(m, m->i_fc[i]), BT, F, C));
        AR_TRY(linear_dw(m, G(m, m->i_fc[i]), m->grad_mlp, b.xn_mlp, BT, F, C));
        AR_TRY(ar_rmsnorm_bwd(st, m->grad_x_norm, m->grad_x_norm, b.x, b.rms_mlp, BT, C));  // Q7
        AR_TRY(ar_add_residual_fwd(st, m->grad_x, m->grad_x, m->grad_x_norm, BT * C));
        // attention output projection (Q2: read all of dY, then write dX)
        AR_TRY(linear_dx(m, m->grad_attn_out, m->grad_x, P(m, m->i_proj[i]), BT, C, C));
        AR_TRY(linear_dw(m, G(m, m->i_proj[i]), m->grad_x, b.attn_out, BT, C, C));
        const int64_t ws = window_size(c, i);
        AR_TRY(ar_flash_attn_bwd_precompute_d(st, m->d_buf, b.attn_out, m->grad_attn_out, m->B, m->T, H, hd));
        AR_TRY(attention(m, AttnOp::DQ, m->grad_q, nullptr, b.q, b.k, b.v, m->grad_attn_out, b.lse, m->d_buf, ws));
        AR_TRY(attention(m, AttnOp::DKV, m->grad_k, m->grad_v, b.q, b.k, b.v, m->grad_attn_out, b.lse, m->d_buf,
                         ws));
        // Q6: q/k per-head norm backward skipped
        if (has_ve(c, i)) {
            AR_TRY(ar_ve_apply_bwd(st, m->grad_ve, m->grad_gate, m->grad_v, b.gate, b.ve, BT, H, hd));
            AR_TRY(ar_embedding_bwd_sorted(st, G(m, m->i_ve[i]), m->grad_ve, m->sorted_ids, m->sorted_tok, BT, kv,
                                           m->scratch));
        }
        AR_TRY(rope_model(m, m->grad_q, true));
        AR_TRY(rope_model(m, m->grad_k, true));
        AR_TRY(linear_dx(m, m->grad_x_norm, m->grad_q, P(m, m->i_q[i]), BT, C, C));
        AR_TRY(linear_dw(m, G(m, m->i_q[i]), m->grad_q, b.xn_attn, BT, C, C));
        AR_TRY(linear_dx(m, m->grad_tmp, m->grad_k, P(m, m->i_k[i]), BT, kv, C));
        AR_TRY(ar_add_residual_fwd(st, m->grad_x_norm, m->grad_x_norm, m->grad_tmp, BT * C));
        AR_TRY(linear_dw(m, G(m, m->i_k[i]), m->grad_k, b.xn_attn, BT, kv, C));
        AR_TRY(linear_dx(m, m->grad_tmp, m->grad_v, P(m, m->i_v[i]), BT, kv, C));
        AR_TRY(ar_add_residual_fwd(st, m->grad_x_norm, m->grad_x_norm, m->grad_tmp, BT * C));
        AR_TRY(linear_dw(m, G(m, m->i_v[i]), m->grad_v, b.xn_attn, BT, kv, C));
        if (has_ve(c, i))
            AR_TRY(ve_gate_bwd(m->st, m->grad_x_norm, G(m, m->i_gate[i]), m->grad_gate, b.gate, b.xn_attn,
                               P(m, m->i_gate[i]), BT, H, kGateChannels, C, C, m->scratch));
        AR_TRY(ar_rmsnorm_bwd(st, m->grad_x_norm, m->grad_x_norm, b.x, b.rms_attn, BT, C));
        AR_TRY(ar_add_residual_fwd(st, m->grad_x, m->grad_x, m->grad_x_norm, BT * C));
        // Q8: post-scaled-add saved x; Q9: grad_x0 assigned and never consumed
        AR_TRY(fixed_sum(m->st, G(m, m->i_res), m->grad_x, b.x, BT * C, 2, 1, i, m->scratch));
        AR_TRY(fixed_sum(m->st, G(m, m->i_x0), m->grad_x, m->x0, BT * C, 2, 1, i, m->scratch));
        AR_TRY(ar_scaled_add_bwd(st, m->grad_x, m->grad_x0, m->grad_x, P(m, m->i_res), P(m, m->i_x0), i, BT * C));
    }
    // Q10: embedding norm backward skipped
    AR_TRY(ar_embedding_bwd_sorted(st, G(m, m->i_wte), m->grad_x, m->sorted_ids, m->sorted_tok, BT, C, m->scratch));
    return AR_OK;
}

// model.mojo:819-1037 (quirks Q4-Q10 of the reference backward reproduced)
extern "C" int32_t ar_gpt_backward(ar_gpt* m, const int64_t* inputs, const int64_t* targets, float loss_scale) {
    AR_CHECK_ARG(m && inputs && targets, "gpt_backward: null pointer");
    AR_TRY(sort_tokens(m, inputs));
    return m->bf16 ? backward_bf16(m, inputs, targets, loss_scale) : backward_fp32(m, inputs, targets, loss_scale);
}

// train.mojo:25-33
static double lr_multiplier(double progress) {
    const double kWarmup = 0.0, kWarmdown = 0.5, kFinal = 0.0;  // config.mojo:81-83
    if (progress < kWarmup) return kWarmup > 0 ? progress / kWarmup : 1.0;
    if (progress < 1.0 - kWarmdown) return 1.0;
    const double cd = (1.0 - progress) / kWarmdown;
    return cd + (1.0 - cd) * kFinal;
}

// Step-dependent optimizer scalars (train.mojo:246-281), computed on the
// host as the reference does and handed to the kernels through device memory
// (m->dsc) so a recorded graph replays with each step's values.
enum {
    kScLrLm = 0, kScLrWte, kScLrRes, kScLrX0, kScLrVe, kScLrGate,  // AdamW group lr (f32(lr_g * lrm))
    kScBc1Default, kScBc1X0, kScBc2,                             // 1 - beta^step
    kScMuonLr0,                                                  // + shape class 0 / 1 / 2
    kScMu = kScMuonLr0 + 3, kScWd, kScCount
};
struct StepScalars {
    float v[16];
};
static_assert(kScCount <= 16, "step scalars");

__global__ void set_scalars_k(float* dst, StepScalars s) {
    if (threadIdx.x < kScCount) dst[threadIdx.x] = s.v[threadIdx.x];
}

// Muon shape classes: c_q / c_k / c_v / c_proj [C, C], c_fc [4C, C], mlp_proj [C, 4C].
static int muon_class(const ar_gpt* m, int64_t ti) {
    const Tensor& t = m->t[ti];
    return t.rows == t.cols ? 0 : (t.rows > t.cols ? 1 : 2);
}

// Advances the AdamW step counter (train.mojo:253) and returns the scalars.
static StepScalars step_scalars(ar_gpt* m, double progress) {
    const ar_gpt_config& c = m->c;
    if (progress > 1.0) progress = 1.0;
    const double lrm = lr_multiplier(progress);
    const double lr_scale = pow((double)c.n_embd / 768.0, -0.5);  // train.mojo:167
    m->adam_step += 1;
    StepScalars s{};
    s.v[kScLrLm] = (float)(0.004 * lr_scale * lrm);    // UNEMBEDDING_LR
    s.v[kScLrWte] = (float)(0.6 * lr_scale * lrm);     // EMBEDDING_LR
    s.v[kScLrRes] = (float)(0.5 * 0.01 * lrm);         // SCALAR_LR * 0.01
    s.v[kScLrX0] = (float)(0.5 * lrm);                 // SCALAR_LR (beta1 0.96)
    s.v[kScLrVe] = (float)(0.6 * lr_scale * lrm);      // EMBEDDING_LR
    s.v[kScLrGate] = (float)(0.04 * lrm);              // MATRIX_LR
    // optimizer.mojo:114-118: bias corrections by repeated f32 multiplication
    float p08 = 1.f, p096 = 1.f, p095 = 1.f;
    for (int64_t k = 0; k < m->adam_step; ++k) {
        p08 *= 0.8f;
        p096 *= 0.96f;
        p095 *= 0.95f;
    }
    s.v[kScBc1Default] = 1.f - p08;
    s.v[kScBc1X0] = 1.f - p096;
    s.v[kScBc2] = 1.f - p095;
    // Muon: lr = f32(0.04 lrm sqrt(max(1, rows/cols))); momentum 0.85 -> 0.95
    // over 300 steps (train.mojo:268-271); wd = 0.2 (1 - progress) (train.mojo:272)
    const double shapes[3][2] = {{(double)c.n_embd, (double)c.n_embd},
                                 {(double)kMlpExpansion * c.n_embd, (double)c.n_embd},
                                 {(double)c.n_embd, (double)kMlpExpansion * c.n_embd}};
    for (int k = 0; k < 3; ++k)
        s.v[kScMuonLr0 + k] = (float)(0.04 * lrm * muon_lr_factor((int64_t)shapes[k][0], (int64_t)shapes[k][1]));
    double frac = (double)m->adam_step / 300.0;
    if (frac > 1.0) frac = 1.0;
    s.v[kScMu] = (float)((1.0 - frac) * 0.85 + frac * 0.95);
    s.v[kScWd] = (float)(0.2 * (1.0 - progress));
    return s;
}

// The optimizer's kernels, all scalars read from m->dsc; fork: the AdamW
// updates and the mlp_proj Muon group on side stream 1, the c_fc group on
// side stream 0, the square group on st.
static int32_t optimizer_body(ar_gpt* m, bool fork) {
    const ar_gpt_config& c = m->c;
    const hipStream_t ast = fork ? m->side[1] : m->st;
    // every AdamW tensor in one launch
    std::vector<AdamEntry> adam;
    auto add = [&](int64_t ti, int lr_i, int bc1_i, float b1) {
        const Tensor& t = m->t[ti];
        adam.push_back(AdamEntry{t.offset, t.size, lr_i, bc1_i, b1});
    };
    add(m->i_lm, kScLrLm, kScBc1Default, 0.8f);
    add(m->i_wte, kScLrWte, kScBc1Default, 0.8f);
    add(m->i_res, kScLrRes, kScBc1Default, 0.8f);
    add(m->i_x0, kScLrX0, kScBc1X0, 0.96f);
    for (int64_t i = 0; i < c.n_layer; ++i)
        if (has_ve(c, i)) {
            add(m->i_ve[i], kScLrVe, kScBc1Default, 0.8f);
            add(m->i_gate[i], kScLrGate, kScBc1Default, 0.8f);
        }
    AR_TRY(adamw_multi(ast, m->params, m->grads, m->adam_m, m->adam_v, adam.data(), (int)adam.size(), m->dsc,
                       kScBc2, 0.95f, 1e-10f, 0.0f));
    // Muon on every 2-D matrix, grouped by shape and run as batched GEMMs.
    std::vector<int64_t> sq, fc, mp;
    for (int64_t i = 0; i < c.n_layer; ++i) {
        sq.push_back(m->i_q[i]);
        sq.push_back(m->i_k[i]);
        sq.push_back(m->i_v[i]);
        sq.push_back(m->i_proj[i]);
        fc.push_back(m->i_fc[i]);
        mp.push_back(m->i_mlpp[i]);
    }
    int gi = 0;
    for (const std::vector<int64_t>* grp : {&sq, &fc, &mp}) {
        const hipStream_t gst = fork && gi > 0 ? m->side[gi - 1] : m->st;
        float* const gscratch = m->scratch + m->muon_off[gi];
        ++gi;
        const int64_t total = (int64_t)grp->size();
        const int64_t ngroups = (total + kMuonMaxGroup - 1) / kMuonMaxGroup;
        const int64_t per = (total + ngroups - 1) / ngroups;
        for (int64_t g0 = 0; g0 < total; g0 += per) {
            const int n = (int)(g0 + per <= total ? per : total - g0);
            float* ps[kMuonMaxGroup];
            const float* gs[kMuonMaxGroup];
            float* ms[kMuonMaxGroup];
            const Tensor& t0 = m->t[(*grp)[g0]];
            for (int j = 0; j < n; ++j) {
                const Tensor& t = m->t[(*grp)[g0 + j]];
                ps[j] = m->params + t.offset;
                gs[j] = m->grads + t.offset;
                ms[j] = m->muon_buf + t.offset;
            }
            MuonDev dev;
            dev.dsc = m->dsc;
            dev.lr_i = kScMuonLr0 + muon_class(m, (*grp)[g0]);
            dev.mu_i = kScMu;
            dev.wd_i = kScWd;
            const int e = prof_begin(m);
            AR_TRY(muon_group_step(gst, ps, gs, ms, n, t0.rows, t0.cols, 0.04, 1.0, 0.0, 0.0, m->bf16, gscratch,
                                   dev));
            const double smd = (double)(t0.rows < t0.cols ? t0.rows : t0.cols);
            const double lgd = (double)(t0.rows < t0.cols ? t0.cols : t0.rows);
            prof_end(m, e, 6, n * 5.0 * (4.0 * lgd * smd * smd + 2.0 * smd * smd * smd));
        }
    }
    return AR_OK;
}

static int32_t optimizer_kernels(ar_gpt* m) {
    // Profiling runs keep every kernel on st, in order, so that each Muon
    // group's events bracket only its own kernels.
    const bool fork = !m->prof;
    if (!fork) return optimizer_body(m, false);
    if (hipEventRecord(m->fork_ev, m->st) != hipSuccess || hipStreamWaitEvent(m->side[0], m->fork_ev, 0) != hipSuccess ||
        hipStreamWaitEvent(m->side[1], m->fork_ev, 0) != hipSuccess)
        return set_error(AR_EHIP, "optimizer: fork");
    // The side streams are joined back into st on every path, also after a
    // failed launch: st then still orders after everything queued on them
    // (and a capture of st ends with every forked stream joined).
    const int32_t r = optimizer_body(m, true);
    int32_t rj = AR_OK;
    for (int i = 0; i < 2; ++i)
        if (hipEventRecord(m->join_ev[i], m->side[i]) != hipSuccess ||
            hipStreamWaitEvent(m->st, m->join_ev[i], 0) != hipSuccess)
            rj = set_error(AR_EHIP, "optimizer: join");
    return r != AR_OK ? r : rj;
}

// train.mojo:246-281
extern "C" int32_t ar_gpt_optimizer_step(ar_gpt* m, double progress) {
    AR_CHECK_ARG(m != nullptr, "gpt_optimizer_step: null model");
    const StepScalars s = step_scalars(m, progress);
    set_scalars_k<<<1, 64, 0, m->st>>>(m->dsc, s);
    AR_TRY(check_launch("gpt_optimizer_step: scalars"));
    return optimizer_kernels(m);
}

// train.mojo:231-282
extern "C" int32_t ar_gpt_train_step(ar_gpt* m, const int64_t* inputs, const int64_t* targets, double progress,
                                     float* loss_host) {
    AR_CHECK_ARG(m && inputs && targets, "gpt_train_step: null pointer");
    AR_TRY(ar_gpt_zero_grads(m));
    AR_TRY(ar_gpt_forward(m, inputs, targets, nullptr));
    AR_TRY(ar_gpt_backward(m, inputs, targets, 1.0f));
    AR_TRY(ar_gpt_optimizer_step(m, progress));
    if (loss_host) {
        if (hipMemcpyAsync(loss_host, m->mean_loss, sizeof(float), hipMemcpyDeviceToHost, m->st) != hipSuccess ||
            hipStreamSynchronize(m->st) != hipSuccess)
            return set_error(AR_EHIP, "gpt_train_step: loss copy failed");
    }
    return AR_OK;
}

// ar_gpt_train_step from a HIP graph: [set scalars] -> [zero_grads, forward,
// token-id sort, backward, optimizer kernels].  The scalar node's kernel
// arguments are replaced before each launch (hipGraphExecKernelNodeSetParams
// copies them), so the host never races a pending replay.
extern "C" int32_t ar_gpt_train_step_graph(ar_gpt* m, const int64_t* inputs, const int64_t* targets,
                                           double progress, float* loss_host) {
    AR_CHECK_ARG(m && inputs && targets, "gpt_train_step_graph: null pointer");
    AR_CHECK_ARG(m->st != nullptr, "gpt_train_step_graph: the model's stream must not be the null stream");
    // events recorded by graph nodes give no usable elapsed times on this runtime
    AR_CHECK_ARG(!m->prof, "gpt_train_step_graph: disable profiling (ar_gpt_profile) first");
    StepScalars s = step_scalars(m, progress);
    void* sargs[] = {&m->dsc, &s};
    hipKernelNodeParams kp{};
    kp.func = reinterpret_cast<void*>(set_scalars_k);
    kp.gridDim = dim3(1);
    kp.blockDim = dim3(64);
    kp.sharedMemBytes = 0;
    kp.kernelParams = sargs;
    kp.extra = nullptr;
    if (!m->graph_exec || m->graph_in != inputs || m->graph_tg != targets) {
        if (m->graph_exec) hipGraphExecDestroy(m->graph_exec);
        if (m->graph) hipGraphDestroy(m->graph);
        m->graph_exec = nullptr;
        m->graph = nullptr;
        if (hipStreamSynchronize(m->st) != hipSuccess) return set_error(AR_EHIP, "gpt_train_step_graph: sync failed");
        hipGraph_t body = nullptr;
        if (hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal) != hipSuccess)
            return set_error(AR_EHIP, "gpt_train_step_graph: begin capture failed");
        int32_t r = ar_zero_buffer(AS(m), m->grads, m->nparams);
        if (!r) r = m->bf16 ? forward_bf16(m, inputs, targets) : forward_fp32(m, inputs, targets);
        if (!r) r = sort_tokens(m, inputs);
        if (!r) r = m->bf16 ? backward_bf16(m, inputs, targets, 1.0f) : backward_fp32(m, inputs, targets, 1.0f);
        if (!r) r = optimizer_kernels(m);
        const hipError_t ec = hipStreamEndCapture(m->st, &body);
        if (r) {
            if (body) hipGraphDestroy(body);
            return r;
        }
        if (ec != hipSuccess || !body) return set_error(AR_EHIP, "gpt_train_step_graph: capture failed");
        hipGraph_t g = nullptr;
        hipGraphNode_t sn = nullptr, cn = nullptr;
        bool ok = hipGraphCreate(&g, 0) == hipSuccess && hipGraphAddKernelNode(&sn, g, nullptr, 0, &kp) == hipSuccess &&
                  hipGraphAddChildGraphNode(&cn, g, &sn, 1, body) == hipSuccess;
        hipGraphDestroy(body);  // the child node holds its own copy
        hipGraphExec_t ex = nullptr;
        ok = ok && hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) == hipSuccess;
        if (!ok) {
            if (g) hipGraphDestroy(g);
            return set_error(AR_EHIP, "gpt_train_step_graph: graph build failed");
        }
        m->graph = g;
        m->graph_exec = ex;
        m->graph_scalars = sn;
        m->graph_in = inputs;
        m->graph_tg = targets;
    } else if (hipGraphExecKernelNodeSetParams(m->graph_exec, m->graph_scalars, &kp) != hipSuccess) {
        return set_error(AR_EHIP, "gpt_train_step_graph: scalar update failed");
    }
    if (hipGraphLaunch(m->graph_exec, m->st) != hipSuccess) return set_error(AR_EHIP, "gpt_train_step_graph: launch failed");
    if (loss_host) {
        if (hipMemcpyAsync(loss_host, m->mean_loss, sizeof(float), hipMemcpyDeviceToHost, m->st) != hipSuccess ||
            hipStreamSynchronize(m->st) != hipSuccess)
            return set_error(AR_EHIP, "gpt_train_step_graph: loss copy failed");
    }
    return AR_OK;
}

extern "C" int32_t ar_gpt_profile(ar_gpt* m, int32_t enable) {
    AR_CHECK_ARG(m != nullptr, "gpt_profile: null model");
    if (hipStreamSynchronize(m->st) != hipSuccess) return set_error(AR_EHIP, "gpt_profile: sync failed");
    m->prof = enable != 0;
    m->recs.clear();
    m->ev_used = 0;
    return AR_OK;
}

extern "C" int32_t ar_gpt_profile_read(ar_gpt* m, int32_t cls, double* ms, int64_t* launches, double* flops) {
    AR_CHECK_ARG(m && ms && launches && flops, "gpt_profile_read: null pointer");
    if (hipStreamSynchronize(m->st) != hipSuccess) return set_error(AR_EHIP, "gpt_profile_read: sync failed");
    double t = 0, f = 0;
    int64_t n = 0;
    for (const auto& r : m->recs) {
        if (r.cls != cls) continue;
        float e = 0.f;
        if (hipEventElapsedTime(&e, m->ev[r.e0], m->ev[r.e1]) != hipSuccess)
            return set_error(AR_EHIP, "gpt_profile_read: elapsed time failed");
        t += e;
        f += r.flops;
        ++n;
    }
    *ms = t;
    *launches = n;
    *flops = f;
    return AR_OK;
}
