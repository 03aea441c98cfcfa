// ar_internal.hpp -- library-internal entry points shared by the C ABI
// wrappers, the Muon composite and the whole-step driver.  Unlike the ABI
// wrappers these never touch the library workspace: every scratch buffer is
// passed in by the caller, so composites can carve one allocation into
// non-overlapping pieces.
#pragma once

#include "ar_common.hpp"

namespace ar {

// ---- GEMM (ar_gemm.hip) ----
// layout 0 NT: C[M,N]  = X[M,K] . W[N,K]^T            (linear_fwd)
//        1 NN: C[M,K]  = X[M,N] . W[N,K]              (linear_bwd_dx, X = dY)
//        2 TN: C[N,K] (+)= X[M,N]^T . W[M,K]          (linear_bwd_dw, X = dY, W = input)
// splits: 1 = no reduction split; 0 = choose automatically (TN only).
// partial: fp32 scratch of at least gemm_partial_elems(...) elements when the
// chosen split count is > 1 (may be null otherwise).
// bf16_operands: both operands stored as bf16 (the persistent kernel's case).
int64_t gemm_auto_splits(int layout, bool bf16, bool bf16_operands, int64_t M, int64_t N, int64_t K);
int64_t gemm_partial_elems(int layout, int64_t M, int64_t N, int64_t K, int64_t splits);
int32_t gemm_f32(hipStream_t st, int layout, bool bf16, float* C, const float* X, const float* W, int64_t M,
                 int64_t N, int64_t K, bool accumulate, int64_t splits, float* partial);
// Y = X W^T (layout 0 of gemm_f32) added to R in the epilogue: C = R + Y,
// the add in fp32 exactly as a separate residual add does it (R may alias C).
int32_t gemm_f32_add(hipStream_t st, bool bf16, float* C, const float* X, const float* W, const float* R, int64_t M,
                     int64_t N, int64_t K);
// Same, with each operand stored as bf16 (flag set) or fp32; bf16 compute.
int32_t gemm_bf16io(hipStream_t st, int layout, void* C, int c_bf16, const void* X, int x_bf16, const void* W,
                    int w_bf16, int64_t M, int64_t N, int64_t K, bool accumulate, int64_t splits, float* partial);
// NT (layout 0) / NN (layout 1) GEMM with a fused epilogue, bf16 compute:
// epi 3 ADD (C = aux + acc, aux fp32), 4 RELU2 (C = relu(acc)^2),
// 5 SOFTCAP (C = cap tanh(acc/cap)), 6 RELU2_BWD (C = aux > 0 ? 2 sqrt(aux) acc : 0,
// aux = the activation relu(h)^2).
enum { GEMM_EPI_ADD = 3, GEMM_EPI_RELU2 = 4, GEMM_EPI_SOFTCAP = 5, GEMM_EPI_RELU2_BWD = 6 };
int32_t gemm_epilogue(hipStream_t st, int layout, int epi, void* C, int c_bf16, const void* X, int x_bf16,
                      const void* W, int w_bf16, int64_t M, int64_t N, int64_t K, const void* aux, void* aux_out,
                      float cap);
// Row-complete NT product for C = 512 output columns with the row pass of
// resid_norm in its epilogue: x = r + A W^T (x0 null), or
// x = sa[layer] (r + A W^T) + sb[layer] x0; writes x (fp32, may alias r),
// rms = sqrt(mean(x^2) + 1e-5), xn = bf16(x / rms), and with gate_out set the
// value-embedding gate (xg = (x / rms)[:, :32], gate = 2 sigmoid(gate_w xg)).
// A: bf16 [M, K], W: bf16 [512, K].
bool gemm_rc_fusable(int64_t M, int64_t C, int64_t K);
int32_t gemm_rc_norm(hipStream_t st, const bf16* A, const bf16* W, int64_t M, int64_t K, const float* r, float* x_out,
                     float* rms_out, bf16* xn_out, const float* x0, const float* sa, const float* sb, int64_t layer,
                     float* xg_out, float* gate_out, const float* gate_w, int64_t nkv);
// Whether gemm_qkv_fused / gemm_dout_d_fused take this shape.
bool gemm_head_fusable(int64_t M, int64_t C, int64_t hd);
// The bf16 step's q|k|v forward product xn [M, C] . Wqkv [3C, C]^T with
// qkv_post fused into its epilogue (persistent kernel, head-aligned waves):
// q and k rotated (table row = row % period) and head-normed, v plus
// gate x table[idx] when gate is set, each as bf16 [M, C].  The rope and the
// norm act on the fp32 products (qkv_post rounds them to bf16 first).
// AR_EUNSUPPORTED (nothing launched) when the shape does not fit: head_dim
// 64 / 128, C % 256 == 0, M % 256 == 0.
int32_t gemm_qkv_fused(hipStream_t st, bf16* q, bf16* k, bf16* v, const bf16* xn, const bf16* w, int64_t M, int64_t C,
                       int64_t hd, const float* cos_t, const float* sin_t, int64_t period, const float* gate,
                       const float* table, const int64_t* idx);
// The c_proj dX product dO = gy [M, C] . wt [C, C]^T (bf16 out) with
// D[row, head] = sum_d bf16(dO) O (fp32 O [M, C]) in its epilogue, [M, C / hd].
// AR_EUNSUPPORTED when the shape does not fit (as gemm_qkv_fused).
int32_t gemm_dout_d_fused(hipStream_t st, bf16* dout, float* d, const bf16* gy, const bf16* wt, const float* o,
                          int64_t M, int64_t C, int64_t hd);
// Batched GEMM-space form: C_b[mo,no] = sum_r A_b(mo,r) B_b(no,r); ak / bk
// select K-major (r contiguous, row stride lda/ldb) vs MN-major storage.
// With aux: C_b = alpha * (A_b B_b^T) + beta * aux_b (aux laid out as C).
int32_t gemm_batched_f32(hipStream_t st, bool bf16, bool ak, bool bk, float* C, const float* A, const float* B,
                         int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                         int64_t sA, int64_t sB, int64_t sC, const float* aux = nullptr, float alpha = 1.f,
                         float beta = 0.f);
// The same with bf16 operands in memory and an optional bf16 copy Cb of the
// fp32 result (same strides as C).
int32_t gemm_batched_bf16(hipStream_t st, bool ak, bool bk, float* C, bf16* Cb, const bf16* A, const bf16* B,
                          int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                          int64_t sA, int64_t sB, int64_t sC, const float* aux = nullptr, float alpha = 1.f,
                          float beta = 0.f);

// ---- reductions (ar_reduce.hip) ----
constexpr int kSumBlocks = 512;
// mode_in: 0 sum a, 1 sum a*a, 2 sum a*b.  mode_out: 0 out[idx] = s/n,
// 1 out[idx] += s, 2 out[0] = 1/(sqrt(s)*1.02 + 1e-6).  partial: kSumBlocks floats.
int32_t fixed_sum(hipStream_t st, float* out, const float* a, const float* b, int64_t n, int mode_in, int mode_out,
                  int64_t idx, float* partial);
// data /= (||data||_F * 1.02 + 1e-6); scratch: kSumBlocks + 1 floats.
int32_t frob_normalize(hipStream_t st, float* data, int64_t n, float* scratch);
constexpr int kGateBlocks = 256;
// partial: kGateBlocks * n_kv_head * gate_channels floats.  gx has row
// stride C, xn row stride ldx.
int32_t ve_gate_bwd(hipStream_t st, float* gx, float* gw, const float* ggate, const float* gate, const float* xn,
                    const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C, int64_t ldx, float* partial);
// the same, adding into a bf16 gx (read, add in fp32, round)
int32_t ve_gate_bwd(hipStream_t st, bf16* gx, float* gw, const float* ggate, const float* gate, const float* xn,
                    const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C, int64_t ldx, float* partial);
constexpr int kGateMaxH = 16;

// ---- attention (ar_attention.hip) ----
enum class AttnOp { FWD, DQ, DKV };
// scale: the softmax scale; 0 = 1/sqrt(HD).  A caller that zero-pads rows
// from a smaller head_dim to HD passes 1/sqrt of the unpadded head_dim.
template <bool BF16, typename TIN>
int32_t attn_dispatch(hipStream_t st, AttnOp op, float* o1, float* o2, const TIN* q, const TIN* k, const TIN* v,
                      const TIN* dout, const float* lse, const float* dbuf, int64_t B, int64_t T, int64_t H,
                      int64_t HD, int64_t window, float scale = 0.f);

// bf16-stored operands (ar_flash.hip): q, k, v, dout bf16.  fp32 outputs
// (may be null except LSE): FWD o1 = O, o2 = LSE; DQ o1 = dQ; DKV o1 = dK,
// o2 = dV.  bf16 outputs per FlashOut: FWD b1 = O; DQ b1 = dQ; DKV b1 = dK,
// b2 = dV (row stride brs, 0 = H*hd); with cos_t / sin_t the bf16 dQ / dK are
// rotated back by the inverse rope (table row = flat token % period).
struct FlashOut {
    bf16* b1 = nullptr;
    bf16* b2 = nullptr;
    int64_t brs = 0;
    const float* cos_t = nullptr;
    const float* sin_t = nullptr;
    int64_t period = 0;
    // DKV only: when set, the bf16 dS tiles are stored here for flash_dq_ds_bf16
    // (flash_ds_elems(B, T, H) bf16 elements).
    bf16* ds = nullptr;
};
int32_t flash_attn_bf16(hipStream_t st, AttnOp op, float* o1, float* o2, const FlashOut& fo, const bf16* q,
                        const bf16* k, const bf16* v, const bf16* dout, const float* lse, const float* dbuf, int64_t B,
                        int64_t T, int64_t H, int64_t HD, int64_t window, float scale = 0.f);
// dS workspace size (bf16 elements) of a DKV launch with FlashOut::ds.
int64_t flash_ds_elems(int64_t B, int64_t T, int64_t H);
// D = rowsum(dO * O) per (token, head) from bf16 dO [B, T, H, hd] and fp32 O.
int32_t flash_d_bf16(hipStream_t st, float* d, const float* o, const bf16* dout, int64_t B, int64_t T, int64_t H,
                     int64_t HD);
// dQ = scale * dS K from the dS tiles a DKV launch stored (same window): bf16
// to fo.b1 (row stride fo.brs), inverse-rope rotated with fo.cos_t / sin_t.
int32_t flash_dq_ds_bf16(hipStream_t st, const FlashOut& fo, const bf16* k, const bf16* ds, int64_t B, int64_t T,
                         int64_t H, int64_t HD, int64_t window);

// ---- element-wise (ar_elementwise.hip) ----
int32_t rope(hipStream_t st, float* out, const float* in, const float* cos_t, const float* sin_t, int64_t nt,
             int64_t nh, int64_t hd, int64_t period, bool inverse);
// AdamW (optimizer.mojo:27-57) with lr = sc[lr_i], bias corrections
// 1 - b1^t = sc[bc1_i], 1 - b2^t = sc[bc2_i] read from device memory.
int32_t adamw_dev(hipStream_t st, float* p, const float* g, float* m, float* v, int64_t n, const float* sc,
                  int lr_i, int bc1_i, int bc2_i, float b1, float b2, float eps, float wd);

// AdamW over several tensors of the same arenas in one launch: tensor j is
// elements [offset, offset + size) of p, g, m and v, with its own lr
// (sc[lr_i]), bias correction 1 - b1^t (sc[bc1_i]) and beta1.
struct AdamEntry {
    int64_t offset, size;
    int lr_i, bc1_i;
    float b1;
};
constexpr int kAdamMaxTensors = 32;
struct AdamTable {
    int n;
    int64_t off[kAdamMaxTensors], size[kAdamMaxTensors], blk0[kAdamMaxTensors];
    int lr_i[kAdamMaxTensors], bc1_i[kAdamMaxTensors];
    float b1[kAdamMaxTensors];
};
int32_t adamw_multi(hipStream_t st, float* p, const float* g, float* m, float* v, const AdamEntry* e, int n,
                    const float* sc, int bc2_i, float b2, float eps, float wd);

// ---- fused row kernels of the bf16 step (ar_fused.hip) ----
// mode 0: x0 = rmsnorm(table[idx]), x = sa[l] x0 + sb[l] x0; 1: x = sa[l] xin +
// sb[l] x0; 2: x = xin.  Then rms, xn = bf16(x / rms); with gate_out also
// xg = xn[:, :gc] (fp32) and gate = 2 sigmoid(gate_w . xg).
int32_t resid_norm(hipStream_t st, int mode, float* x0_out, float* x_out, float* rms_out, bf16* xn_out,
                   float* xg_out, float* gate_out, const float* xin, const float* x0, const float* table,
                   const int64_t* idx, const float* sa, const float* sb, int64_t layer, const float* gate_w,
                   int64_t nkv, int64_t gc, int64_t rows, int64_t C);
// qkv [nt, 3C] bf16 -> q, k (rope + per-head rmsnorm), v (+ gate * table[idx]), bf16.
int32_t qkv_post(hipStream_t st, bf16* q, bf16* k, bf16* v, const bf16* qkv, const float* cos_t, const float* sin_t,
                 int64_t period, const float* gate, const float* table, const int64_t* idx, int64_t nt, int64_t C,
                 int64_t H, int64_t hd);
// loss (may be null) and bf16 grad = (softmax - onehot) * scale per row.
int32_t ce_fused(hipStream_t st, float* loss, bf16* grad, const float* logits, const int64_t* targets, int64_t rows,
                 int64_t V, float scale);
// the same from bf16 (softcapped) logits
int32_t ce_fused(hipStream_t st, float* loss, bf16* grad, const bf16* logits, const int64_t* targets, int64_t rows,
                 int64_t V, float scale);
// gve = gate * dv, ggate = per-head sum of table[idx] * dv (dv bf16, row stride ldv).
int32_t ve_bwd(hipStream_t st, float* gve, float* ggate, const bf16* gv, int64_t ldv, const float* gate,
               const float* table, const int64_t* idx, int64_t nt, int64_t C, int64_t H, int64_t hd);
// mode 0: gx = rmsnorm_bwd(gx); 1: gx += rmsnorm_bwd(gn); 2: g = gx +
// rmsnorm_bwd(gn), g_res[l] += g.x, g_x0[l] += g.x0, gx = res[l] g.  gxb = bf16(gx).
// Modes 1 and 2 take gn either fp32 (gn) or bf16 (gnb), not both.
// partial: 2 * kNormBwdWaves floats (mode 2).
constexpr int kNormBwdWaves = 4096;
int32_t norm_bwd(hipStream_t st, int mode, float* gx, bf16* gxb, const float* gn, const float* x, const float* rms,
                 const float* x0, const float* res, int64_t layer, float* g_res, float* g_x0, float* partial,
                 int64_t rows, int64_t C, const bf16* gnb = nullptr);
int32_t to_bf16(hipStream_t st, bf16* out, const float* in, int64_t n);
// One matrix of a batched transpose: fp32 [rows, cols] at in + src becomes
// bf16 [cols, rows] at out + dst; tile0 = 64 x 64 tiles of the entries before.
struct TransposeEntry {
    int64_t src, dst, rows, cols, tile0;
};
// tab: n entries in device memory; tiles: total 64 x 64 tiles.
int32_t transpose_bf16(hipStream_t st, bf16* out, const float* in, const TransposeEntry* tab, int n,
                       int64_t tiles);
// D = rowsum(O * dO), dO stored as bf16.
int32_t precompute_d_mixed(hipStream_t st, float* d, const float* o, const bf16* g, int64_t rows, int64_t hd);

// ---- Muon (ar_optim.hip) ----
constexpr int kMuonMaxGroup = 48;
// lr factor sqrt(max(1, rows / cols)) of a [rows, cols] matrix.
double muon_lr_factor(int64_t rows, int64_t cols);
// Scratch (floats) for a group of n same-shape [rows, cols] matrices.
int64_t muon_scratch_elems(int64_t rows, int64_t cols, bool bf16, int64_t n);
// MuonState.step for n same-shape matrices at once (batched GEMMs).  With
// dsc set, the step's lr, momentum and weight decay are read from device
// memory (dsc[lr_i], dsc[mu_i], dsc[wd_i]) instead of the value arguments.
struct MuonDev {
    const float* dsc = nullptr;
    int lr_i = 0, mu_i = 0, wd_i = 0;
};
int32_t muon_group_step(hipStream_t st, float* const* params, const float* const* grads, float* const* mbufs, int n,
                        int64_t rows, int64_t cols, double initial_lr, double lrm, double momentum, double wd,
                        bool bf16, float* scratch, const MuonDev& dev = MuonDev());

}  // namespace ar

extern "C" {
// Stable sort of token ids (radix sort on the low end_bit bits).  With
// scratch == NULL only *scratch_needed is set.
int32_t ar_embedding_sort(ar_stream_t stream, uint32_t* sorted_ids, int32_t* sorted_tokens, const int64_t* indices,
                          int64_t num_tokens, int32_t end_bit, void* scratch, size_t scratch_bytes,
                          size_t* scratch_needed);
// embedding_bwd given the stable sort; partial: num_tokens * embd_dim floats.
int32_t ar_embedding_bwd_sorted(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                const uint32_t* sorted_ids, const int32_t* sorted_tokens, int64_t num_tokens,
                                int64_t embd_dim, float* partial);
}
