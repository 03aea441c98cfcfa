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
int64_t gemm_auto_splits(int layout, bool bf16, int64_t M, int64_t N, int64_t K);
int64_t gemm_partial_elems(int layout, int64_t M, int64_t N, int64_t K, int64_t splits);
int32_t gemm_f32(hipStream_t st, int layout, bool bf16, float* C, const float* X, const float* W, int64_t M,
                 int64_t N, int64_t K, bool accumulate, int64_t splits, float* partial);
// Same, with each operand stored as bf16 (flag set) or fp32; bf16 compute.
int32_t gemm_bf16io(hipStream_t st, int layout, void* C, int c_bf16, const void* X, int x_bf16, const void* W,
                    int w_bf16, int64_t M, int64_t N, int64_t K, bool accumulate, int64_t splits, float* partial);
// NT (layout 0) / NN (layout 1) GEMM with a fused epilogue, bf16 compute:
// epi 3 ADD (C = aux + acc, aux fp32), 4 RELU2 (C = acc, aux_out = relu(acc)^2),
// 5 SOFTCAP (C = cap tanh(acc/cap)), 6 RELU2_BWD (C = aux > 0 ? 2 aux acc : 0).
enum { GEMM_EPI_ADD = 3, GEMM_EPI_RELU2 = 4, GEMM_EPI_SOFTCAP = 5, GEMM_EPI_RELU2_BWD = 6 };
int32_t gemm_epilogue(hipStream_t st, int layout, int epi, void* C, int c_bf16, const void* X, int x_bf16,
                      const void* W, int w_bf16, int64_t M, int64_t N, int64_t K, const void* aux, void* aux_out,
                      float cap);
// Batched GEMM-space form: C_b[mo,no] = sum_r A_b(mo,r) B_b(no,r); ak / bk
// select K-major (r contiguous, row stride lda/ldb) vs MN-major storage.
int32_t gemm_batched_f32(hipStream_t st, bool bf16, bool ak, bool bk, float* C, const float* A, const float* B,
                         int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                         int64_t sA, int64_t sB, int64_t sC);

// ---- reductions (ar_reduce.hip) ----
constexpr int kSumBlocks = 512;
// mode_in: 0 sum a, 1 sum a*a, 2 sum a*b.  mode_out: 0 out[idx] = s/n,
// 1 out[idx] += s, 2 out[0] = 1/(sqrt(s)*1.02 + 1e-6).  partial: kSumBlocks floats.
int32_t fixed_sum(hipStream_t st, float* out, const float* a, const float* b, int64_t n, int mode_in, int mode_out,
                  int64_t idx, float* partial);
// data /= (||data||_F * 1.02 + 1e-6); scratch: kSumBlocks + 1 floats.
int32_t frob_normalize(hipStream_t st, float* data, int64_t n, float* scratch);
constexpr int kGateBlocks = 256;
// partial: kGateBlocks * n_kv_head * gate_channels floats.
int32_t ve_gate_bwd(hipStream_t st, float* gx, float* gw, const float* ggate, const float* gate, const float* xn,
                    const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C, float* partial);

// ---- attention (ar_attention.hip) ----
enum class AttnOp { FWD, DQ, DKV };
template <bool BF16, typename TIN>
int32_t attn_dispatch(hipStream_t st, AttnOp op, float* o1, float* o2, const TIN* q, const TIN* k, const TIN* v,
                      const TIN* dout, const float* lse, const float* dbuf, int64_t B, int64_t T, int64_t H,
                      int64_t HD, int64_t window);

// ---- element-wise (ar_elementwise.hip) ----
int32_t rope(hipStream_t st, float* out, const float* in, const float* cos_t, const float* sin_t, int64_t nt,
             int64_t nh, int64_t hd, int64_t period, bool inverse);

// ---- Muon (ar_optim.hip) ----
constexpr int kMuonMaxGroup = 48;
// Scratch (floats) for a group of n same-shape [rows, cols] matrices.
int64_t muon_scratch_elems(int64_t rows, int64_t cols, bool bf16, int64_t n);
// MuonState.step for n same-shape matrices at once (batched GEMMs).
int32_t muon_group_step(hipStream_t st, float* const* params, const float* const* grads, float* const* mbufs, int n,
                        int64_t rows, int64_t cols, double initial_lr, double lrm, double momentum, double wd,
                        bool bf16, float* scratch);

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
