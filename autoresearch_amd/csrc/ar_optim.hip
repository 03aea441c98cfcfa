// ar_optim.hip -- Muon (optimizer.mojo:255-342): Nesterov momentum ->
// Frobenius normalisation -> 5 Polar Express iterations -> cautious update,
// built on the MFMA GEMMs.
#include <math.h>

#include "ar_internal.hpp"

namespace ar {

// config.mojo:93-112
static const double kPolarA[5] = {8.156554524902461, 4.042929935166739, 3.8916678022926607, 3.285753657755655,
                                  2.3465413258596377};
static const double kPolarB[5] = {-22.48329292557795, -2.808917465908714, -2.772484153217685,
                                  -2.3681294933425376, -1.7097828382687081};
static const double kPolarC[5] = {15.878769915207462, 0.5000178451051316, 0.5060648178503393,
                                  0.46449024233003106, 0.42323551169305323};

static inline int64_t align64(int64_t n) { return (n + 63) & ~int64_t(63); }

int64_t muon_scratch_elems(int64_t rows, int64_t cols, bool bf16) {
    const int64_t size = rows * cols;
    const int64_t small = rows >= cols ? cols : rows;
    int64_t gram_partial = 0;
    if (rows >= cols) gram_partial = gemm_partial_elems(2, rows, cols, cols, gemm_auto_splits(2, bf16, rows, cols, cols));
    return align64(kSumBlocks + 64) + align64(size) + 3 * align64(small * small) + align64(gram_partial);
}

int32_t muon_step(hipStream_t st, float* params, float* grads, float* momentum_buf, int64_t rows, int64_t cols,
                  double initial_lr, double lrm, double momentum, double wd, bool bf16, float* scratch) {
    const int64_t size = rows * cols;
    const int64_t small = rows >= cols ? cols : rows;
    const int64_t ss = small * small;
    const bool tall = rows >= cols;
    float* sum_scratch = scratch;
    float* X = sum_scratch + align64(kSumBlocks + 64);
    float* A = X + align64(size);
    float* AA = A + align64(ss);
    float* Bm = AA + align64(ss);
    float* partial = Bm + align64(ss);
    ar_stream_t s = reinterpret_cast<ar_stream_t>(st);

    const double aspect = (double)rows / (double)cols;
    const float lr = (float)(initial_lr * lrm * (aspect > 1.0 ? sqrt(aspect) : 1.0));
    int32_t r;
    if ((r = ar_nesterov_momentum(s, X, grads, momentum_buf, (float)momentum, size))) return r;
    if ((r = frob_normalize(st, X, size, sum_scratch))) return r;
    for (int it = 0; it < 5; ++it) {
        const float ca = (float)kPolarA[it], cb = (float)kPolarB[it], cc = (float)kPolarC[it];
        if (tall)  // A = X^T X (the reference zero-fills then accumulates; storing is identical)
            r = gemm_f32(st, 2, bf16, A, X, X, rows, cols, cols, false, 0, partial);
        else  // A = X X^T
            r = gemm_f32(st, 0, bf16, A, X, X, rows, rows, cols, false, 1, nullptr);
        if (r) return r;
        if ((r = gemm_f32(st, 1, bf16, AA, A, A, small, small, small, false, 1, nullptr))) return r;  // A @ A
        if ((r = ar_scale_add(s, Bm, A, AA, cb, cc, ss))) return r;
        if (tall)  // grads := X @ B
            r = gemm_f32(st, 1, bf16, grads, X, Bm, rows, cols, cols, false, 1, nullptr);
        else  // grads := B @ X
            r = gemm_f32(st, 1, bf16, grads, Bm, X, rows, rows, cols, false, 1, nullptr);
        if (r) return r;
        if ((r = ar_scale_add(s, X, X, grads, ca, 1.0f, size))) return r;
    }
    return ar_muon_update(s, params, X, lr, (float)wd, size);
}

}  // namespace ar

extern "C" int32_t ar_muon_step(ar_stream_t stream, float* params, float* grads, float* momentum_buf, int64_t rows,
                                int64_t cols, double initial_lr, double lr_multiplier, double momentum,
                                double weight_decay, int32_t precision) {
    AR_CHECK_ARG(params && grads && momentum_buf, "muon_step: null pointer");
    AR_CHECK_ARG(rows > 0 && cols > 0 && rows % 8 == 0 && cols % 8 == 0, "muon_step: rows, cols must be multiples of 8");
    const bool bf = precision == AR_PREC_BF16;
    int32_t st;
    float* scratch = (float*)ar::workspace((size_t)ar::muon_scratch_elems(rows, cols, bf) * sizeof(float), &st);
    if (!scratch) return st;
    return ar::muon_step(ar::S(stream), params, grads, momentum_buf, rows, cols, initial_lr, lr_multiplier, momentum,
                         weight_decay, bf, scratch);
}
