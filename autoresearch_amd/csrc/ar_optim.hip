// ar_optim.hip -- Muon (optimizer.mojo:255-342): Nesterov momentum ->
// Frobenius normalisation -> 5 Polar Express iterations -> cautious update,
// for a *group* of same-shape matrices at once.
//
// The reference runs ~27 launches per matrix, one matrix at a time (about
// 1,300 launches per step at depth 8, most of them 512x512 GEMMs that fill a
// fraction of the GPU).  Here every product of an iteration is one batched
// MFMA GEMM over the whole group (e.g. all 32 512x512 attention matrices),
// and the element-wise steps are multi-tensor kernels over the group:
// 18 launches per group per step.  A wide matrix (rows < cols) uses the
// A = X X^T / B @ X formulation directly through the GEMM operand layouts,
// exactly as the reference's wide branch (optimizer.mojo:297-303, 327-332).
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

namespace {

constexpr int kNormBlocks = 64;  // fixed per-matrix partial count (deterministic)

struct GroupTable {
    float* p[kMuonMaxGroup];
    const float* g[kMuonMaxGroup];
    float* m[kMuonMaxGroup];
};

inline int64_t align64(int64_t n) { return (n + 63) & ~int64_t(63); }

// The element-wise kernels run a float4 path (VEC) when every matrix of the
// group is 16-byte aligned and its size a multiple of 4 (all model shapes);
// the element order of each thread's sums is then 4 consecutive elements per
// step, still fixed for a given shape.
__device__ __forceinline__ float4 ld4v(const float* p, int64_t i4) { return reinterpret_cast<const float4*>(p)[i4]; }
__device__ __forceinline__ void st4v(float* p, int64_t i4, float4 v) { reinterpret_cast<float4*>(p)[i4] = v; }

// X_j = (1-mu) g + mu * (mu buf + (1-mu) g); buf updated (optimizer.mojo:132-146);
// partial[j][b] = this block's sum of X^2.
template <bool VEC>
__global__ void nesterov_multi_k(GroupTable t, float* X, int64_t size, float mu, const float* dmu, float* partial,
                                 int64_t rows, int64_t cols, int64_t cols_p) {
    __shared__ float red[4];
    if (dmu) mu = *dmu;
    const int j = blockIdx.y;
    const float* g = t.g[j];
    float* buf = t.m[j];
    float* x = X + (int64_t)j * size;
    float ss = 0.f;
    auto one = [&](float gv, float bv, float& mm, float& o) {
        mm = mu * bv + (1.0f - mu) * gv;
        o = (1.0f - mu) * gv + mu * mm;
        ss += o * o;
    };
    if constexpr (VEC) {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < size / 4;
             i += (int64_t)gridDim.x * blockDim.x) {
            const float4 gv = ld4v(g, i), bv = ld4v(buf, i);
            float4 mm, o;
            one(gv.x, bv.x, mm.x, o.x);
            one(gv.y, bv.y, mm.y, o.y);
            one(gv.z, bv.z, mm.z, o.z);
            one(gv.w, bv.w, mm.w, o.w);
            st4v(buf, i, mm);
            st4v(x, i, o);
        }
    } else {
        // X may be zero-padded to [rows_p, cols_p] (size = rows_p * cols_p);
        // g and buf are [rows, cols]
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < size;
             i += (int64_t)gridDim.x * blockDim.x) {
            const int64_t r = i / cols_p, c = i - r * cols_p;
            if (r < rows && c < cols) {
                const int64_t e = r * cols + c;
                float mm, o;
                one(g[e], buf[e], mm, o);
                buf[e] = mm;
                x[i] = o;
            } else {
                x[i] = 0.0f;
            }
        }
    }
    ss = block_sum(ss, red);
    if (threadIdx.x == 0) partial[j * kNormBlocks + blockIdx.x] = ss;
}

// X_j *= s_j with s_j = 1 / (||X_j||_F * 1.02 + 1e-6) (optimizer.mojo:178),
// the norm summed from the kNormBlocks (= one wave's lanes) partials of
// nesterov_multi_k in the same fixed order by every wave; Xb (if set) =
// bf16(X).
template <bool VEC>
__global__ void scale_multi_k(float* X, bf16* Xb, int64_t size, const float* partial) {
    static_assert(kNormBlocks == kWave, "one partial per lane");
    const int j = blockIdx.y;
    const float ss = wave_sum(partial[j * kNormBlocks + threadIdx.x % kWave]);
    const float sc = 1.0f / (sqrtf(ss) * 1.02f + 1e-6f);
    float* x = X + (int64_t)j * size;
    bf16* xb = Xb ? Xb + (int64_t)j * size : nullptr;
    if constexpr (VEC) {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < size / 4;
             i += (int64_t)gridDim.x * blockDim.x) {
            float4 v = ld4v(x, i);
            v = make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc);
            st4v(x, i, v);
            if (xb) {
                bf16x4 b;
                b[0] = (bf16)v.x;
                b[1] = (bf16)v.y;
                b[2] = (bf16)v.z;
                b[3] = (bf16)v.w;
                reinterpret_cast<bf16x4*>(xb)[i] = b;
            }
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < size;
             i += (int64_t)gridDim.x * blockDim.x) {
            const float v = x[i] * sc;
            x[i] = v;
            if (xb) xb[i] = (bf16)v;
        }
    }
}

// p -= lr (X + wd p [X p >= 0])  (optimizer.mojo:197-210)
__device__ __forceinline__ float cautious(float pv, float gv, float lr, float wd) {
    const float decay = (gv * pv) >= 0.0f ? wd * pv : 0.0f;
    return pv - lr * (gv + decay);
}
template <bool VEC>
__global__ void update_multi_k(GroupTable t, const float* X, int64_t size, float lr, float wd, const float* dlr,
                               const float* dwd, int64_t cols, int64_t xsize, int64_t cols_p) {
    if (dlr) {
        lr = *dlr;
        wd = *dwd;
    }
    const int j = blockIdx.y;
    float* p = t.p[j];
    const float* x = X + (int64_t)j * xsize;
    if constexpr (VEC) {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < size / 4;
             i += (int64_t)gridDim.x * blockDim.x) {
            const float4 pv = ld4v(p, i), gv = ld4v(x, i);
            st4v(p, i, make_float4(cautious(pv.x, gv.x, lr, wd), cautious(pv.y, gv.y, lr, wd),
                                   cautious(pv.z, gv.z, lr, wd), cautious(pv.w, gv.w, lr, wd)));
        }
    } else {
        // p is [rows, cols] (size = rows * cols); X may be padded to cols_p columns
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < size;
             i += (int64_t)gridDim.x * blockDim.x) {
            const int64_t r = i / cols, c = i - r * cols;
            p[i] = cautious(p[i], x[r * cols_p + c], lr, wd);
        }
    }
}

}  // namespace

// optimizer.mojo:266-268: lr * sqrt(max(1, rows / cols))
double muon_lr_factor(int64_t rows, int64_t cols) {
    const double aspect = (double)rows / (double)cols;
    return aspect > 1.0 ? sqrt(aspect) : 1.0;
}

int64_t muon_scratch_elems(int64_t rows, int64_t cols, bool bf16, int64_t n) {
    rows = (rows + 7) & ~int64_t(7);  // the products' zero-padded shape
    cols = (cols + 7) & ~int64_t(7);
    const int64_t size = rows * cols;
    const int64_t small = rows >= cols ? cols : rows;
    const int64_t f32 = align64(n * kNormBlocks) + 2 * align64(n * size) + 2 * align64(n * small * small);
    // bf16 operand copies of X, Y, A, Bm (two per float)
    return bf16 ? f32 + 2 * align64((n * size + 1) / 2) + 2 * align64((n * small * small + 1) / 2) : f32;
}

int32_t muon_group_step(hipStream_t st, float* const* params, const float* const* grads, float* const* mbufs, int n,
                        int64_t rows, int64_t cols, double initial_lr, double lrm, double momentum, double wd,
                        bool bf16, float* scratch, const MuonDev& dev) {
    if (n <= 0) return AR_OK;
    if (n > kMuonMaxGroup) return set_error(AR_EINVAL, "muon: group of %d > %d matrices", n, kMuonMaxGroup);
    // The products work on X zero-padded to multiples of 8 rows and columns
    // (the batched GEMMs' 16-byte operand rows).  Zero rows and columns stay
    // zero through every Polar Express iteration (A = X^T X, B = b A + c A^2
    // and X' = a X + X B are zero wherever X is) and add nothing to the
    // Frobenius norm; the tall / wide choice and the lr factor are the
    // unpadded shape's (optimizer.mojo:266-268, 297-303).
    const int64_t psize = rows * cols;
    const bool tall = rows >= cols;
    rows = (rows + 7) & ~int64_t(7);
    const int64_t cols_u = cols;
    cols = (cols + 7) & ~int64_t(7);
    const int64_t size = rows * cols;
    const int64_t sm = tall ? cols : rows;
    const int64_t ss = sm * sm;
    float* partial = scratch;
    float* X = partial + align64(n * kNormBlocks);
    float* Y = X + align64(n * size);
    float* A = Y + align64(n * size);
    float* Bm = A + align64(n * ss);
    // bf16 step: the products read bf16 copies of their operands, written by
    // the kernel that produces each operand (the same rounding the fp32-operand
    // products apply on load, so the results are the same)
    ::ar::bf16* Xb = bf16 ? reinterpret_cast<::ar::bf16*>(Bm + align64(n * ss)) : nullptr;
    ::ar::bf16* Yb = bf16 ? Xb + 2 * align64((n * size + 1) / 2) : nullptr;
    ::ar::bf16* Ab = bf16 ? Yb + 2 * align64((n * size + 1) / 2) : nullptr;
    ::ar::bf16* Bmb = bf16 ? Ab + 2 * align64((n * ss + 1) / 2) : nullptr;

    GroupTable t{};
    bool vec = size == psize && size % 4 == 0;
    for (int j = 0; j < n; ++j) {
        t.p[j] = params[j];
        t.g[j] = grads[j];
        t.m[j] = mbufs[j];
        vec = vec && ((reinterpret_cast<uintptr_t>(params[j]) | reinterpret_cast<uintptr_t>(grads[j]) |
                       reinterpret_cast<uintptr_t>(mbufs[j])) & 15) == 0;
    }
    const int64_t rows_u = psize / cols_u;
    const float lr = (float)(initial_lr * lrm * muon_lr_factor(rows_u, cols_u));
    const dim3 eg(kNormBlocks, n);
    const float* dmu = dev.dsc ? dev.dsc + dev.mu_i : nullptr;
    if (vec) nesterov_multi_k<true><<<eg, 256, 0, st>>>(t, X, size, (float)momentum, dmu, partial, rows, cols, cols);
    else nesterov_multi_k<false><<<eg, 256, 0, st>>>(t, X, size, (float)momentum, dmu, partial, rows_u, cols_u, cols);
    if (vec) scale_multi_k<true><<<eg, 256, 0, st>>>(X, Xb, size, partial);
    else scale_multi_k<false><<<eg, 256, 0, st>>>(X, Xb, size, partial);
    int32_t r = check_launch("muon: normalise");
    if (r) return r;
    ar_stream_t s = reinterpret_cast<ar_stream_t>(st);
    // Each iteration's combinations ride on the product before them:
    // Bm = cb A + cc (A A) in the A.A epilogue, and X' = ca X + (B X or X B)
    // in the last product's epilogue, written to the other of X / Y.
    // A = X^T X (or X X^T) is symmetric bit for bit: entries (i, j) and
    // (j, i) sum the same products in the same k order.  So is A A, and with
    // it Bm.  A symmetric operand read as the B side of a product is read
    // K-major (its own transpose), the GEMM's faster LDS path, with the same
    // values in the same order.
    float* Xc = X;
    float* Yc = Y;
    ::ar::bf16* Xbc = Xb;
    ::ar::bf16* Ybc = Yb;
    for (int it = 0; it < 5 && bf16; ++it) {
        const float ca = (float)kPolarA[it], cb = (float)kPolarB[it], cc = (float)kPolarC[it];
        if (tall)
            r = gemm_batched_bf16(st, false, false, A, Ab, Xbc, Xbc, cols, cols, rows, cols, cols, cols, n, size, size,
                                  ss);
        else
            r = gemm_batched_bf16(st, true, true, A, Ab, Xbc, Xbc, rows, rows, cols, cols, cols, rows, n, size, size,
                                  ss);
        if (r) return r;
        // only the bf16 copy of Bm is read (as the next product's operand),
        // and the last iteration's X is read in fp32 only (the update)
        if ((r = gemm_batched_bf16(st, true, true, nullptr, Bmb, Ab, Ab, sm, sm, sm, sm, sm, sm, n, ss, ss, ss, A,
                                   cc, cb)))
            return r;
        ::ar::bf16* const Yout = it < 4 ? Ybc : nullptr;
        if (tall)
            r = gemm_batched_bf16(st, true, true, Yc, Yout, Xbc, Bmb, rows, cols, cols, cols, cols, cols, n, size, ss,
                                  size, Xc, 1.0f, ca);
        else
            r = gemm_batched_bf16(st, true, false, Yc, Yout, Bmb, Xbc, rows, cols, rows, rows, cols, cols, n, ss, size,
                                  size, Xc, 1.0f, ca);
        if (r) return r;
        float* tmp = Xc;
        Xc = Yc;
        Yc = tmp;
        ::ar::bf16* tb = Xbc;
        Xbc = Ybc;
        Ybc = tb;
    }
    for (int it = 0; it < 5 && !bf16; ++it) {
        const float ca = (float)kPolarA[it], cb = (float)kPolarB[it], cc = (float)kPolarC[it];
        if (tall)  // A = X^T X : mo = c1, no = c2, r = row (both operands MN-major)
            r = gemm_batched_f32(st, bf16, false, false, A, Xc, Xc, cols, cols, rows, cols, cols, cols, n, size, size,
                                 ss);
        else  // A = X X^T : mo = r1, no = r2, r = col (both K-major)
            r = gemm_batched_f32(st, bf16, true, true, A, Xc, Xc, rows, rows, cols, cols, cols, rows, n, size, size,
                                 ss);
        if (r) return r;
        // Bm = cb A + cc (A @ A)
        if ((r = gemm_batched_f32(st, bf16, true, true, Bm, A, A, sm, sm, sm, sm, sm, sm, n, ss, ss, ss, A, cc, cb)))
            return r;
        if (tall)  // X' = ca X + X @ B (B symmetric: read K-major)
            r = gemm_batched_f32(st, bf16, true, true, Yc, Xc, Bm, rows, cols, cols, cols, cols, cols, n, size, ss,
                                 size, Xc, 1.0f, ca);
        else  // X' = ca X + B @ X
            r = gemm_batched_f32(st, bf16, true, false, Yc, Bm, Xc, rows, cols, rows, rows, cols, cols, n, ss, size,
                                 size, Xc, 1.0f, ca);
        if (r) return r;
        float* tmp = Xc;
        Xc = Yc;
        Yc = tmp;
    }
    const float* dlr = dev.dsc ? dev.dsc + dev.lr_i : nullptr;
    const float* dwd = dev.dsc ? dev.dsc + dev.wd_i : nullptr;
    if (vec) update_multi_k<true><<<eg, 256, 0, st>>>(t, Xc, size, lr, (float)wd, dlr, dwd, cols, size, cols);
    else update_multi_k<false><<<eg, 256, 0, st>>>(t, Xc, psize, lr, (float)wd, dlr, dwd, cols_u, size, cols);
    return check_launch("muon: update");
}

}  // namespace ar

// optimizer.mojo:255-342 for one matrix (a group of one).
extern "C" int32_t ar_muon_step(ar_stream_t stream, float* params, float* grads, float* momentum_buf, int64_t rows,
                                int64_t cols, double initial_lr, double lr_multiplier, double momentum,
                                double weight_decay, int32_t precision) {
    AR_CHECK_ARG(params && grads && momentum_buf, "muon_step: null pointer");
    AR_CHECK_ARG(rows > 0 && cols > 0, "muon_step: bad shape");
    const bool bf = precision == AR_PREC_BF16;
    int32_t st;
    float* scratch = (float*)ar::workspace(ar::S(stream), (size_t)ar::muon_scratch_elems(rows, cols, bf, 1) * sizeof(float), &st);
    if (!scratch) return st;
    float* p[1] = {params};
    const float* g[1] = {grads};
    float* m[1] = {momentum_buf};
    return ar::muon_group_step(ar::S(stream), p, g, m, 1, rows, cols, initial_lr, lr_multiplier, momentum,
                               weight_decay, bf, scratch);
}
