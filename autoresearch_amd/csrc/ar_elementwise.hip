// ar_elementwise.hip -- bandwidth-bound element-wise kernels of the training
// step: gathers, RoPE, ReLU^2, softcap, residual and scaling kernels, the
// element-wise optimizer updates and the weight-init kernels.
//
// Every kernel is a grid-stride loop over float4 (16 B per lane, 1 KiB per
// wave per access) when all operands are 16-byte aligned and the size is a
// multiple of 4, and over scalars otherwise.  All are HBM-bound: their
// roofline is 8 TB/s against the bytes each reads and writes once.
#include <math.h>

#include "ar_internal.hpp"

using namespace ar;

namespace {

constexpr int kBlock = 256;

__host__ __device__ inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__device__ __forceinline__ int64_t gtid() { return (int64_t)blockIdx.x * blockDim.x + threadIdx.x; }
__device__ __forceinline__ int64_t gstride() { return (int64_t)gridDim.x * blockDim.x; }

// Applies f(i) for i in [0, n) where f processes elements [4i, 4i+4) when VEC
// and element i otherwise.
#define AR_GRID_LOOP(i, n) for (int64_t i = gtid(); i < (n); i += gstride())

template <bool VEC>
inline unsigned grid_for(int64_t n) {
    return flat_grid(VEC ? cdiv(n, 4) : n, kBlock * 4);
}

// ---------------- K1 embedding_fwd (ops.mojo:41-55) ----------------
// One wave per token row: the id is read once per row, the row is copied
// with float4 accesses.
__global__ void embedding_fwd_k(float* out, const float* weight, const int64_t* idx, int64_t n, int64_t dim) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
    for (int64_t t = wave; t < n; t += nwaves) {
        const int64_t v = idx[t];
        const float* src = weight + v * dim;
        float* dst = out + t * dim;
        if ((dim & 3) == 0 && al16(src) && al16(dst)) {
            for (int64_t d = lane; d < dim / 4; d += kWave)
                reinterpret_cast<float4*>(dst)[d] = reinterpret_cast<const float4*>(src)[d];
        } else {
            for (int64_t d = lane; d < dim; d += kWave) dst[d] = src[d];
        }
    }
}

// ---------------- K4 / K22 RoPE (ops.mojo:209-238, 1091-1120) ----------------
// Table row = (flat token index) % period; period = num_tokens reproduces the
// reference's flat indexing.  sign = +1 forward, -1 backward (inverse rotation).
__global__ void rope_k(float* out, const float* in, const float* cos_t, const float* sin_t, int64_t num_tokens,
                       int64_t heads, int64_t head_dim, int64_t period, float sign) {
    const int64_t half = head_dim / 2;
    const int64_t total = num_tokens * heads * half;
    AR_GRID_LOOP(i, total) {
        const int64_t th = i / half, d = i % half;
        const int64_t tok = (th / heads) % period;
        const float* x = in + th * head_dim;
        const float x1 = x[d], x2 = x[half + d];
        const float c = cos_t[tok * half + d];
        const float s = sign * sin_t[tok * half + d];
        float* y = out + th * head_dim;
        y[d] = x1 * c + x2 * s;
        y[half + d] = x1 * (-s) + x2 * c;
    }
}

// ---------------- K9 / K23 ReLU^2 ----------------
template <bool VEC>
__global__ void relu2_fwd_k(float* out, const float* in, int64_t n) {
    if (VEC) {
        AR_GRID_LOOP(i, n / 4) {
            float4 x = reinterpret_cast<const float4*>(in)[i];
            x.x = x.x > 0.f ? x.x * x.x : 0.f;
            x.y = x.y > 0.f ? x.y * x.y : 0.f;
            x.z = x.z > 0.f ? x.z * x.z : 0.f;
            x.w = x.w > 0.f ? x.w * x.w : 0.f;
            reinterpret_cast<float4*>(out)[i] = x;
        }
    } else {
        AR_GRID_LOOP(i, n) {
            float x = in[i];
            float r = x > 0.f ? x : 0.f;
            out[i] = r * r;
        }
    }
}

template <bool VEC>
__global__ void relu2_bwd_k(float* dx, const float* dy, const float* x, int64_t n) {
    if (VEC) {
        AR_GRID_LOOP(i, n / 4) {
            float4 a = reinterpret_cast<const float4*>(x)[i];
            float4 g = reinterpret_cast<const float4*>(dy)[i];
            float4 r;
            r.x = a.x > 0.f ? 2.f * a.x * g.x : 0.f;
            r.y = a.y > 0.f ? 2.f * a.y * g.y : 0.f;
            r.z = a.z > 0.f ? 2.f * a.z * g.z : 0.f;
            r.w = a.w > 0.f ? 2.f * a.w * g.w : 0.f;
            reinterpret_cast<float4*>(dx)[i] = r;
        }
    } else {
        AR_GRID_LOOP(i, n) dx[i] = x[i] > 0.f ? 2.f * x[i] * dy[i] : 0.f;
    }
}

// ---------------- K10 softcap ----------------
__global__ void softcap_k(float* out, const float* in, float cap, int64_t n) {
    AR_GRID_LOOP(i, n) out[i] = cap * tanhf(in[i] / cap);
}

// ---------------- K12 ve_apply_fwd ----------------
__global__ void ve_apply_k(float* v, const float* gate, const float* ve, int64_t n, int64_t head_dim) {
    AR_GRID_LOOP(i, n) v[i] += gate[i / head_dim] * ve[i];
}

// ---------------- K13 add_residual / K33 scale_add / K14 scaled_add ----------------
template <bool VEC>
__global__ void axpby_k(float* out, const float* a, const float* b, float sa, float sb, const float* psa,
                        const float* psb, int64_t idx, int64_t n, int plain_add) {
    // plain_add: out = a + b exactly (no multiply), as ops.mojo:576.
    if (psa) {
        sa = psa[idx];
        sb = psb[idx];
    }
    if (VEC) {
        AR_GRID_LOOP(i, n / 4) {
            float4 x = reinterpret_cast<const float4*>(a)[i];
            float4 y = reinterpret_cast<const float4*>(b)[i];
            float4 r;
            if (plain_add) {
                r.x = x.x + y.x; r.y = x.y + y.y; r.z = x.z + y.z; r.w = x.w + y.w;
            } else {
                r.x = sa * x.x + sb * y.x; r.y = sa * x.y + sb * y.y;
                r.z = sa * x.z + sb * y.z; r.w = sa * x.w + sb * y.w;
            }
            reinterpret_cast<float4*>(out)[i] = r;
        }
    } else {
        AR_GRID_LOOP(i, n) out[i] = plain_add ? a[i] + b[i] : sa * a[i] + sb * b[i];
    }
}

// ---------------- K25 scaled_add_bwd ----------------
template <bool VEC>
__global__ void scaled_add_bwd_k(float* ga, float* gb, const float* g, const float* sa, const float* sb,
                                 int64_t idx, int64_t n) {
    const float s1 = sa[idx], s2 = sb[idx];
    if (VEC) {
        AR_GRID_LOOP(i, n / 4) {
            float4 x = reinterpret_cast<const float4*>(g)[i];
            reinterpret_cast<float4*>(gb)[i] = make_float4(s2 * x.x, s2 * x.y, s2 * x.z, s2 * x.w);
            reinterpret_cast<float4*>(ga)[i] = make_float4(s1 * x.x, s1 * x.y, s1 * x.z, s1 * x.w);
        }
    } else {
        AR_GRID_LOOP(i, n) {
            float x = g[i];
            gb[i] = s2 * x;
            ga[i] = s1 * x;
        }
    }
}

// ---------------- K29 / K37 / K38 fill ----------------
template <bool VEC>
__global__ void fill_k(float* out, float value, int64_t n) {
    if (VEC) {
        AR_GRID_LOOP(i, n / 4) reinterpret_cast<float4*>(out)[i] = make_float4(value, value, value, value);
    } else {
        AR_GRID_LOOP(i, n) out[i] = value;
    }
}

// ---------------- K30 AdamW (optimizer.mojo:27-57) ----------------
__global__ void adamw_k(float* p, const float* g, float* m, float* v, float lr, float b1, float b2, float eps,
                        float wd, float bc1, float bc2, int64_t n) {
    AR_GRID_LOOP(i, n) {
        float pv = p[i], gv = g[i];
        pv = pv * (1.0f - lr * wd);
        float mm = b1 * m[i] + (1.0f - b1) * gv;
        m[i] = mm;
        float vv = b2 * v[i] + (1.0f - b2) * gv * gv;
        v[i] = vv;
        p[i] = pv - lr * (mm / bc1) / (sqrtf(vv / bc2) + eps);
    }
}

// adamw_k with the step-dependent scalars (lr, 1 - b1^t, 1 - b2^t) read from
// device memory (sc[lr_i], sc[bc1_i], sc[bc2_i]) so a recorded HIP graph
// picks up each step's values.
__global__ void adamw_dev_k(float* p, const float* g, float* m, float* v, const float* sc, int lr_i, int bc1_i,
                            int bc2_i, float b1, float b2, float eps, float wd, int64_t n) {
    const float lr = sc[lr_i], bc1 = sc[bc1_i], bc2 = sc[bc2_i];
    AR_GRID_LOOP(i, n) {
        float pv = p[i], gv = g[i];
        pv = pv * (1.0f - lr * wd);
        float mm = b1 * m[i] + (1.0f - b1) * gv;
        m[i] = mm;
        float vv = b2 * v[i] + (1.0f - b2) * gv * gv;
        v[i] = vv;
        p[i] = pv - lr * (mm / bc1) / (sqrtf(vv / bc2) + eps);
    }
}

// adamw_dev_k over several tensors of one set of arenas (p, g, m, v at the
// same element offsets) in one launch: block b updates 1024 elements of the
// tensor whose block range holds b, with that tensor's lr, bias correction
// and beta1.  Per element the arithmetic is adamw_dev_k's.
__global__ __launch_bounds__(256) void adamw_multi_k(AdamTable t, float* p, const float* g, float* m, float* v,
                                                     const float* sc, int bc2_i, float b2, float eps, float wd) {
    const int64_t bid = blockIdx.x;
    int j = 0;
    while (j + 1 < t.n && bid >= t.blk0[j + 1]) ++j;
    const float lr = sc[t.lr_i[j]], bc1 = sc[t.bc1_i[j]], bc2 = sc[bc2_i], b1 = t.b1[j];
    const int64_t off = t.off[j], size = t.size[j];
    const int64_t i0 = (bid - t.blk0[j]) * 1024 + threadIdx.x * 4;
    auto one = [&](float& pv, float gv, float& mm, float& vv) {
        pv = pv * (1.0f - lr * wd);
        mm = b1 * mm + (1.0f - b1) * gv;
        vv = b2 * vv + (1.0f - b2) * gv * gv;
        pv = pv - lr * (mm / bc1) / (sqrtf(vv / bc2) + eps);
    };
    if (i0 + 4 <= size && (off & 3) == 0) {
        float4* const p4 = reinterpret_cast<float4*>(p + off + i0);
        float4* const m4 = reinterpret_cast<float4*>(m + off + i0);
        float4* const v4 = reinterpret_cast<float4*>(v + off + i0);
        float4 pv = *p4, mm = *m4, vv = *v4;
        const float4 gv = *reinterpret_cast<const float4*>(g + off + i0);
        one(pv.x, gv.x, mm.x, vv.x);
        one(pv.y, gv.y, mm.y, vv.y);
        one(pv.z, gv.z, mm.z, vv.z);
        one(pv.w, gv.w, mm.w, vv.w);
        *m4 = mm;
        *v4 = vv;
        *p4 = pv;
    } else {
        for (int64_t i = i0; i < i0 + 4 && i < size; ++i) {
            float pv = p[off + i], mm = m[off + i], vv = v[off + i];
            one(pv, g[off + i], mm, vv);
            m[off + i] = mm;
            v[off + i] = vv;
            p[off + i] = pv;
        }
    }
}

// ---------------- K31 Nesterov (optimizer.mojo:132-146) ----------------
__global__ void nesterov_k(float* out, const float* g, float* buf, float mu, int64_t n) {
    AR_GRID_LOOP(i, n) {
        float gv = g[i];
        float mm = mu * buf[i] + (1.0f - mu) * gv;
        buf[i] = mm;
        out[i] = (1.0f - mu) * gv + mu * mm;
    }
}

// ---------------- K34 cautious Muon update (optimizer.mojo:197-210) ----------------
__global__ void muon_update_k(float* p, const float* g, float lr, float wd, int64_t n) {
    AR_GRID_LOOP(i, n) {
        float pv = p[i], gv = g[i];
        float decay = (gv * pv) >= 0.0f ? wd * pv : 0.0f;
        p[i] = pv - lr * (gv + decay);
    }
}

// ---------------- K35 / K36 init PRNG (model.mojo:86-134) ----------------
__device__ __forceinline__ uint64_t xs_mix(uint64_t s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s;
}

// Contraction is off for the init kernels so every product and sum rounds
// where the reference expression does (hipcc otherwise fuses lo + u*span).
__global__ void fill_normal_k(float* out, uint64_t seed, float std_, int64_t n) {
#pragma clang fp contract(off)
    const float PI = 3.14159265358979323846f;
    AR_GRID_LOOP(i, n) {
        uint64_t st = seed + (uint64_t)i * 6364136223846793005ULL + 1442695040888963407ULL;
        st = xs_mix(st);
        float u1 = (float)(st & 0xFFFFFFULL) / 16777216.0f + 1e-10f;
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        st = xs_mix(st);
        float u2 = (float)(st & 0xFFFFFFULL) / 16777216.0f;
        float z = sqrtf(-2.0f * logf(u1)) * cosf(2.0f * PI * u2);
        out[i] = z * std_;
    }
}

__global__ void fill_uniform_k(float* out, uint64_t seed, float lo, float hi, int64_t n) {
#pragma clang fp contract(off)
    AR_GRID_LOOP(i, n) {
        uint64_t st = seed + (uint64_t)i * 6364136223846793005ULL + 1442695040888963407ULL;
        st = xs_mix(st);
        float u = (float)(st & 0xFFFFFFULL) / 16777216.0f;
        out[i] = lo + u * (hi - lo);
    }
}

}  // namespace

// =====================================================================
// C ABI
// =====================================================================

#define AR_ENSURE(p) AR_CHECK_ARG((p) != nullptr, "%s: null pointer", __func__)
#define AR_NONNEG(n) AR_CHECK_ARG((n) >= 0, "%s: negative size", __func__)

extern "C" int32_t ar_embedding_fwd(ar_stream_t stream, float* output, const float* weight,
                                    const int64_t* indices, int64_t num_tokens, int64_t embd_dim) {
    AR_ENSURE(output); AR_ENSURE(weight); AR_ENSURE(indices);
    AR_CHECK_ARG(num_tokens >= 0 && embd_dim > 0, "embedding_fwd: bad shape");
    if (num_tokens == 0) return AR_OK;
    unsigned grid = flat_grid(num_tokens, kBlock / kWave);
    embedding_fwd_k<<<grid, kBlock, 0, S(stream)>>>(output, weight, indices, num_tokens, embd_dim);
    return AR_LAUNCH_CHECK("embedding_fwd");
}

static int32_t rope_launch(ar_stream_t stream, float* out, const float* in, const float* c, const float* s,
                           int64_t nt, int64_t nh, int64_t hd, int64_t period, float sign, const char* nm) {
    AR_CHECK_ARG(out && in && c && s, "%s: null pointer", nm);
    AR_CHECK_ARG(nt >= 0 && nh > 0 && hd > 0 && hd % 2 == 0 && period > 0, "%s: bad shape", nm);
    if (nt == 0) return AR_OK;
    rope_k<<<flat_grid(nt * nh * hd / 2, kBlock * 4), kBlock, 0, S(stream)>>>(out, in, c, s, nt, nh, hd, period,
                                                                                 sign);
    return AR_LAUNCH_CHECK(nm);
}

extern "C" int32_t ar_rope_fwd(ar_stream_t stream, float* output, const float* input, const float* cos_buf,
                               const float* sin_buf, int64_t num_tokens, int64_t num_heads, int64_t head_dim) {
    return rope_launch(stream, output, input, cos_buf, sin_buf, num_tokens, num_heads, head_dim,
                       num_tokens > 0 ? num_tokens : 1, 1.0f, "rope_fwd");
}

extern "C" int32_t ar_rope_bwd(ar_stream_t stream, float* grad_input, const float* grad_output, const float* cos_buf,
                               const float* sin_buf, int64_t num_tokens, int64_t num_heads, int64_t head_dim) {
    return rope_launch(stream, grad_input, grad_output, cos_buf, sin_buf, num_tokens, num_heads, head_dim,
                       num_tokens > 0 ? num_tokens : 1, -1.0f, "rope_bwd");
}

// Table row = flat token % period (period = T gives per-sequence positions).
int32_t ar::rope(hipStream_t st, float* out, const float* in, const float* cos_t, const float* sin_t, int64_t nt,
                 int64_t nh, int64_t hd, int64_t period, bool inverse) {
    return rope_launch(reinterpret_cast<ar_stream_t>(st), out, in, cos_t, sin_t, nt, nh, hd, period,
                       inverse ? -1.0f : 1.0f, "rope");
}

extern "C" int32_t ar_relu_squared_fwd(ar_stream_t stream, float* output, const float* input, int64_t size) {
    AR_ENSURE(output); AR_ENSURE(input); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    if (size % 4 == 0 && al16(output) && al16(input))
        relu2_fwd_k<true><<<grid_for<true>(size), kBlock, 0, S(stream)>>>(output, input, size);
    else
        relu2_fwd_k<false><<<grid_for<false>(size), kBlock, 0, S(stream)>>>(output, input, size);
    return AR_LAUNCH_CHECK("relu_squared_fwd");
}

extern "C" int32_t ar_relu_squared_bwd(ar_stream_t stream, float* grad_input, const float* grad_output,
                                       const float* input, int64_t size) {
    AR_ENSURE(grad_input); AR_ENSURE(grad_output); AR_ENSURE(input); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    if (size % 4 == 0 && al16(grad_input) && al16(grad_output) && al16(input))
        relu2_bwd_k<true><<<grid_for<true>(size), kBlock, 0, S(stream)>>>(grad_input, grad_output, input, size);
    else
        relu2_bwd_k<false><<<grid_for<false>(size), kBlock, 0, S(stream)>>>(grad_input, grad_output, input, size);
    return AR_LAUNCH_CHECK("relu_squared_bwd");
}

extern "C" int32_t ar_softcap_fwd(ar_stream_t stream, float* output, const float* input, float cap, int64_t size) {
    AR_ENSURE(output); AR_ENSURE(input); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    softcap_k<<<flat_grid(size, kBlock * 4), kBlock, 0, S(stream)>>>(output, input, cap, size);
    return AR_LAUNCH_CHECK("softcap_fwd");
}

extern "C" int32_t ar_ve_apply_fwd(ar_stream_t stream, float* v, const float* gate, const float* ve,
                                   int64_t num_tokens, int64_t n_kv_head, int64_t head_dim) {
    AR_ENSURE(v); AR_ENSURE(gate); AR_ENSURE(ve);
    AR_CHECK_ARG(num_tokens >= 0 && n_kv_head > 0 && head_dim > 0, "ve_apply_fwd: bad shape");
    int64_t n = num_tokens * n_kv_head * head_dim;
    if (n == 0) return AR_OK;
    ve_apply_k<<<flat_grid(n, kBlock * 4), kBlock, 0, S(stream)>>>(v, gate, ve, n, head_dim);
    return AR_LAUNCH_CHECK("ve_apply_fwd");
}

static int32_t axpby(ar_stream_t stream, float* out, const float* a, const float* b, float sa, float sb,
                     const float* psa, const float* psb, int64_t idx, int64_t n, int plain, const char* nm) {
    AR_CHECK_ARG(out && a && b, "%s: null pointer", nm);
    AR_CHECK_ARG(n >= 0, "%s: negative size", nm);
    if (n == 0) return AR_OK;
    if (n % 4 == 0 && al16(out) && al16(a) && al16(b))
        axpby_k<true><<<grid_for<true>(n), kBlock, 0, S(stream)>>>(out, a, b, sa, sb, psa, psb, idx, n, plain);
    else
        axpby_k<false><<<grid_for<false>(n), kBlock, 0, S(stream)>>>(out, a, b, sa, sb, psa, psb, idx, n, plain);
    return AR_LAUNCH_CHECK(nm);
}

extern "C" int32_t ar_add_residual_fwd(ar_stream_t stream, float* output, const float* residual, const float* input,
                                       int64_t size) {
    return axpby(stream, output, residual, input, 1.f, 1.f, nullptr, nullptr, 0, size, 1, "add_residual_fwd");
}

extern "C" int32_t ar_scaled_add_fwd(ar_stream_t stream, float* output, const float* a, const float* b,
                                     const float* scale_a, const float* scale_b, int64_t idx, int64_t size) {
    AR_ENSURE(scale_a); AR_ENSURE(scale_b);
    AR_CHECK_ARG(idx >= 0, "scaled_add_fwd: negative idx");
    return axpby(stream, output, a, b, 0.f, 0.f, scale_a, scale_b, idx, size, 0, "scaled_add_fwd");
}

extern "C" int32_t ar_scale_add(ar_stream_t stream, float* output, const float* a, const float* b, float sa,
                                float sb, int64_t size) {
    return axpby(stream, output, a, b, sa, sb, nullptr, nullptr, 0, size, 0, "scale_add");
}

extern "C" int32_t ar_scaled_add_bwd(ar_stream_t stream, float* grad_a, float* grad_b, const float* grad_output,
                                     const float* scale_a, const float* scale_b, int64_t idx, int64_t size) {
    AR_ENSURE(grad_a); AR_ENSURE(grad_b); AR_ENSURE(grad_output); AR_ENSURE(scale_a); AR_ENSURE(scale_b);
    AR_NONNEG(size);
    AR_CHECK_ARG(idx >= 0, "scaled_add_bwd: negative idx");
    AR_CHECK_ARG(grad_b != grad_output && grad_b != grad_a, "scaled_add_bwd: grad_b must not alias");
    if (size == 0) return AR_OK;
    if (size % 4 == 0 && al16(grad_a) && al16(grad_b) && al16(grad_output))
        scaled_add_bwd_k<true><<<grid_for<true>(size), kBlock, 0, S(stream)>>>(grad_a, grad_b, grad_output, scale_a,
                                                                              scale_b, idx, size);
    else
        scaled_add_bwd_k<false><<<grid_for<false>(size), kBlock, 0, S(stream)>>>(grad_a, grad_b, grad_output,
                                                                                scale_a, scale_b, idx, size);
    return AR_LAUNCH_CHECK("scaled_add_bwd");
}

static int32_t fill(ar_stream_t stream, float* out, float value, int64_t n, const char* nm) {
    AR_CHECK_ARG(out != nullptr, "%s: null pointer", nm);
    AR_CHECK_ARG(n >= 0, "%s: negative size", nm);
    if (n == 0) return AR_OK;
    if (n % 4 == 0 && al16(out))
        fill_k<true><<<grid_for<true>(n), kBlock, 0, S(stream)>>>(out, value, n);
    else
        fill_k<false><<<grid_for<false>(n), kBlock, 0, S(stream)>>>(out, value, n);
    return AR_LAUNCH_CHECK(nm);
}

extern "C" int32_t ar_zero_buffer(ar_stream_t stream, float* buf, int64_t size) {
    return fill(stream, buf, 0.f, size, "zero_buffer");
}
extern "C" int32_t ar_fill_zeros(ar_stream_t stream, float* output, int64_t size) {
    return fill(stream, output, 0.f, size, "fill_zeros");
}
extern "C" int32_t ar_fill_value(ar_stream_t stream, float* output, float value, int64_t size) {
    return fill(stream, output, value, size, "fill_value");
}

extern "C" int32_t ar_fill_normal(ar_stream_t stream, float* output, uint64_t seed_base, float std_, int64_t size) {
    AR_ENSURE(output); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    fill_normal_k<<<flat_grid(size, kBlock * 4), kBlock, 0, S(stream)>>>(output, seed_base, std_, size);
    return AR_LAUNCH_CHECK("fill_normal");
}

extern "C" int32_t ar_fill_uniform(ar_stream_t stream, float* output, uint64_t seed_base, float low, float high,
                                   int64_t size) {
    AR_ENSURE(output); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    fill_uniform_k<<<flat_grid(size, kBlock * 4), kBlock, 0, S(stream)>>>(output, seed_base, low, high, size);
    return AR_LAUNCH_CHECK("fill_uniform");
}

extern "C" int32_t ar_adamw(ar_stream_t stream, float* params, const float* grads, float* exp_avg, float* exp_avg_sq,
                            float lr, float beta1, float beta2, float eps, float weight_decay, float bias_corr1,
                            float bias_corr2, int64_t size) {
    AR_ENSURE(params); AR_ENSURE(grads); AR_ENSURE(exp_avg); AR_ENSURE(exp_avg_sq); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    adamw_k<<<flat_grid(size, kBlock * 4), kBlock, 0, S(stream)>>>(params, grads, exp_avg, exp_avg_sq, lr, beta1,
                                                                   beta2, eps, weight_decay, bias_corr1, bias_corr2,
                                                                   size);
    return AR_LAUNCH_CHECK("adamw");
}

extern "C" int32_t ar_adamw_step_group(ar_stream_t stream, float* params, const float* grads, float* exp_avg,
                                       float* exp_avg_sq, int64_t size, double lr_group, double beta1, double beta2,
                                       double eps, double weight_decay, double lr_multiplier, int64_t step) {
    // optimizer.mojo:108-125: f32 lr, f32 betas, bias corrections by repeated
    // f32 multiplication on the host.
    float lr = (float)(lr_group * lr_multiplier);
    float b1 = (float)beta1, b2 = (float)beta2;
    float bc1 = 1.0f, bc2 = 1.0f;
    for (int64_t s = 0; s < step; ++s) {
        bc1 *= b1;
        bc2 *= b2;
    }
    return ar_adamw(stream, params, grads, exp_avg, exp_avg_sq, lr, b1, b2, (float)eps, (float)weight_decay,
                    1.0f - bc1, 1.0f - bc2, size);
}

extern "C" int32_t ar_nesterov_momentum(ar_stream_t stream, float* output, const float* grads, float* momentum_buf,
                                        float momentum, int64_t size) {
    AR_ENSURE(output); AR_ENSURE(grads); AR_ENSURE(momentum_buf); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    nesterov_k<<<flat_grid(size, kBlock * 4), kBlock, 0, S(stream)>>>(output, grads, momentum_buf, momentum, size);
    return AR_LAUNCH_CHECK("nesterov_momentum");
}

extern "C" int32_t ar_muon_update(ar_stream_t stream, float* params, const float* grads, float lr, float wd,
                                  int64_t size) {
    AR_ENSURE(params); AR_ENSURE(grads); AR_NONNEG(size);
    if (size == 0) return AR_OK;
    muon_update_k<<<flat_grid(size, kBlock * 4), kBlock, 0, S(stream)>>>(params, grads, lr, wd, size);
    return AR_LAUNCH_CHECK("muon_update");
}

// model.mojo:57-81: the table is computed on the host in f64 and copied.
extern "C" int32_t ar_precompute_rope(ar_stream_t stream, float* cos_buf, float* sin_buf, int64_t seq_len,
                                      int64_t head_dim, double base) {
    AR_ENSURE(cos_buf); AR_ENSURE(sin_buf);
    AR_CHECK_ARG(seq_len > 0 && head_dim > 0 && head_dim % 2 == 0, "precompute_rope: bad shape");
    const int64_t half = head_dim / 2, n = seq_len * half;
    float* hc = (float*)malloc((size_t)n * sizeof(float));
    float* hs = (float*)malloc((size_t)n * sizeof(float));
    if (!hc || !hs) {
        free(hc);
        free(hs);
        return set_error(AR_ENOMEM, "precompute_rope: host allocation failed");
    }
    for (int64_t t = 0; t < seq_len; ++t)
        for (int64_t d = 0; d < half; ++d) {
            double freq = (double)t / pow(base, (double)(2 * d) / (double)head_dim);
            hc[t * half + d] = (float)cos(freq);
            hs[t * half + d] = (float)sin(freq);
        }
    hipError_t e1 = hipMemcpyAsync(cos_buf, hc, (size_t)n * sizeof(float), hipMemcpyHostToDevice, S(stream));
    hipError_t e2 = hipMemcpyAsync(sin_buf, hs, (size_t)n * sizeof(float), hipMemcpyHostToDevice, S(stream));
    hipError_t e3 = hipStreamSynchronize(S(stream));
    free(hc);
    free(hs);
    if (e1 != hipSuccess || e2 != hipSuccess || e3 != hipSuccess)
        return set_error(AR_EHIP, "precompute_rope: copy failed");
    return AR_OK;
}

int32_t ar::adamw_multi(hipStream_t st, float* p, const float* g, float* m, float* v, const AdamEntry* e, int n,
                        const float* sc, int bc2_i, float b2, float eps, float wd) {
    for (int j0 = 0; j0 < n; j0 += kAdamMaxTensors) {
        AdamTable t{};
        int64_t blocks = 0;
        t.n = n - j0 < kAdamMaxTensors ? n - j0 : kAdamMaxTensors;
        for (int j = 0; j < t.n; ++j) {
            const AdamEntry& x = e[j0 + j];
            t.off[j] = x.offset;
            t.size[j] = x.size;
            t.blk0[j] = blocks;
            t.lr_i[j] = x.lr_i;
            t.bc1_i[j] = x.bc1_i;
            t.b1[j] = x.b1;
            blocks += (x.size + 1023) / 1024;
        }
        if (blocks == 0) continue;
        if (blocks > INT32_MAX) return set_error(AR_EINVAL, "adamw: %lld blocks", (long long)blocks);
        adamw_multi_k<<<(unsigned)blocks, 256, 0, st>>>(t, p, g, m, v, sc, bc2_i, b2, eps, wd);
        const int32_t r = AR_LAUNCH_CHECK("adamw_multi");
        if (r) return r;
    }
    return AR_OK;
}

int32_t ar::adamw_dev(hipStream_t st, float* p, const float* g, float* m, float* v, int64_t n, const float* sc,
                      int lr_i, int bc1_i, int bc2_i, float b1, float b2, float eps, float wd) {
    if (n == 0) return AR_OK;
    adamw_dev_k<<<flat_grid(n, kBlock * 4), kBlock, 0, st>>>(p, g, m, v, sc, lr_i, bc1_i, bc2_i, b1, b2, eps, wd, n);
    return AR_LAUNCH_CHECK("adamw");
}
