// ar_fused.hip -- fused row kernels of the bf16 whole-step path.
//
// In bf16 mode every GEMM / attention operand is stored as bf16: the kernel
// that produces it rounds it once, where the fp32-storage path rounds the
// same fp32 value inside every consumer.  The small element-wise steps of the
// reference around each GEMM are folded into single passes over a row:
//
//   resid_norm    scaled_add_fwd + rmsnorm_fwd (ops.mojo:579-594, 61-104),
//                 on layer 0 also embedding_fwd + its rmsnorm (model.mojo:
//                 605-615), on value-embedding layers also ve_gate_fwd
//                 (ops.mojo:516-541) from the fp32 normalised row
//   qkv_post      rope_fwd of q and k (ops.mojo:209-238), their per-head
//                 rmsnorm (model.mojo:679-687), ve_apply_fwd on v
//                 (ops.mojo:544-560), written as bf16 attention operands
//   ce_fused      cross_entropy_fwd + cross_entropy_softcap_bwd (ops.mojo:
//                 672-740, 778-864) from one read of the logits row
//   ve_bwd        ve_apply_bwd (ops.mojo:1193-1237) from the bf16 dV that the
//                 attention backward writes into the packed [dq | dk | dv]
//                 buffer (it also applies rope_bwd to dq / dk there)
//   norm_bwd      rmsnorm_bwd (ops.mojo:1039-1085) + add_residual, and on the
//                 attention norm the two learned-scalar gradient dots
//                 (ops.mojo:1277-1308) and scaled_add_bwd (ops.mojo:1170-1190)
//
// Per element the arithmetic is the reference kernels'; only the order of
// the row sums (wave reductions) differs.  All reductions are fixed-order.
#include <math.h>

#include "ar_internal.hpp"

#include <type_traits>

namespace ar {
namespace {

constexpr int kBlock = 256;
constexpr float kNormEps = 1e-5f;  // ops.mojo:61-104

// Row outputs are stored with the nontemporal hint: these kernels stream
// their rows once, and their outputs (up to 1 GB for the logits gradient)
// would otherwise flush the L2 of data other waves are still reading.
__device__ __forceinline__ void st_bf16x4(bf16* p, float4 v) {
    bf16x4 o;
    o[0] = (bf16)v.x;
    o[1] = (bf16)v.y;
    o[2] = (bf16)v.z;
    o[3] = (bf16)v.w;
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned long long, o), reinterpret_cast<unsigned long long*>(p));
}
__device__ __forceinline__ void st_f4(float4* p, float4 v) {
    __builtin_nontemporal_store(v.x, &p->x);
    __builtin_nontemporal_store(v.y, &p->y);
    __builtin_nontemporal_store(v.z, &p->z);
    __builtin_nontemporal_store(v.w, &p->w);
}
__device__ __forceinline__ float4 ld_bf16x4(const bf16* p) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}
__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
__device__ __forceinline__ float4 axpby4(float sa, float4 a, float sb, float4 b) {
    return make_float4(sa * a.x + sb * b.x, sa * a.y + sb * b.y, sa * a.z + sb * b.z, sa * a.w + sb * b.w);
}
__device__ __forceinline__ float4 div4(float4 a, float s) { return make_float4(a.x / s, a.y / s, a.z / s, a.w / s); }
__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ __forceinline__ float4 mul4(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }

__device__ __forceinline__ int64_t wave_id() { return ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave; }
__device__ __forceinline__ int64_t wave_count() { return ((int64_t)gridDim.x * blockDim.x) / kWave; }

// Sum over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// ---------------------------------------------------------------------
// resid_norm: one wave per row; the row stays in registers (NC float4 per
// lane, chunk i = lane + 64 j).
//   MODE 0 (layer 0): x0 = rmsnorm(table[idx]); x = sa x0 + sb x0
//   MODE 1:           x = sa xin + sb x0
//   MODE 2:           x = xin (no residual mix; x not written)
// then rms = sqrt(mean(x^2) + eps), xn = x / rms (bf16), and with a gate:
// xg = xn[:, :gc] (fp32) and gate[h] = 2 sigmoid(sum_c w[h, c] xn[c]).
struct NormArgs {
    float* x0_out;
    float* x_out;
    float* rms_out;
    bf16* xn_out;
    float* xg_out;
    float* gate_out;
    const float* xin;
    const float* x0;
    const float* table;
    const int64_t* idx;
    const float* sa;
    const float* sb;
    const float* gate_w;
    int64_t layer, rows, C;
    int nkv, gc;
};

template <int NC, int MODE>
__global__ __launch_bounds__(kBlock) void resid_norm_k(NormArgs a) {
    const int lane = threadIdx.x % kWave;
    const int64_t C4 = a.C / 4;
    float sa = 0.f, sb = 0.f;
    if (MODE != 2) {
        sa = a.sa[a.layer];
        sb = a.sb[a.layer];
    }
    for (int64_t r = wave_id(); r < a.rows; r += wave_count()) {
        float4 v[NC];
        if (MODE == 0) {
            const float4* e = reinterpret_cast<const float4*>(a.table + a.idx[r] * a.C);
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int64_t i = lane + 64 * j;
                v[j] = i < C4 ? e[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                ss += dot4(v[j], v[j]);
            }
            ss = wave_sum(ss);
            const float rms0 = sqrtf(ss / (float)a.C + kNormEps);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int64_t i = lane + 64 * j;
                v[j] = div4(v[j], rms0);
                if (i < C4) st_f4(reinterpret_cast<float4*>(a.x0_out + r * a.C) + i, v[j]);
                v[j] = axpby4(sa, v[j], sb, v[j]);
            }
        } else {
            const float4* xi = reinterpret_cast<const float4*>(a.xin + r * a.C);
            const float4* x0 = reinterpret_cast<const float4*>(a.x0 + r * a.C);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int64_t i = lane + 64 * j;
                if (i < C4) v[j] = MODE == 1 ? axpby4(sa, xi[i], sb, x0[i]) : xi[i];
                else v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int64_t i = lane + 64 * j;
            if (MODE != 2 && i < C4) st_f4(reinterpret_cast<float4*>(a.x_out + r * a.C) + i, v[j]);
            ss += dot4(v[j], v[j]);
        }
        ss = wave_sum(ss);
        const float rms = sqrtf(ss / (float)a.C + kNormEps);
        if (lane == 0) a.rms_out[r] = rms;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int64_t i = lane + 64 * j;
            v[j] = div4(v[j], rms);
            if (i < C4) st_bf16x4(a.xn_out + r * a.C + 4 * i, v[j]);
        }
        if (a.gate_out) {
            // channels [0, gc) are chunk 0 of lanes [0, gc / 4)
            const bool own = lane < a.gc / 4;
            if (own) reinterpret_cast<float4*>(a.xg_out + r * a.gc)[lane] = v[0];
            for (int h = 0; h < a.nkv; ++h) {
                float p = own ? dot4(reinterpret_cast<const float4*>(a.gate_w + (int64_t)h * a.gc)[lane], v[0]) : 0.f;
                p = wave_sum(p);
                if (lane == h) a.gate_out[r * a.nkv + h] = 2.0f * (1.0f / (1.0f + __expf(-p)));
            }
        }
    }
}

// ---------------------------------------------------------------------
// qkv_post: wave per (token, part); part 0 / 1 = q / k: rope then per-head
// rmsnorm, lane (sub, j) of a head group holding the four pairs
// (d, d + HD/2), d = 4 j .. 4 j + 3, of head h0 + sub (8-byte bf16 loads and
// stores, 16-byte cos / sin loads); part 2 = v (+ gate * value embedding).
// Writes bf16 [nt, C] each.
struct QkvArgs {
    bf16 *q, *k, *v;
    const bf16* qkv;  // [nt, 3C]
    const float *cos_t, *sin_t;
    const float* gate;     // [nt, H] (value-embedding layers)
    const float* table;    // value-embedding table [V, C] or null
    const int64_t* idx;
    int64_t nt, C, period;
    int H;
};

template <int HD>
__global__ __launch_bounds__(kBlock) void qkv_post_k(QkvArgs a) {
    constexpr int HALF = HD / 2;
    constexpr int LPH = HALF / 4;   // lanes per head
    constexpr int HPI = 64 / LPH;   // heads per wave iteration
    const int lane = threadIdx.x % kWave;
    const int sub = lane / LPH, d0 = (lane % LPH) * 4;
    const int64_t C = a.C;
    for (int64_t w = wave_id(); w < a.nt * 3; w += wave_count()) {
        const int64_t t = w / 3;
        const int part = (int)(w % 3);
        const bf16* src = a.qkv + t * 3 * C + part * C;
        if (part < 2) {
            bf16* dst = (part == 0 ? a.q : a.k) + t * C;
            const int64_t tok = t % a.period;
            const float4 c = *reinterpret_cast<const float4*>(a.cos_t + tok * HALF + d0);
            const float4 s = *reinterpret_cast<const float4*>(a.sin_t + tok * HALF + d0);
            for (int h0 = 0; h0 < a.H; h0 += HPI) {
                const int h = h0 + sub;
                float4 y1 = make_float4(0.f, 0.f, 0.f, 0.f), y2 = y1;
                if (h < a.H) {
                    const float4 x1 = ld_bf16x4(src + h * HD + d0), x2 = ld_bf16x4(src + h * HD + HALF + d0);
                    y1 = make_float4(x1.x * c.x + x2.x * s.x, x1.y * c.y + x2.y * s.y, x1.z * c.z + x2.z * s.z,
                                     x1.w * c.w + x2.w * s.w);
                    y2 = make_float4(x1.x * (-s.x) + x2.x * c.x, x1.y * (-s.y) + x2.y * c.y,
                                     x1.z * (-s.z) + x2.z * c.z, x1.w * (-s.w) + x2.w * c.w);
                }
                const float ss = group_sum<LPH>(y1.x * y1.x + y2.x * y2.x + y1.y * y1.y + y2.y * y2.y +
                                                y1.z * y1.z + y2.z * y2.z + y1.w * y1.w + y2.w * y2.w);
                const float inv = 1.0f / sqrtf(ss / (float)HD + kNormEps);
                if (h < a.H) {
                    st_bf16x4(dst + h * HD + d0, make_float4(y1.x * inv, y1.y * inv, y1.z * inv, y1.w * inv));
                    st_bf16x4(dst + h * HD + HALF + d0, make_float4(y2.x * inv, y2.y * inv, y2.z * inv, y2.w * inv));
                }
            }
        } else {
            bf16* dst = a.v + t * C;
            const float4* ve = a.table ? reinterpret_cast<const float4*>(a.table + a.idx[t] * C) : nullptr;
            for (int64_t i = lane; i < C / 4; i += kWave) {
                float4 x = ld_bf16x4(src + 4 * i);
                if (ve) {
                    const float g = a.gate[t * a.H + (4 * i) / HD];
                    const float4 e = ve[i];
                    x = make_float4(x.x + g * e.x, x.y + g * e.y, x.z + g * e.z, x.w + g * e.w);
                }
                st_bf16x4(dst + 4 * i, x);
            }
        }
    }
}

// ---------------------------------------------------------------------
// ce_fused: block per token row.  loss = lse - l[target] (0 for an ignored
// target, < 0 or >= V); grad = (softmax - onehot) * scale as bf16 (0 rows for ignored
// targets).  NV4 > 0: the row is held in registers (NV4 float4 per thread).
template <typename TL>
__device__ __forceinline__ float4 ld_logit4(const TL* p);
template <>
__device__ __forceinline__ float4 ld_logit4<float>(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 ld_logit4<bf16>(const bf16* p) {
    return ld_bf16x4(p);
}

template <int NV4, typename TL>
__global__ __launch_bounds__(kBlock) void ce_fused_k(float* loss, bf16* grad, const TL* logits,
                                                     const int64_t* targets, int64_t V, float scale) {
    __shared__ float red[kBlock / kWave];
    const int64_t t = blockIdx.x;
    const int64_t tg = targets[t];
    const TL* rowp = logits + t * V;
    auto row_at = [&](int64_t i) { return ld_logit4<TL>(rowp + 4 * i); };
    const int64_t V4 = V / 4;
    constexpr int R = NV4 > 0 ? NV4 : 1;
    float4 x[R];
    float m = -INFINITY;
    if (NV4 > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int64_t i = threadIdx.x + (int64_t)kBlock * j;
            x[j] = i < V4 ? row_at(i) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            m = fmaxf(m, fmaxf(fmaxf(x[j].x, x[j].y), fmaxf(x[j].z, x[j].w)));
        }
    } else {
        for (int64_t i = threadIdx.x; i < V4; i += kBlock) {
            const float4 y = row_at(i);
            m = fmaxf(m, fmaxf(fmaxf(y.x, y.y), fmaxf(y.z, y.w)));
        }
    }
    m = block_max(m, red);
    // exp(x - m) once per element: the register-resident row keeps it for the
    // gradient pass, which then scales by 1/s (a multiply, not a division).
    auto ex4 = [&](float4 y) { return make_float4(__expf(y.x - m), __expf(y.y - m), __expf(y.z - m), __expf(y.w - m)); };
    float s = 0.f;
    if (NV4 > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            x[j] = ex4(x[j]);
            s += (x[j].x + x[j].y) + (x[j].z + x[j].w);
        }
    } else {
        for (int64_t i = threadIdx.x; i < V4; i += kBlock) {
            const float4 y = row_at(i);
            s += __expf(y.x - m) + __expf(y.y - m) + __expf(y.z - m) + __expf(y.w - m);
        }
    }
    s = block_sum(s, red);
    const bool live = tg >= 0 && tg < V;  // other targets are ignored rows
    if (loss && threadIdx.x == 0) loss[t] = live ? -(float)logits[t * V + tg] + (m + logf(s)) : 0.f;
    bf16* g = grad + t * V;
    const float rs = 1.0f / s;
    // e = exp(logit - m) for four consecutive columns starting at 4 i
    auto emit = [&](int64_t i, float4 e) {
        float4 o;
        if (!live) {
            o = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            o = mul4(e, rs);
            const int64_t e = tg - 4 * i;
            if (e == 0) o.x -= 1.0f;
            if (e == 1) o.y -= 1.0f;
            if (e == 2) o.z -= 1.0f;
            if (e == 3) o.w -= 1.0f;
            o = mul4(o, scale);
        }
        st_bf16x4(g + 4 * i, o);
    };
    if (NV4 > 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int64_t i = threadIdx.x + (int64_t)kBlock * j;
            if (i < V4) emit(i, x[j]);
        }
    } else {
        for (int64_t i = threadIdx.x; i < V4; i += kBlock) emit(i, ex4(row_at(i)));
    }
}

// The same for bf16 logits with V % 8 == 0: 16-byte loads and stores, 8
// columns per thread and step (the row is NV8 x 8 registers per thread).
template <int NV8>
__global__ __launch_bounds__(kBlock) void ce_fused8_k(float* loss, bf16* grad, const bf16* logits,
                                                      const int64_t* targets, int64_t V, float scale) {
    __shared__ float red[kBlock / kWave];
    const int64_t t = blockIdx.x;
    const int64_t tg = targets[t];
    const bf16* rowp = logits + t * V;
    const int64_t V8 = V / 8;
    float x[NV8][8];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV8; ++j) {
        const int64_t i = threadIdx.x + (int64_t)kBlock * j;
        if (i < V8) {
            const bf16x8 v = *reinterpret_cast<const bf16x8*>(rowp + 8 * i);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[j][e] = (float)v[e];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[j][e] = -INFINITY;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, x[j][e]);
    }
    m = block_max(m, red);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV8; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[j][e] = __expf(x[j][e] - m);
        s += (x[j][0] + x[j][1]) + (x[j][2] + x[j][3]);
        s += (x[j][4] + x[j][5]) + (x[j][6] + x[j][7]);
    }
    s = block_sum(s, red);
    const bool live = tg >= 0 && tg < V;  // other targets are ignored rows
    if (loss && threadIdx.x == 0) loss[t] = live ? -(float)logits[t * V + tg] + (m + logf(s)) : 0.f;
    bf16* g = grad + t * V;
    const float rs = 1.0f / s;
#pragma unroll
    for (int j = 0; j < NV8; ++j) {
        const int64_t i = threadIdx.x + (int64_t)kBlock * j;
        if (i >= V8) continue;
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = 0.f;
            if (live) {
                v = x[j][e] * rs;
                if (tg == 8 * i + e) v -= 1.0f;
                v *= scale;
            }
            o[e] = (bf16)v;
        }
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), reinterpret_cast<u32x4*>(g + 8 * i));
    }
}

// ---------------------------------------------------------------------
// ve_bwd (ve_apply_bwd, ops.mojo:1193-1237) from a bf16 dV with row stride
// ldv: wave per token; gve = gate * dv, ggate[h] = sum_d ve[d] dv[d]
// (groups of HD/4 lanes hold one head).
struct VeBwdArgs {
    float* gve;  // [nt, C]
    float* ggate;
    const bf16* gv;
    const float* gate;
    const float* table;
    const int64_t* idx;
    int64_t nt, C, ldv;
    int H;
};

template <int HD>
__global__ __launch_bounds__(kBlock) void ve_bwd_k(VeBwdArgs a) {
    constexpr int G = HD / 4;
    const int lane = threadIdx.x % kWave;
    const int64_t C = a.C;
    for (int64_t t = wave_id(); t < a.nt; t += wave_count()) {
        const bf16* src = a.gv + t * a.ldv;
        const float4* ve = reinterpret_cast<const float4*>(a.table + a.idx[t] * C);
        for (int64_t i0 = 0; i0 < C / 4; i0 += kWave) {
            const int64_t i = i0 + lane;
            const bool ok = i < C / 4;
            const int h = (int)((4 * i) / HD);
            float dg = 0.f;
            if (ok) {
                const float4 x = ld_bf16x4(src + 4 * i);
                const float g = a.gate[t * a.H + h];
                reinterpret_cast<float4*>(a.gve + t * C)[i] = mul4(x, g);
                dg = dot4(ve[i], x);
            }
            dg = group_sum<G>(dg);
            if (ok && lane % G == 0) a.ggate[t * a.H + h] = dg;
        }
    }
}

// ---------------------------------------------------------------------
// norm_bwd: wave per row, row in registers.
//   MODE 0: gx = rmsnorm_bwd(gx, x, rms)                      (final norm)
//   MODE 1: gx = gx + rmsnorm_bwd(gn, x, rms)                 (MLP norm)
//   MODE 2: g = gx + rmsnorm_bwd(gn, x, rms); dots g.x, g.x0 into this
//           wave's partial; gx = res[layer] * g               (attention norm)
// and gxb = bf16(gx).  GB: gn is read from its bf16 copy gnb.  MODE 2 runs on a fixed grid of kNormBwdWaves waves.
struct NormBwdArgs {
    float* gx;
    bf16* gxb;
    const float* gn;
    const bf16* gnb;  // gn stored as bf16 (GB instantiations)
    const float* x;
    const float* rms;
    const float* x0;
    const float* res;
    float* partial;
    int64_t layer, rows, C;
};

template <int NC, int MODE, bool GB>
__global__ __launch_bounds__(kBlock) void norm_bwd_k(NormBwdArgs a) {
    const int lane = threadIdx.x % kWave;
    const int64_t C4 = a.C / 4;
    const float scale = MODE == 2 ? a.res[a.layer] : 1.0f;
    float p1 = 0.f, p2 = 0.f;
    for (int64_t r = wave_id(); r < a.rows; r += wave_count()) {
        const float4* g4 = reinterpret_cast<const float4*>((MODE == 0 ? a.gx : a.gn) + r * a.C);
        const bf16* gb = a.gnb + r * a.C;
        const float4* x4 = reinterpret_cast<const float4*>(a.x + r * a.C);
        float4 g[NC], x[NC];
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int64_t i = lane + 64 * j;
            if constexpr (GB) g[j] = i < C4 ? ld_bf16x4(gb + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            else g[j] = i < C4 ? g4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            x[j] = i < C4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            dot += dot4(g[j], x[j]);
        }
        dot = wave_sum(dot);
        const float rr = a.rms[r];
        const float coef = dot / ((float)a.C * (rr * rr));
        float4* o4 = reinterpret_cast<float4*>(a.gx + r * a.C);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int64_t i = lane + 64 * j;
            if (i >= C4) continue;
            float4 o = make_float4((g[j].x - x[j].x * coef) / rr, (g[j].y - x[j].y * coef) / rr,
                                   (g[j].z - x[j].z * coef) / rr, (g[j].w - x[j].w * coef) / rr);
            if (MODE != 0) o = add4(o4[i], o);
            if (MODE == 2) {
                p1 += dot4(o, x[j]);
                p2 += dot4(o, reinterpret_cast<const float4*>(a.x0 + r * a.C)[i]);
                o = mul4(o, scale);
            }
            st_f4(o4 + i, o);
            st_bf16x4(a.gxb + r * a.C + 4 * i, o);
        }
    }
    if (MODE == 2) {
        p1 = wave_sum(p1);
        p2 = wave_sum(p2);
        if (lane == 0) {
            a.partial[2 * wave_id()] = p1;
            a.partial[2 * wave_id() + 1] = p2;
        }
    }
}

__global__ void scalar_finish_k(float* g_res, float* g_x0, const float* partial, int64_t nwaves, int64_t layer) {
    __shared__ float red[kBlock / kWave];
    float s1 = 0.f, s2 = 0.f;
    for (int64_t i = threadIdx.x; i < nwaves; i += kBlock) {
        s1 += partial[2 * i];
        s2 += partial[2 * i + 1];
    }
    s1 = block_sum(s1, red);
    s2 = block_sum(s2, red);
    if (threadIdx.x == 0) {
        g_res[layer] += s1;
        g_x0[layer] += s2;
    }
}

__global__ void to_bf16_k(bf16* out, const float* in, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
        st_bf16x4(out + 4 * i, reinterpret_cast<const float4*>(in)[i]);
}

// Batched fp32 -> bf16 transpose: entry e maps the [rows, cols] fp32 matrix
// at in + src to the [cols, rows] bf16 matrix at out + dst.  One 64 x 64
// tile per workgroup (tiles numbered per entry from tab[e].tile0), staged
// through LDS so both the read (rows of the source) and the write (rows of
// the transpose) are coalesced.
__global__ __launch_bounds__(256) void transpose_bf16_k(bf16* out, const float* in, const TransposeEntry* tab,
                                                         int n) {
    __shared__ float t[64][65];
    int e = 0;
    while (e + 1 < n && (int64_t)blockIdx.x >= tab[e + 1].tile0) ++e;
    const TransposeEntry te = tab[e];
    const int64_t local = (int64_t)blockIdx.x - te.tile0;
    const int64_t tcols = (te.cols + 63) / 64;
    const int64_t r0 = (local / tcols) * 64, c0 = (local % tcols) * 64;
    const float* src = in + te.src;
    bf16* dst = out + te.dst;
    const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
    for (int r = ty; r < 64; r += 4) {
        const int64_t gr = r0 + r, gc = c0 + tx;
        t[r][tx] = gr < te.rows && gc < te.cols ? src[gr * te.cols + gc] : 0.f;
    }
    __syncthreads();
    for (int c = ty; c < 64; c += 4) {
        const int64_t gc = c0 + c, gr = r0 + tx;
        if (gc < te.cols && gr < te.rows) dst[gc * te.rows + gr] = (bf16)t[tx][c];
    }
}

// D[r] = sum_d O[r, d] * dO[r, d] with dO stored as bf16; groups of HD/4
// lanes hold one row.
template <int G>
__global__ __launch_bounds__(kBlock) void precompute_d_mixed_k(float* d, const float* o, const bf16* g, int64_t rows) {
    const int lane = threadIdx.x % kWave;
    const int64_t total = rows * G;
    for (int64_t base = wave_id() * kWave; base < total; base += wave_count() * kWave) {
        const int64_t f = base + lane;
        float s = 0.f;
        if (f < total) {
            const float4 ov = reinterpret_cast<const float4*>(o)[f];
            const bf16x4 gv = reinterpret_cast<const bf16x4*>(g)[f];
            s = ov.x * (float)gv[0] + ov.y * (float)gv[1] + ov.z * (float)gv[2] + ov.w * (float)gv[3];
        }
        s = group_sum<G>(s);
        if (f < total && lane % G == 0) d[f / G] = s;
    }
}

inline unsigned wave_blocks(int64_t rows) { return flat_grid(rows, kBlock / kWave); }

}  // namespace

// ---------------------------------------------------------------------
// host entry points (shapes validated by the caller, ar_model.hip)

int32_t resid_norm(hipStream_t st, int mode, float* x0_out, float* x_out, float* rms_out, bf16* xn_out,
                   float* xg_out, float* gate_out, const float* xin, const float* x0, const float* table,
                   const int64_t* idx, const float* sa, const float* sb, int64_t layer, const float* gate_w,
                   int64_t nkv, int64_t gc, int64_t rows, int64_t C) {
    if (C % 4 != 0 || C > 256 * 16) return set_error(AR_EUNSUPPORTED, "resid_norm: n_embd %lld", (long long)C);
    if (gate_out && (gc % 4 != 0 || gc > 256 || gc > C))
        return set_error(AR_EUNSUPPORTED, "resid_norm: gate channels %lld", (long long)gc);
    NormArgs a{x0_out, x_out, rms_out, xn_out, xg_out, gate_out, xin, x0, table, idx, sa, sb, gate_w,
               layer, rows, C, (int)nkv, (int)gc};
    const int nc = (int)cdiv(C, 256);
    const unsigned grid = wave_blocks(rows);
#define AR_RN(NC)                                                                              \
    do {                                                                                       \
        if (mode == 0) resid_norm_k<NC, 0><<<grid, kBlock, 0, st>>>(a);                        \
        else if (mode == 1) resid_norm_k<NC, 1><<<grid, kBlock, 0, st>>>(a);                   \
        else resid_norm_k<NC, 2><<<grid, kBlock, 0, st>>>(a);                                  \
    } while (0)
    if (nc <= 1) AR_RN(1);
    else if (nc <= 2) AR_RN(2);
    else if (nc <= 4) AR_RN(4);
    else if (nc <= 8) AR_RN(8);
    else AR_RN(16);
#undef AR_RN
    return check_launch("resid_norm");
}

int32_t qkv_post(hipStream_t st, bf16* q, bf16* k, bf16* v, const bf16* qkv, const float* cos_t, const float* sin_t,
                 int64_t period, const float* gate, const float* table, const int64_t* idx, int64_t nt, int64_t C,
                 int64_t H, int64_t hd) {
    QkvArgs a{q, k, v, qkv, cos_t, sin_t, gate, table, idx, nt, C, period, (int)H};
    const unsigned grid = wave_blocks(nt * 3);
    switch (hd) {
        case 32: qkv_post_k<32><<<grid, kBlock, 0, st>>>(a); break;
        case 64: qkv_post_k<64><<<grid, kBlock, 0, st>>>(a); break;
        case 128: qkv_post_k<128><<<grid, kBlock, 0, st>>>(a); break;
        default: return set_error(AR_EUNSUPPORTED, "qkv_post: head_dim %lld", (long long)hd);
    }
    return check_launch("qkv_post");
}

template <typename TL>
static int32_t ce_fused_t(hipStream_t st, float* loss, bf16* grad, const TL* logits, const int64_t* targets,
                          int64_t rows, int64_t V, float scale) {
    if (V % 4 != 0) return set_error(AR_EUNSUPPORTED, "ce_fused: vocab %lld not a multiple of 4", (long long)V);
    if (rows == 0) return AR_OK;
    if (rows > 0x7fffffff) return set_error(AR_EINVAL, "ce_fused: too many rows");
    const int64_t nv4 = cdiv(V, 4 * kBlock);
    const unsigned grid = (unsigned)rows;
    if constexpr (std::is_same<TL, bf16>::value) {
        const int64_t nv8 = cdiv(V, 8 * kBlock);
        if (V % 8 == 0 && nv8 <= 8) {
            if (nv8 <= 1) ce_fused8_k<1><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
            else if (nv8 <= 2) ce_fused8_k<2><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
            else if (nv8 <= 4) ce_fused8_k<4><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
            else ce_fused8_k<8><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
            return check_launch("ce_fused");
        }
    }
    if (nv4 <= 2) ce_fused_k<2, TL><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
    else if (nv4 <= 4) ce_fused_k<4, TL><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
    else if (nv4 <= 8) ce_fused_k<8, TL><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
    else if (nv4 <= 16) ce_fused_k<16, TL><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
    else ce_fused_k<0, TL><<<grid, kBlock, 0, st>>>(loss, grad, logits, targets, V, scale);
    return check_launch("ce_fused");
}
int32_t ce_fused(hipStream_t st, float* loss, bf16* grad, const float* logits, const int64_t* targets, int64_t rows,
                 int64_t V, float scale) {
    return ce_fused_t(st, loss, grad, logits, targets, rows, V, scale);
}
int32_t ce_fused(hipStream_t st, float* loss, bf16* grad, const bf16* logits, const int64_t* targets, int64_t rows,
                 int64_t V, float scale) {
    return ce_fused_t(st, loss, grad, logits, targets, rows, V, scale);
}

int32_t ve_bwd(hipStream_t st, float* gve, float* ggate, const bf16* gv, int64_t ldv, const float* gate,
               const float* table, const int64_t* idx, int64_t nt, int64_t C, int64_t H, int64_t hd) {
    VeBwdArgs a{gve, ggate, gv, gate, table, idx, nt, C, ldv, (int)H};
    const unsigned grid = wave_blocks(nt);
    switch (hd) {
        case 32: ve_bwd_k<32><<<grid, kBlock, 0, st>>>(a); break;
        case 64: ve_bwd_k<64><<<grid, kBlock, 0, st>>>(a); break;
        case 128: ve_bwd_k<128><<<grid, kBlock, 0, st>>>(a); break;
        default: return set_error(AR_EUNSUPPORTED, "ve_bwd: head_dim %lld", (long long)hd);
    }
    return check_launch("ve_bwd");
}

int32_t norm_bwd(hipStream_t st, int mode, float* gx, bf16* gxb, const float* gn, const float* x, const float* rms,
                 const float* x0, const float* res, int64_t layer, float* g_res, float* g_x0, float* partial,
                 int64_t rows, int64_t C, const bf16* gnb) {
    if (C % 4 != 0 || C > 256 * 16) return set_error(AR_EUNSUPPORTED, "norm_bwd: n_embd %lld", (long long)C);
    if (mode != 0 && (gn != nullptr) == (gnb != nullptr))
        return set_error(AR_EINVAL, "norm_bwd: give the normed-input gradient once, fp32 or bf16");
    NormBwdArgs a{gx, gxb, gn, gnb, x, rms, x0, res, partial, layer, rows, C};
    const int nc = (int)cdiv(C, 256);
    const unsigned grid = mode == 2 ? (unsigned)(kNormBwdWaves / (kBlock / kWave)) : wave_blocks(rows);
    const bool gb = mode != 0 && gnb != nullptr;
#define AR_NB(NC)                                                                            \
    do {                                                                                     \
        if (mode == 0) norm_bwd_k<NC, 0, false><<<grid, kBlock, 0, st>>>(a);                 \
        else if (mode == 1 && gb) norm_bwd_k<NC, 1, true><<<grid, kBlock, 0, st>>>(a);       \
        else if (mode == 1) norm_bwd_k<NC, 1, false><<<grid, kBlock, 0, st>>>(a);            \
        else if (gb) norm_bwd_k<NC, 2, true><<<grid, kBlock, 0, st>>>(a);                    \
        else norm_bwd_k<NC, 2, false><<<grid, kBlock, 0, st>>>(a);                           \
    } while (0)
    if (nc <= 1) AR_NB(1);
    else if (nc <= 2) AR_NB(2);
    else if (nc <= 4) AR_NB(4);
    else if (nc <= 8) AR_NB(8);
    else AR_NB(16);
#undef AR_NB
    if (mode == 2) scalar_finish_k<<<1, kBlock, 0, st>>>(g_res, g_x0, partial, kNormBwdWaves, layer);
    return check_launch("norm_bwd");
}

int32_t to_bf16(hipStream_t st, bf16* out, const float* in, int64_t n) {
    if (n % 4 != 0) return set_error(AR_EINVAL, "to_bf16: size %lld not a multiple of 4", (long long)n);
    if (n == 0) return AR_OK;
    to_bf16_k<<<flat_grid(n / 4, kBlock * 4), kBlock, 0, st>>>(out, in, n / 4);
    return check_launch("to_bf16");
}

int32_t transpose_bf16(hipStream_t st, bf16* out, const float* in, const TransposeEntry* tab, int n,
                       int64_t tiles) {
    if (n <= 0 || tiles <= 0) return AR_OK;
    transpose_bf16_k<<<(unsigned)tiles, 256, 0, st>>>(out, in, tab, n);
    return check_launch("transpose_bf16");
}

int32_t precompute_d_mixed(hipStream_t st, float* d, const float* o, const bf16* g, int64_t rows, int64_t hd) {
    if (rows == 0) return AR_OK;
    const unsigned grid = flat_grid(cdiv(rows * hd / 4, kWave), kBlock / kWave);
    switch (hd) {
        case 32: precompute_d_mixed_k<8><<<grid, kBlock, 0, st>>>(d, o, g, rows); break;
        case 64: precompute_d_mixed_k<16><<<grid, kBlock, 0, st>>>(d, o, g, rows); break;
        case 128: precompute_d_mixed_k<32><<<grid, kBlock, 0, st>>>(d, o, g, rows); break;
        default: return set_error(AR_EUNSUPPORTED, "precompute_d: head_dim %lld", (long long)hd);
    }
    return check_launch("precompute_d_mixed");
}

}  // namespace ar

// The bf16 step's LM-head loss as one C-ABI call (the same two launches the
// training step runs: the SOFTCAP-epilogue GEMM, then ce_fused).
extern "C" int32_t ar_lm_head_softcap_ce_bf16(ar_stream_t stream, float* loss_out, void* grad_logits, void* logits,
                                              const void* input, const void* weight, const int64_t* targets,
                                              int64_t num_tokens, int64_t vocab_size, int64_t embd_dim, float cap,
                                              float loss_scale) {
    AR_CHECK_ARG(grad_logits && logits && input && weight && targets, "lm_head_softcap_ce: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && vocab_size > 0 && embd_dim > 0, "lm_head_softcap_ce: bad sizes");
    AR_CHECK_ARG(((num_tokens | vocab_size | embd_dim) & 7) == 0,
                 "lm_head_softcap_ce: num_tokens, vocab_size and embd_dim must be multiples of 8");
    AR_CHECK_ARG(((reinterpret_cast<uintptr_t>(grad_logits) | reinterpret_cast<uintptr_t>(logits) |
                   reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(weight)) & 15) == 0,
                 "lm_head_softcap_ce: operands must be 16-byte aligned");
    AR_CHECK_ARG(cap > 0.f, "lm_head_softcap_ce: cap must be positive");
    if (num_tokens == 0) return AR_OK;
    const hipStream_t st = ar::S(stream);
    const int32_t r = ar::gemm_epilogue(st, 0, ar::GEMM_EPI_SOFTCAP, logits, 1, input, 1, weight, 1, num_tokens,
                                        vocab_size, embd_dim, nullptr, nullptr, cap);
    if (r != AR_OK) return r;
    return ar::ce_fused(st, loss_out, static_cast<ar::bf16*>(grad_logits), static_cast<const ar::bf16*>(logits),
                        targets, num_tokens, vocab_size, loss_scale);
}
