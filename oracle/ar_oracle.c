/*
 * ar_oracle.c -- CPU restatement of the Mojo reference's training step.
 * TEST INFRASTRUCTURE ONLY (the parity checker); see ar_oracle.h.
 * Citations are to /root/reference/ (sergeytimoshin/autoresearch).
 */
#include "ar_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ===================== kernels/ops.mojo ===================== */

/* ops.mojo:41-55 */
void orc_embedding_fwd(float* out, const float* weight, const int64_t* idx, int64_t n, int64_t dim) {
    for (int64_t i = 0; i < n; ++i)
        memcpy(out + i * dim, weight + idx[i] * dim, (size_t)dim * sizeof(float));
}

/* ops.mojo:61-104: rms = sqrt(mean(x^2) + 1e-5); y = x / rms */
void orc_rmsnorm_fwd(float* out, float* rms_out, const float* in, int64_t rows, int64_t dim) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* x = in + r * dim;
        double ss = 0.0;
        for (int64_t i = 0; i < dim; ++i) ss += (double)x[i] * (double)x[i];
        float mean_sq = (float)ss / (float)dim;
        float rms = sqrtf(mean_sq + 1e-5f);
        rms_out[r] = rms;
        for (int64_t i = 0; i < dim; ++i) out[r * dim + i] = x[i] / rms;
    }
}

/* Inner product of two fp32 rows accumulated in double (4 partial sums). */
static inline double dot_d(const float* a, const float* b, int64_t K) {
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    int64_t r = 0;
    for (; r + 4 <= K; r += 4) {
        s0 += (double)a[r] * (double)b[r];
        s1 += (double)a[r + 1] * (double)b[r + 1];
        s2 += (double)a[r + 2] * (double)b[r + 2];
        s3 += (double)a[r + 3] * (double)b[r + 3];
    }
    for (; r < K; ++r) s0 += (double)a[r] * (double)b[r];
    return (s0 + s1) + (s2 + s3);
}

/* C[m,n] (=|+=) sum_r A[m,r] * B[n,r]; both operands have row stride K. */
static void gemm_nt_d(float* C, const float* A, const float* Bm, int64_t M, int64_t N, int64_t K,
                      int accumulate) {
    const int64_t MB = 16, NB = 128;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t mb = 0; mb < M; mb += MB) {
        int64_t me = mb + MB < M ? mb + MB : M;
        for (int64_t nb = 0; nb < N; nb += NB) {
            int64_t ne = nb + NB < N ? nb + NB : N;
            for (int64_t m = mb; m < me; ++m)
                for (int64_t n = nb; n < ne; ++n) {
                    double acc = dot_d(A + m * K, Bm + n * K, K);
                    if (accumulate) C[m * N + n] += (float)acc;
                    else C[m * N + n] = (float)acc;
                }
        }
    }
}

static float* transpose_copy(const float* X, int64_t rows, int64_t cols) {
    float* t = (float*)malloc((size_t)rows * cols * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < cols; ++c)
        for (int64_t r = 0; r < rows; ++r) t[c * rows + r] = X[r * cols + c];
    return t;
}

/* ops.mojo:110-120 docstring contract: Y[m,n] = sum_k X[m,k] W[n,k] (overwrite).
 * The reference body stores only a quarter of Y (quirk Q1); the docstring
 * contract is what is restated. */
void orc_linear_fwd(float* out, const float* in, const float* w, int64_t M, int64_t N, int64_t K) {
    gemm_nt_d(out, in, w, M, N, K, 0);
}

/* ops.mojo:870-880: dX[m,k] = sum_n dY[m,n] W[n,k] (overwrite).  dX may alias
 * dY (model.mojo:906, quirk Q2): all of dY is read before dX is written. */
void orc_linear_bwd_dx(float* dx, const float* dy, const float* w, int64_t M, int64_t N, int64_t K) {
    float* wt = transpose_copy(w, N, K); /* [K, N] */
    float* dyc = (float*)malloc((size_t)M * N * sizeof(float));
    memcpy(dyc, dy, (size_t)M * N * sizeof(float));
    gemm_nt_d(dx, dyc, wt, M, K, N, 0);
    free(dyc);
    free(wt);
}

/* ops.mojo:953-963: dW[n,k] += sum_m dY[m,n] X[m,k] (accumulate). */
void orc_linear_bwd_dw(float* dw, const float* dy, const float* x, int64_t M, int64_t N, int64_t K) {
    float* dyt = transpose_copy(dy, M, N); /* [N, M] */
    float* xt = transpose_copy(x, M, K);   /* [K, M] */
    gemm_nt_d(dw, dyt, xt, N, K, M, 1);
    free(dyt);
    free(xt);
}

/* ops.mojo:209-238: table row = flat token index (quirk Q3). */
void orc_rope_fwd(float* out, const float* in, const float* cos_t, const float* sin_t,
                  int64_t num_tokens, int64_t num_heads, int64_t head_dim) {
    int64_t half = head_dim / 2;
#pragma omp parallel for schedule(static)
    for (int64_t th = 0; th < num_tokens * num_heads; ++th) {
        int64_t tok = th / num_heads;
        const float* x = in + th * head_dim;
        float* y = out + th * head_dim;
        for (int64_t d = 0; d < half; ++d) {
            float x1 = x[d], x2 = x[half + d];
            float c = cos_t[tok * half + d], s = sin_t[tok * half + d];
            y[d] = x1 * c + x2 * s;
            y[half + d] = x1 * (-s) + x2 * c;
        }
    }
}

/* ops.mojo:1091-1120: inverse rotation. */
void orc_rope_bwd(float* dx, const float* dy, const float* cos_t, const float* sin_t,
                  int64_t num_tokens, int64_t num_heads, int64_t head_dim) {
    int64_t half = head_dim / 2;
#pragma omp parallel for schedule(static)
    for (int64_t th = 0; th < num_tokens * num_heads; ++th) {
        int64_t tok = th / num_heads;
        const float* g = dy + th * head_dim;
        float* o = dx + th * head_dim;
        for (int64_t d = 0; d < half; ++d) {
            float dy1 = g[d], dy2 = g[half + d];
            float c = cos_t[tok * half + d], s = sin_t[tok * half + d];
            o[d] = dy1 * c - dy2 * s;
            o[half + d] = dy1 * s + dy2 * c;
        }
    }
}

/* Key kp is visible from query qp iff kp <= qp and (window <= 0 or
 * kp >= qp - window): ops.mojo:289-293, ops.mojo:386-390, ops.mojo:450-453. */
static inline int64_t attn_kstart(int64_t qp, int64_t window) {
    if (window > 0 && qp - window > 0) return qp - window;
    return 0;
}

/* ops.mojo:244-323.  Softmax attention with scale 1/sqrt(hd); LSE = m + log(l)
 * in scaled-score units.  Computed with a two-pass softmax in double (equal to
 * the reference's online alpha/beta renormalisation up to rounding, Q15). */
void orc_flash_attn_fwd(float* out, float* lse, const float* q, const float* k, const float* v,
                        int64_t B, int64_t T, int64_t H, int64_t hd, int64_t window) {
    const double scale = 1.0 / sqrt((double)(float)hd);
    const float scale_f = 1.0f / sqrtf((float)hd);
    (void)scale;
#pragma omp parallel
    {
        double* s = (double*)malloc((size_t)T * sizeof(double));
        double* o = (double*)malloc((size_t)hd * sizeof(double));
#pragma omp for schedule(dynamic, 16)
        for (int64_t tid = 0; tid < B * T * H; ++tid) {
            int64_t bt = tid / H, h = tid % H, b = bt / T, qp = bt % T;
            const float* qr = q + tid * hd;
            int64_t k0 = attn_kstart(qp, window);
            double mx = -INFINITY;
            for (int64_t kp = k0; kp <= qp; ++kp) {
                const float* kr = k + ((b * T + kp) * H + h) * hd;
                double acc = 0.0;
                for (int64_t d = 0; d < hd; ++d) acc += (double)qr[d] * (double)kr[d];
                s[kp] = acc * (double)scale_f;
                if (s[kp] > mx) mx = s[kp];
            }
            double l = 0.0;
            for (int64_t d = 0; d < hd; ++d) o[d] = 0.0;
            for (int64_t kp = k0; kp <= qp; ++kp) {
                double p = exp(s[kp] - mx);
                l += p;
                const float* vr = v + ((b * T + kp) * H + h) * hd;
                for (int64_t d = 0; d < hd; ++d) o[d] += p * (double)vr[d];
            }
            for (int64_t d = 0; d < hd; ++d) out[tid * hd + d] = (float)(o[d] / l);
            lse[tid] = (l > 0.0) ? (float)(mx + log(l)) : -INFINITY; /* Q13 */
        }
        free(s);
        free(o);
    }
}

/* ops.mojo:329-346 */
void orc_flash_attn_bwd_precompute_d(float* d, const float* out, const float* dout,
                                     int64_t B, int64_t T, int64_t H, int64_t hd) {
#pragma omp parallel for schedule(static)
    for (int64_t tid = 0; tid < B * T * H; ++tid) {
        double acc = 0.0;
        for (int64_t j = 0; j < hd; ++j) acc += (double)out[tid * hd + j] * (double)dout[tid * hd + j];
        d[tid] = (float)acc;
    }
}

/* ops.mojo:349-411: dQ = scale * sum_kp P (dP - D) K, P = exp(s - lse). */
void orc_flash_attn_bwd_dq(float* dq, const float* q, const float* k, const float* v,
                           const float* dout, const float* lse, const float* dd,
                           int64_t B, int64_t T, int64_t H, int64_t hd, int64_t window) {
    const float scale_f = 1.0f / sqrtf((float)hd);
#pragma omp parallel
    {
        double* acc = (double*)malloc((size_t)hd * sizeof(double));
#pragma omp for schedule(dynamic, 16)
        for (int64_t bth = 0; bth < B * T * H; ++bth) {
            int64_t bt = bth / H, h = bth % H, b = bt / T, qp = bt % T;
            const float* qr = q + bth * hd;
            const float* gr = dout + bth * hd;
            for (int64_t j = 0; j < hd; ++j) acc[j] = 0.0;
            for (int64_t kp = attn_kstart(qp, window); kp <= qp; ++kp) {
                const float* kr = k + ((b * T + kp) * H + h) * hd;
                const float* vr = v + ((b * T + kp) * H + h) * hd;
                double sc = 0.0, da = 0.0;
                for (int64_t j = 0; j < hd; ++j) {
                    sc += (double)qr[j] * (double)kr[j];
                    da += (double)gr[j] * (double)vr[j];
                }
                double a = exp(sc * (double)scale_f - (double)lse[bth]);
                double ds = a * (da - (double)dd[bth]);
                for (int64_t j = 0; j < hd; ++j) acc[j] += ds * (double)kr[j];
            }
            for (int64_t j = 0; j < hd; ++j) dq[bth * hd + j] = (float)(acc[j] * (double)scale_f);
        }
        free(acc);
    }
}

/* ops.mojo:414-480: query range [kp, kp+window] (inclusive) when windowed. */
void orc_flash_attn_bwd_dkv(float* dk, float* dv, const float* q, const float* k, const float* v,
                            const float* dout, const float* lse, const float* dd,
                            int64_t B, int64_t T, int64_t H, int64_t hd, int64_t window) {
    const float scale_f = 1.0f / sqrtf((float)hd);
#pragma omp parallel
    {
        double* ak = (double*)malloc((size_t)hd * sizeof(double));
        double* av = (double*)malloc((size_t)hd * sizeof(double));
#pragma omp for schedule(dynamic, 16)
        for (int64_t bth = 0; bth < B * T * H; ++bth) {
            int64_t bt = bth / H, h = bth % H, b = bt / T, kp = bt % T;
            const float* kr = k + bth * hd;
            const float* vr = v + bth * hd;
            int64_t qend = T;
            if (window > 0 && kp + window < T) qend = kp + window + 1;
            for (int64_t j = 0; j < hd; ++j) ak[j] = av[j] = 0.0;
            for (int64_t qp = kp; qp < qend; ++qp) {
                int64_t qi = (b * T + qp) * H + h;
                const float* qr = q + qi * hd;
                const float* gr = dout + qi * hd;
                double sc = 0.0, da = 0.0;
                for (int64_t j = 0; j < hd; ++j) {
                    sc += (double)qr[j] * (double)kr[j];
                    da += (double)gr[j] * (double)vr[j];
                }
                double a = exp(sc * (double)scale_f - (double)lse[qi]);
                double ds = a * (da - (double)dd[qi]);
                for (int64_t j = 0; j < hd; ++j) {
                    av[j] += a * (double)gr[j];
                    ak[j] += ds * (double)qr[j];
                }
            }
            for (int64_t j = 0; j < hd; ++j) {
                dk[bth * hd + j] = (float)(ak[j] * (double)scale_f);
                dv[bth * hd + j] = (float)av[j];
            }
        }
        free(ak);
        free(av);
    }
}

/* ops.mojo:486-497 */
void orc_relu_squared_fwd(float* out, const float* in, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) {
        float x = in[i];
        float r = x > 0.0f ? x : 0.0f;
        out[i] = r * r;
    }
}

/* ops.mojo:500-510 */
void orc_softcap_fwd(float* out, const float* in, float cap, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) out[i] = cap * (float)tanh((double)(in[i] / cap));
}

/* ops.mojo:516-541: gate = 2*sigmoid(sum_c W[h,c] x[t,c]), c < gate_channels. */
void orc_ve_gate_fwd(float* gate, const float* xn, const float* w, int64_t nt, int64_t nkv,
                     int64_t gc, int64_t C) {
    for (int64_t t = 0; t < nt; ++t)
        for (int64_t h = 0; h < nkv; ++h) {
            double acc = 0.0;
            for (int64_t c = 0; c < gc; ++c) acc += (double)w[h * gc + c] * (double)xn[t * C + c];
            float a = (float)acc;
            float sig = (float)(1.0 / (1.0 + exp(-(double)a)));
            gate[t * nkv + h] = 2.0f * sig;
        }
}

/* ops.mojo:544-560 (in place on v) */
void orc_ve_apply_fwd(float* v, const float* gate, const float* ve, int64_t nt, int64_t nkv, int64_t hd) {
    for (int64_t i = 0; i < nt * nkv * hd; ++i) v[i] += gate[i / hd] * ve[i];
}

/* ops.mojo:566-576 */
void orc_add_residual_fwd(float* out, const float* res, const float* in, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) out[i] = res[i] + in[i];
}

/* ops.mojo:579-594 */
void orc_scaled_add_fwd(float* out, const float* a, const float* b, const float* sa,
                        const float* sb, int64_t idx, int64_t size) {
    float s1 = sa[idx], s2 = sb[idx];
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) out[i] = s1 * a[i] + s2 * b[i];
}

/* ops.mojo:672-740: loss = lse(row) - row[target]; target < 0 gives 0. */
void orc_cross_entropy_fwd(float* loss, const float* logits, const int64_t* targets,
                           int64_t nt, int64_t V) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < nt; ++t) {
        const float* row = logits + t * V;
        float mx = -INFINITY;
        for (int64_t i = 0; i < V; ++i)
            if (row[i] > mx) mx = row[i];
        double s = 0.0;
        for (int64_t i = 0; i < V; ++i) s += exp((double)(row[i] - mx));
        float lse = mx + (float)log(s);
        int64_t tg = targets[t];
        loss[t] = (tg >= 0 && tg < V) ? -row[tg] + lse : 0.0f;  /* tg >= V: ignored (the reference reads out of bounds) */
    }
}

/* ops.mojo:746-772 */
void orc_mean_reduce(float* out, const float* in, int64_t size) {
    double s = 0.0;
    for (int64_t i = 0; i < size; ++i) s += in[i];
    out[0] = (float)s / (float)size;
}

/* ops.mojo:778-864: grad = (softmax(capped) - onehot) * loss_scale, with no
 * softcap derivative (quirk Q4). */
void orc_cross_entropy_softcap_bwd(float* grad, const float* logits, const int64_t* targets,
                                   float cap, int64_t nt, int64_t V, float loss_scale) {
    (void)cap;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < nt; ++t) {
        const float* row = logits + t * V;
        float* g = grad + t * V;
        int64_t tg = targets[t];
        if (tg < 0 || tg >= V) {
            for (int64_t i = 0; i < V; ++i) g[i] = 0.0f;
            continue;
        }
        float mx = -INFINITY;
        for (int64_t i = 0; i < V; ++i)
            if (row[i] > mx) mx = row[i];
        double s = 0.0;
        for (int64_t i = 0; i < V; ++i) s += exp((double)(row[i] - mx));
        for (int64_t i = 0; i < V; ++i) {
            float sm = (float)(exp((double)(row[i] - mx)) / s);
            g[i] = (i == tg ? (sm - 1.0f) : sm) * loss_scale;
        }
    }
}

/* ops.mojo:1039-1085: dx = (dy - x * <dy,x> / (dim * rms^2)) / rms.
 * dx may alias dy (model.mojo:858, 892, 998). */
void orc_rmsnorm_bwd(float* dx, const float* dy, const float* x, const float* rms, int64_t rows,
                     int64_t dim) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        double dot = 0.0;
        for (int64_t i = 0; i < dim; ++i) dot += (double)dy[r * dim + i] * (double)x[r * dim + i];
        float dot_f = (float)dot;
        float rr = rms[r];
        float rms_sq = rr * rr;
        for (int64_t i = 0; i < dim; ++i) {
            float xv = x[r * dim + i], g = dy[r * dim + i];
            dx[r * dim + i] = (g - xv * dot_f / ((float)dim * rms_sq)) / rr;
        }
    }
}

/* ops.mojo:1126-1140 */
void orc_relu_squared_bwd(float* dx, const float* dy, const float* x, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) dx[i] = x[i] > 0.0f ? 2.0f * x[i] * dy[i] : 0.0f;
}

/* ops.mojo:1146-1164: G[idx[i], :] += dY[i, :].  The reference uses float
 * atomics (summation order undefined, Q11); this build fixes one order, which
 * the HIP kernel reproduces bit-exactly:
 *   tokens are sorted stably by id; the sorted list is cut into chunks that
 *   start at every position p with p % 64 == 0 or id[p] != id[p-1]; a chunk's
 *   rows are summed in token order starting from its first row; then
 *   G[v] = ((G[v] + chunk_0) + chunk_1) + ... over v's chunks in order. */
#define EMB_CHUNK 64
void orc_embedding_bwd(float* gw, const float* dy, const int64_t* idx, int64_t nt, int64_t dim) {
    if (nt <= 0) return;
    /* stable counting sort by id */
    int64_t vmax = 0;
    for (int64_t t = 0; t < nt; ++t)
        if (idx[t] > vmax) vmax = idx[t];
    int64_t* cnt = (int64_t*)calloc((size_t)(vmax + 2), sizeof(int64_t));
    int64_t* order = (int64_t*)malloc((size_t)nt * sizeof(int64_t));
    for (int64_t t = 0; t < nt; ++t) cnt[idx[t] + 1]++;
    for (int64_t v = 0; v <= vmax; ++v) cnt[v + 1] += cnt[v];
    for (int64_t t = 0; t < nt; ++t) order[cnt[idx[t]]++] = t;
    free(cnt);
    float* part = (float*)malloc((size_t)dim * sizeof(float));
    int64_t p = 0;
    while (p < nt) {
        const int64_t v = idx[order[p]];
        int64_t end = p;
        while (end < nt && idx[order[end]] == v) ++end;
        float* row = gw + v * dim;
        for (int64_t c = p; c < end;) {
            int64_t q = c + 1;
            while (q < end && (q % EMB_CHUNK) != 0) ++q;
            for (int64_t d = 0; d < dim; ++d) part[d] = dy[order[c] * dim + d];
            for (int64_t r = c + 1; r < q; ++r)
                for (int64_t d = 0; d < dim; ++d) part[d] += dy[order[r] * dim + d];
            for (int64_t d = 0; d < dim; ++d) row[d] += part[d];
            c = q;
        }
        p = end;
    }
    free(part);
    free(order);
}

/* ops.mojo:1170-1190 (assign both outputs; ga may alias g) */
void orc_scaled_add_bwd(float* ga, float* gb, const float* g, const float* sa, const float* sb,
                        int64_t idx, int64_t size) {
    float s1 = sa[idx], s2 = sb[idx];
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) {
        float gv = g[i];
        gb[i] = s2 * gv;
        ga[i] = s1 * gv;
    }
}

/* ops.mojo:1193-1237 */
void orc_ve_apply_bwd(float* gve, float* ggate, const float* gv, const float* gate, const float* ve,
                      int64_t nt, int64_t nkv, int64_t hd) {
    for (int64_t row = 0; row < nt * nkv; ++row) {
        float g = gate[row];
        double dg = 0.0;
        for (int64_t d = 0; d < hd; ++d) {
            float x = gv[row * hd + d];
            gve[row * hd + d] = g * x;
            dg += (double)ve[row * hd + d] * (double)x;
        }
        ggate[row] = (float)dg;
    }
}

/* ops.mojo:1240-1274: dz = gg*g*(1-g/2); gW[h,c] += sum_t dz x[t,c];
 * gx[t,c] += sum_h dz W[h,c] (accumulate, c < gate_channels). */
void orc_ve_gate_bwd(float* gxn, float* gw, const float* ggate, const float* gate, const float* xn,
                     const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C) {
    double* accw = (double*)calloc((size_t)(nkv * gc), sizeof(double));
    for (int64_t t = 0; t < nt; ++t) {
        for (int64_t c = 0; c < gc; ++c) {
            double ax = 0.0;
            for (int64_t h = 0; h < nkv; ++h) {
                float g = gate[t * nkv + h];
                float dz = ggate[t * nkv + h] * g * (1.0f - g / 2.0f);
                ax += (double)dz * (double)w[h * gc + c];
                accw[h * gc + c] += (double)dz * (double)xn[t * C + c];
            }
            gxn[t * C + c] += (float)ax;
        }
    }
    for (int64_t i = 0; i < nkv * gc; ++i) gw[i] += (float)accw[i];
    free(accw);
}

/* ops.mojo:1277-1308: gs[idx] += sum(g * x) */
void orc_scalar_grad_reduce(float* gs, const float* g, const float* x, int64_t idx, int64_t size) {
    double s = 0.0;
#pragma omp parallel for reduction(+ : s) schedule(static)
    for (int64_t i = 0; i < size; ++i) s += (double)g[i] * (double)x[i];
    gs[idx] += (float)s;
}

/* ops.mojo:1314-1322 */
void orc_zero_buffer(float* buf, int64_t size) { memset(buf, 0, (size_t)size * sizeof(float)); }

/* ===================== optimizer.mojo ===================== */

/* optimizer.mojo:27-57 */
void orc_adamw(float* p, const float* g, float* m, float* v, float lr, float b1, float b2, float eps,
               float wd, float bc1, float bc2, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) {
        float pv = p[i], gv = g[i];
        pv = pv * (1.0f - lr * wd);
        float mm = b1 * m[i] + (1.0f - b1) * gv;
        m[i] = mm;
        float vv = b2 * v[i] + (1.0f - b2) * gv * gv;
        v[i] = vv;
        p[i] = pv - lr * (mm / bc1) / (sqrtf(vv / bc2) + eps);
    }
}

/* optimizer.mojo:132-146 */
void orc_nesterov_momentum(float* out, const float* g, float* buf, float mu, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) {
        float gv = g[i];
        float m = mu * buf[i] + (1.0f - mu) * gv;
        buf[i] = m;
        out[i] = (1.0f - mu) * gv + mu * m;
    }
}

/* optimizer.mojo:149-180 */
void orc_normalize_frobenius(float* x, int64_t size) {
    double s = 0.0;
    for (int64_t i = 0; i < size; ++i) s += (double)x[i] * (double)x[i];
    float inv = 1.0f / (sqrtf((float)s) * 1.02f + 1e-6f);
    for (int64_t i = 0; i < size; ++i) x[i] = x[i] * inv;
}

/* optimizer.mojo:183-194 */
void orc_scale_add(float* out, const float* a, const float* b, float sa, float sb, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) out[i] = sa * a[i] + sb * b[i];
}

/* optimizer.mojo:197-210: cautious decay only where g*p >= 0. */
void orc_muon_update(float* p, const float* g, float lr, float wd, int64_t size) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < size; ++i) {
        float pv = p[i], gv = g[i];
        float decay = (gv * pv) >= 0.0f ? wd * pv : 0.0f;
        p[i] = pv - lr * (gv + decay);
    }
}

/* config.mojo:93-112 */
static const double POLAR_A[5] = {8.156554524902461, 4.042929935166739, 3.8916678022926607,
                                  3.285753657755655, 2.3465413258596377};
static const double POLAR_B[5] = {-22.48329292557795, -2.808917465908714, -2.772484153217685,
                                  -2.3681294933425376, -1.7097828382687081};
static const double POLAR_C[5] = {15.878769915207462, 0.5000178451051316, 0.5060648178503393,
                                  0.46449024233003106, 0.42323551169305323};

/* optimizer.mojo:255-342 (MuonState.step) for one [rows, cols] matrix. */
void orc_muon_step(float* param, float* grads, float* mbuf, int64_t rows, int64_t cols,
                   double initial_lr, double lrm, double momentum, double wd) {
    int64_t size = rows * cols;
    int64_t small = rows >= cols ? cols : rows;
    double aspect = (double)rows / (double)cols;
    float lr = (float)(initial_lr * lrm * (aspect > 1.0 ? sqrt(aspect) : 1.0));
    float* X = (float*)malloc((size_t)size * sizeof(float));
    float* A = (float*)malloc((size_t)small * small * sizeof(float));
    float* AA = (float*)malloc((size_t)small * small * sizeof(float));
    float* Bm = (float*)malloc((size_t)small * small * sizeof(float));
    orc_nesterov_momentum(X, grads, mbuf, (float)momentum, size);
    orc_normalize_frobenius(X, size);
    int tall = rows >= cols;
    for (int it = 0; it < 5; ++it) {
        float ca = (float)POLAR_A[it], cb = (float)POLAR_B[it], cc = (float)POLAR_C[it];
        if (tall) {
            memset(A, 0, (size_t)small * small * sizeof(float));
            orc_linear_bwd_dw(A, X, X, rows, cols, cols); /* A = X^T X */
        } else {
            orc_linear_fwd(A, X, X, rows, rows, cols); /* A = X X^T */
        }
        orc_linear_bwd_dx(AA, A, A, small, small, small); /* AA = A @ A */
        orc_scale_add(Bm, A, AA, cb, cc, small * small);
        if (tall) orc_linear_bwd_dx(grads, X, Bm, rows, cols, cols); /* X @ B */
        else orc_linear_bwd_dx(grads, Bm, X, rows, rows, cols);      /* B @ X */
        orc_scale_add(X, X, grads, ca, 1.0f, size);
    }
    orc_muon_update(param, X, lr, (float)wd, size);
    free(X);
    free(A);
    free(AA);
    free(Bm);
}

/* ===================== model.mojo init ===================== */

static inline uint64_t xs_mix(uint64_t s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s;
}

/* model.mojo:86-115 */
void orc_fill_normal(float* out, uint64_t seed, float std_, int64_t size) {
    const float PI = 3.14159265358979323846f;
    for (int64_t i = 0; i < size; ++i) {
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

/* model.mojo:118-134 */
void orc_fill_uniform(float* out, uint64_t seed, float lo, float hi, int64_t size) {
    for (int64_t i = 0; i < size; ++i) {
        uint64_t st = seed + (uint64_t)i * 6364136223846793005ULL + 1442695040888963407ULL;
        st = xs_mix(st);
        float u = (float)(st & 0xFFFFFFULL) / 16777216.0f;
        float span = hi - lo;
        float prod = u * span;
        out[i] = lo + prod;
    }
}

/* model.mojo:137-157 */
void orc_fill_zeros(float* out, int64_t size) { memset(out, 0, (size_t)size * sizeof(float)); }
void orc_fill_value(float* out, float value, int64_t size) {
    for (int64_t i = 0; i < size; ++i) out[i] = value;
}

/* model.mojo:57-81: f64 table, cast to f32. */
void orc_precompute_rope(float* cos_t, float* sin_t, int64_t seq_len, int64_t head_dim, double base) {
    int64_t half = head_dim / 2;
    for (int64_t t = 0; t < seq_len; ++t)
        for (int64_t d = 0; d < half; ++d) {
            double freq = (double)t / pow(base, (double)(2 * d) / (double)head_dim);
            cos_t[t * half + d] = (float)cos(freq);
            sin_t[t * half + d] = (float)sin(freq);
        }
}

/* ===================== whole model ===================== */

#define VE_GATE_CHANNELS 32 /* config.mojo:64 */
#define MLP_EXPANSION 4     /* config.mojo:63 */
#define MAX_TENSORS 256

enum { T_WTE = 0, T_LM, T_RES, T_X0, T_Q, T_K, T_V, T_PROJ, T_FC, T_MLPP, T_VE, T_GATE };

typedef struct {
    int64_t offset, size, rows, cols;
    int kind, layer;
    char name[32];
} orc_tensor;

typedef struct {
    float *saved_x, *saved_xn_attn, *saved_q, *saved_k, *saved_v, *saved_lse, *saved_attn_out;
    float *saved_xn_mlp, *saved_mlp_hidden, *saved_mlp_act, *saved_rms_attn, *saved_rms_mlp;
    float *saved_ve, *saved_gate;
} orc_layer_bufs;

struct orc_model {
    orc_config c;
    int64_t B, T, BT, rope_period;
    int64_t nt;
    orc_tensor t[MAX_TENSORS];
    int64_t nparams;
    float *params, *grads;
    /* tensor indices */
    int64_t i_wte, i_lm, i_res, i_x0;
    int64_t i_q[64], i_k[64], i_v[64], i_proj[64], i_fc[64], i_mlpp[64], i_ve[64], i_gate[64];
    float *rope_cos, *rope_sin;
    int64_t rope_rows;
    /* activations */
    float *x, *x0, *x_norm, *rms, *q, *k, *v, *lse, *d_buf, *attn_out, *proj_out, *mlp_hidden,
        *mlp_act, *mlp_out, *logits, *loss, mean_loss;
    orc_layer_bufs* L;
    float *saved_x_pre_final, *saved_rms_final, *saved_x_final;
    float *grad_x, *grad_x0, *grad_logits, *grad_attn_out, *grad_q, *grad_k, *grad_v, *grad_x_norm,
        *grad_mlp_out, *grad_mlp_act, *grad_mlp_hidden, *ve_buf, *ve_gate_buf, *grad_gate, *grad_ve;
    /* optimizer state */
    float *adam_m, *adam_v, *muon_buf;
    int64_t adam_step;
    /* sum_i |g_i x_i| of the last backward's scalar-gradient reductions:
     * the L1 mass that bounds their rounding sensitivity (tests only) */
    double *l1_res, *l1_x0;
};

static int has_ve(const orc_config* c, int64_t i) { return (i % 2) == ((c->n_layer - 1) % 2); } /* config.mojo:45-47 */
static int64_t window_size(const orc_config* c, int64_t i) {                                 /* config.mojo:49-55 */
    if (i == c->n_layer - 1) return c->sequence_len;
    if (i % 4 < 3) return c->sequence_len / 2;
    return c->sequence_len;
}

static int64_t add_tensor(orc_model* m, int kind, int layer, int64_t rows, int64_t cols, const char* nm) {
    int64_t i = m->nt++;
    orc_tensor* t = &m->t[i];
    t->offset = m->nparams;
    t->rows = rows;
    t->cols = cols;
    t->size = rows * cols;
    t->kind = kind;
    t->layer = layer;
    if (layer >= 0) snprintf(t->name, sizeof(t->name), "h%d.%s", layer, nm);
    else snprintf(t->name, sizeof(t->name), "%s", nm);
    m->nparams += t->size;
    return i;
}

static float* fz(int64_t n) { return (float*)calloc((size_t)(n > 0 ? n : 1), sizeof(float)); }

orc_model* orc_model_create(const orc_config* cfg, int64_t B, int64_t T, int64_t rope_period) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    m->B = B;
    m->T = T;
    m->BT = B * T;
    m->rope_period = rope_period;
    int64_t C = cfg->n_embd, V = cfg->vocab_size, Lr = cfg->n_layer, kv = cfg->kv_dim;
    int64_t F = MLP_EXPANSION * C, BT = B * T, H = cfg->n_head;
    /* Tensor order = the order train.mojo registers optimizer groups. */
    m->i_wte = add_tensor(m, T_WTE, -1, V, C, "wte");
    m->i_lm = add_tensor(m, T_LM, -1, V, C, "lm_head");
    m->i_res = add_tensor(m, T_RES, -1, 1, Lr, "resid_lambdas");
    m->i_x0 = add_tensor(m, T_X0, -1, 1, Lr, "x0_lambdas");
    for (int64_t i = 0; i < Lr; ++i) {
        m->i_q[i] = add_tensor(m, T_Q, (int)i, C, C, "c_q");
        m->i_k[i] = add_tensor(m, T_K, (int)i, kv, C, "c_k");
        m->i_v[i] = add_tensor(m, T_V, (int)i, kv, C, "c_v");
        m->i_proj[i] = add_tensor(m, T_PROJ, (int)i, C, C, "c_proj");
        m->i_fc[i] = add_tensor(m, T_FC, (int)i, F, C, "c_fc");
        m->i_mlpp[i] = add_tensor(m, T_MLPP, (int)i, C, F, "mlp_proj");
        if (has_ve(cfg, i)) {
            m->i_ve[i] = add_tensor(m, T_VE, (int)i, V, kv, "value_embeds");
            m->i_gate[i] = add_tensor(m, T_GATE, (int)i, cfg->n_kv_head, VE_GATE_CHANNELS, "ve_gate");
        } else {
            m->i_ve[i] = m->i_gate[i] = -1;
        }
    }
    m->l1_res = (double*)calloc((size_t)Lr, sizeof(double));
    m->l1_x0 = (double*)calloc((size_t)Lr, sizeof(double));
    m->params = fz(m->nparams);
    m->grads = fz(m->nparams);
    m->adam_m = fz(m->nparams);
    m->adam_v = fz(m->nparams);
    m->muon_buf = fz(m->nparams);
    int64_t half = cfg->head_dim / 2;
    m->rope_rows = rope_period > 0 ? rope_period : 2048; /* MAX_SEQ_LEN, model.mojo:307 */
    if (rope_period == 0 && BT > m->rope_rows) m->rope_rows = BT; /* avoid Q3's OOB read */
    m->rope_cos = fz(m->rope_rows * half);
    m->rope_sin = fz(m->rope_rows * half);
    m->x = fz(BT * C); m->x0 = fz(BT * C); m->x_norm = fz(BT * C); m->rms = fz(BT * H);
    m->q = fz(BT * C); m->k = fz(BT * kv); m->v = fz(BT * kv);
    m->lse = fz(BT * H); m->d_buf = fz(BT * H); m->attn_out = fz(BT * C); m->proj_out = fz(BT * C);
    m->mlp_hidden = fz(BT * F); m->mlp_act = fz(BT * F); m->mlp_out = fz(BT * C);
    m->logits = fz(BT * V); m->loss = fz(BT);
    m->L = (orc_layer_bufs*)calloc((size_t)Lr, sizeof(orc_layer_bufs));
    for (int64_t i = 0; i < Lr; ++i) {
        orc_layer_bufs* b = &m->L[i];
        b->saved_x = fz(BT * C); b->saved_xn_attn = fz(BT * C); b->saved_q = fz(BT * C);
        b->saved_k = fz(BT * kv); b->saved_v = fz(BT * kv); b->saved_lse = fz(BT * H);
        b->saved_attn_out = fz(BT * C); b->saved_xn_mlp = fz(BT * C);
        b->saved_mlp_hidden = fz(BT * F); b->saved_mlp_act = fz(BT * F);
        b->saved_rms_attn = fz(BT); b->saved_rms_mlp = fz(BT);
        b->saved_ve = fz(BT * kv); b->saved_gate = fz(BT * H);
    }
    m->saved_x_pre_final = fz(BT * C); m->saved_rms_final = fz(BT); m->saved_x_final = fz(BT * C);
    m->grad_x = fz(BT * C); m->grad_x0 = fz(BT * C); m->grad_logits = fz(BT * V);
    m->grad_attn_out = fz(BT * C); m->grad_q = fz(BT * C); m->grad_k = fz(BT * kv); m->grad_v = fz(BT * kv);
    m->grad_x_norm = fz(BT * C); m->grad_mlp_out = fz(BT * C); m->grad_mlp_act = fz(BT * F);
    m->grad_mlp_hidden = fz(BT * F); m->ve_buf = fz(BT * kv); m->ve_gate_buf = fz(BT * H);
    m->grad_gate = fz(BT * H); m->grad_ve = fz(BT * kv);
    return m;
}

void orc_model_destroy(orc_model* m) {
    if (!m) return;
    free(m->l1_res); free(m->l1_x0);
    free(m->params); free(m->grads); free(m->adam_m); free(m->adam_v); free(m->muon_buf);
    free(m->rope_cos); free(m->rope_sin);
    free(m->x); free(m->x0); free(m->x_norm); free(m->rms); free(m->q); free(m->k); free(m->v);
    free(m->lse); free(m->d_buf); free(m->attn_out); free(m->proj_out); free(m->mlp_hidden);
    free(m->mlp_act); free(m->mlp_out); free(m->logits); free(m->loss);
    for (int64_t i = 0; i < m->c.n_layer; ++i) {
        orc_layer_bufs* b = &m->L[i];
        free(b->saved_x); free(b->saved_xn_attn); free(b->saved_q); free(b->saved_k); free(b->saved_v);
        free(b->saved_lse); free(b->saved_attn_out); free(b->saved_xn_mlp); free(b->saved_mlp_hidden);
        free(b->saved_mlp_act); free(b->saved_rms_attn); free(b->saved_rms_mlp); free(b->saved_ve);
        free(b->saved_gate);
    }
    free(m->L);
    free(m->saved_x_pre_final); free(m->saved_rms_final); free(m->saved_x_final);
    free(m->grad_x); free(m->grad_x0); free(m->grad_logits); free(m->grad_attn_out); free(m->grad_q);
    free(m->grad_k); free(m->grad_v); free(m->grad_x_norm); free(m->grad_mlp_out); free(m->grad_mlp_act);
    free(m->grad_mlp_hidden); free(m->ve_buf); free(m->ve_gate_buf); free(m->grad_gate); free(m->grad_ve);
    free(m);
}

int64_t orc_model_num_tensors(const orc_model* m) { return m->nt; }
int64_t orc_model_tensor_info(const orc_model* m, int64_t i, int64_t* offset, const char** name) {
    if (offset) *offset = m->t[i].offset;
    if (name) *name = m->t[i].name;
    return m->t[i].size;
}
int64_t orc_model_num_params(const orc_model* m) { return m->nparams; }
float* orc_model_params(orc_model* m) { return m->params; }
float* orc_model_grads(orc_model* m) { return m->grads; }
const float* orc_model_token_loss(const orc_model* m) { return m->loss; }
int64_t orc_model_adam_step(const orc_model* m) { return m->adam_step; }
/* Named activation buffers of the last forward/backward (tests only). */
float* orc_model_buffer(orc_model* m, const char* name, int64_t layer) {
    orc_layer_bufs* b = (layer >= 0 && layer < m->c.n_layer) ? &m->L[layer] : NULL;
    if (!strcmp(name, "q") && b) return b->saved_q;
    if (!strcmp(name, "k") && b) return b->saved_k;
    if (!strcmp(name, "v") && b) return b->saved_v;
    if (!strcmp(name, "attn_out") && b) return b->saved_attn_out;
    if (!strcmp(name, "lse") && b) return b->saved_lse;
    if (!strcmp(name, "grad_attn_out")) return m->grad_attn_out;
    if (!strcmp(name, "grad_q")) return m->grad_q;
    return NULL;
}

void orc_model_scalar_grad_l1(const orc_model* m, double* res, double* x0) {
    for (int64_t i = 0; i < m->c.n_layer; ++i) {
        res[i] = m->l1_res[i];
        x0[i] = m->l1_x0[i];
    }
}

#define P(i) (m->params + m->t[(i)].offset)
#define G(i) (m->grads + m->t[(i)].offset)

/* model.mojo:337-427 */
void orc_model_init_weights(orc_model* m, uint64_t seed0) {
    const orc_config* c = &m->c;
    int64_t C = c->n_embd, V = c->vocab_size, Lr = c->n_layer, kv = c->kv_dim, F = MLP_EXPANSION * C;
    float s = (float)(sqrt(3.0) * pow((double)C, -0.5));
    uint64_t seed = seed0;
    orc_fill_normal(P(m->i_wte), seed, 1.0f, V * C); seed++;
    orc_fill_normal(P(m->i_lm), seed, 0.001f, V * C); seed++;
    orc_fill_value(P(m->i_res), 1.0f, Lr);
    orc_fill_value(P(m->i_x0), 0.1f, Lr);
    for (int64_t i = 0; i < Lr; ++i) {
        orc_fill_uniform(P(m->i_q[i]), seed, -s, s, C * C); seed++;
        orc_fill_uniform(P(m->i_k[i]), seed, -s, s, kv * C); seed++;
        orc_fill_uniform(P(m->i_v[i]), seed, -s, s, kv * C); seed++;
        orc_fill_zeros(P(m->i_proj[i]), C * C);
        orc_fill_uniform(P(m->i_fc[i]), seed, -s, s, F * C); seed++;
        orc_fill_zeros(P(m->i_mlpp[i]), C * F);
        if (has_ve(c, i)) {
            orc_fill_uniform(P(m->i_ve[i]), seed, -s, s, V * kv); seed++;
            orc_fill_zeros(P(m->i_gate[i]), c->n_kv_head * VE_GATE_CHANNELS);
        }
    }
    orc_precompute_rope(m->rope_cos, m->rope_sin, m->rope_rows, c->head_dim, 10000.0); /* config.mojo:87 */
}

void orc_model_zero_grads(orc_model* m) { memset(m->grads, 0, (size_t)m->nparams * sizeof(float)); }

/* RoPE over [BT, H, hd] with the table row chosen by rope_period. */
static void model_rope(orc_model* m, float* x, int fwd) {
    int64_t H = m->c.n_head, hd = m->c.head_dim, half = hd / 2;
    int64_t period = m->rope_period > 0 ? m->rope_period : m->BT;
    for (int64_t tok0 = 0; tok0 < m->BT; tok0 += period) {
        int64_t n = m->BT - tok0 < period ? m->BT - tok0 : period;
        float* xs = x + tok0 * H * hd;
        if (fwd) orc_rope_fwd(xs, xs, m->rope_cos, m->rope_sin, n, H, hd);
        else orc_rope_bwd(xs, xs, m->rope_cos, m->rope_sin, n, H, hd);
    }
    (void)half;
}

#define CPY(dst, src, n) memcpy((dst), (src), (size_t)(n) * sizeof(float))

/* model.mojo:576-772 */
float orc_model_forward(orc_model* m, const int64_t* inputs, const int64_t* targets) {
    const orc_config* c = &m->c;
    int64_t C = c->n_embd, V = c->vocab_size, BT = m->BT, H = c->n_head, hd = c->head_dim;
    int64_t kv = c->kv_dim, F = MLP_EXPANSION * C;
    orc_embedding_fwd(m->x, P(m->i_wte), inputs, BT, C);
    orc_rmsnorm_fwd(m->x, m->rms, m->x, BT, C);
    CPY(m->x0, m->x, BT * C);
    for (int64_t i = 0; i < c->n_layer; ++i) {
        orc_layer_bufs* b = &m->L[i];
        int64_t ws = window_size(c, i);
        orc_scaled_add_fwd(m->x, m->x, m->x0, P(m->i_res), P(m->i_x0), i, BT * C);
        CPY(b->saved_x, m->x, BT * C);
        orc_rmsnorm_fwd(b->saved_xn_attn, b->saved_rms_attn, m->x, BT, C);
        CPY(m->x_norm, b->saved_xn_attn, BT * C);
        orc_linear_fwd(m->q, m->x_norm, P(m->i_q[i]), BT, C, C);
        orc_linear_fwd(m->k, m->x_norm, P(m->i_k[i]), BT, kv, C);
        orc_linear_fwd(m->v, m->x_norm, P(m->i_v[i]), BT, kv, C);
        if (has_ve(c, i)) {
            orc_embedding_fwd(m->ve_buf, P(m->i_ve[i]), inputs, BT, kv);
            orc_ve_gate_fwd(m->ve_gate_buf, m->x_norm, P(m->i_gate[i]), BT, H, VE_GATE_CHANNELS, C);
            CPY(b->saved_ve, m->ve_buf, BT * kv);
            CPY(b->saved_gate, m->ve_gate_buf, BT * H);
            orc_ve_apply_fwd(m->v, m->ve_gate_buf, m->ve_buf, BT, H, hd);
        }
        model_rope(m, m->q, 1);
        model_rope(m, m->k, 1);
        orc_rmsnorm_fwd(m->q, m->rms, m->q, BT * H, hd);
        orc_rmsnorm_fwd(m->k, m->rms, m->k, BT * H, hd);
        CPY(b->saved_q, m->q, BT * C);
        CPY(b->saved_k, m->k, BT * kv);
        CPY(b->saved_v, m->v, BT * kv);
        orc_flash_attn_fwd(m->attn_out, m->lse, m->q, m->k, m->v, m->B, m->T, H, hd, ws);
        CPY(b->saved_lse, m->lse, BT * H);
        CPY(b->saved_attn_out, m->attn_out, BT * C);
        orc_linear_fwd(m->proj_out, m->attn_out, P(m->i_proj[i]), BT, C, C);
        orc_add_residual_fwd(m->x, m->x, m->proj_out, BT * C);
        orc_rmsnorm_fwd(m->x_norm, b->saved_rms_mlp, m->x, BT, C);
        CPY(b->saved_xn_mlp, m->x_norm, BT * C);
        orc_linear_fwd(m->mlp_hidden, m->x_norm, P(m->i_fc[i]), BT, F, C);
        CPY(b->saved_mlp_hidden, m->mlp_hidden, BT * F);
        orc_relu_squared_fwd(m->mlp_act, m->mlp_hidden, BT * F);
        CPY(b->saved_mlp_act, m->mlp_act, BT * F);
        orc_linear_fwd(m->mlp_out, m->mlp_act, P(m->i_mlpp[i]), BT, C, F);
        orc_add_residual_fwd(m->x, m->x, m->mlp_out, BT * C);
    }
    CPY(m->saved_x_pre_final, m->x, BT * C);
    orc_rmsnorm_fwd(m->x, m->saved_rms_final, m->x, BT, C);
    CPY(m->saved_x_final, m->x, BT * C);
    orc_linear_fwd(m->logits, m->x, P(m->i_lm), BT, V, C);
    orc_softcap_fwd(m->logits, m->logits, 15.0f, BT * V); /* config.mojo:86 */
    orc_cross_entropy_fwd(m->loss, m->logits, targets, BT, V);
    orc_mean_reduce(&m->mean_loss, m->loss, BT);
    return m->mean_loss;
}

/* model.mojo:819-1037, with quirks Q4-Q10 reproduced. */
void orc_model_backward(orc_model* m, const int64_t* inputs, const int64_t* targets, float loss_scale) {
    const orc_config* c = &m->c;
    int64_t C = c->n_embd, V = c->vocab_size, BT = m->BT, H = c->n_head, hd = c->head_dim;
    int64_t kv = c->kv_dim, F = MLP_EXPANSION * C;
    orc_cross_entropy_softcap_bwd(m->grad_logits, m->logits, targets, 15.0f, BT, V, loss_scale);
    orc_linear_bwd_dx(m->grad_x, m->grad_logits, P(m->i_lm), BT, V, C);
    orc_linear_bwd_dw(G(m->i_lm), m->grad_logits, m->saved_x_final, BT, V, C);
    orc_rmsnorm_bwd(m->grad_x, m->grad_x, m->saved_x_pre_final, m->saved_rms_final, BT, C);
    orc_zero_buffer(m->grad_x0, BT * C);
    for (int64_t r = 0; r < c->n_layer; ++r) {
        int64_t i = c->n_layer - 1 - r;
        orc_layer_bufs* b = &m->L[i];
        CPY(m->grad_mlp_out, m->grad_x, BT * C);
        orc_linear_bwd_dx(m->grad_mlp_act, m->grad_mlp_out, P(m->i_mlpp[i]), BT, C, F);
        orc_linear_bwd_dw(G(m->i_mlpp[i]), m->grad_mlp_out, b->saved_mlp_act, BT, C, F);
        orc_relu_squared_bwd(m->grad_mlp_hidden, m->grad_mlp_act, b->saved_mlp_hidden, BT * F);
        orc_linear_bwd_dx(m->grad_x_norm, m->grad_mlp_hidden, P(m->i_fc[i]), BT, F, C);
        orc_linear_bwd_dw(G(m->i_fc[i]), m->grad_mlp_hidden, b->saved_xn_mlp, BT, F, C);
        /* Q7: saved_x (pre-attention x) with the MLP norm's rms */
        orc_rmsnorm_bwd(m->grad_x_norm, m->grad_x_norm, b->saved_x, b->saved_rms_mlp, BT, C);
        orc_add_residual_fwd(m->grad_x, m->grad_x, m->grad_x_norm, BT * C);
        CPY(m->grad_attn_out, m->grad_x, BT * C);
        orc_linear_bwd_dx(m->grad_attn_out, m->grad_attn_out, P(m->i_proj[i]), BT, C, C); /* Q2 */
        orc_linear_bwd_dw(G(m->i_proj[i]), m->grad_x, b->saved_attn_out, BT, C, C);
        int64_t ws = window_size(c, i);
        orc_flash_attn_bwd_precompute_d(m->d_buf, b->saved_attn_out, m->grad_attn_out, m->B, m->T, H, hd);
        orc_flash_attn_bwd_dq(m->grad_q, b->saved_q, b->saved_k, b->saved_v, m->grad_attn_out,
                              b->saved_lse, m->d_buf, m->B, m->T, H, hd, ws);
        orc_flash_attn_bwd_dkv(m->grad_k, m->grad_v, b->saved_q, b->saved_k, b->saved_v,
                               m->grad_attn_out, b->saved_lse, m->d_buf, m->B, m->T, H, hd, ws);
        /* Q6: q/k per-head norm backward skipped */
        if (has_ve(c, i)) {
            orc_ve_apply_bwd(m->grad_ve, m->grad_gate, m->grad_v, b->saved_gate, b->saved_ve, BT, H, hd);
            orc_embedding_bwd(G(m->i_ve[i]), m->grad_ve, inputs, BT, kv);
        }
        model_rope(m, m->grad_q, 0);
        model_rope(m, m->grad_k, 0);
        orc_linear_bwd_dx(m->grad_x_norm, m->grad_q, P(m->i_q[i]), BT, C, C);
        orc_linear_bwd_dw(G(m->i_q[i]), m->grad_q, b->saved_xn_attn, BT, C, C);
        orc_linear_bwd_dx(m->grad_mlp_out, m->grad_k, P(m->i_k[i]), BT, kv, C);
        orc_add_residual_fwd(m->grad_x_norm, m->grad_x_norm, m->grad_mlp_out, BT * C);
        orc_linear_bwd_dw(G(m->i_k[i]), m->grad_k, b->saved_xn_attn, BT, kv, C);
        orc_linear_bwd_dx(m->grad_mlp_out, m->grad_v, P(m->i_v[i]), BT, kv, C);
        orc_add_residual_fwd(m->grad_x_norm, m->grad_x_norm, m->grad_mlp_out, BT * C);
        orc_linear_bwd_dw(G(m->i_v[i]), m->grad_v, b->saved_xn_attn, BT, kv, C);
        if (has_ve(c, i))
            orc_ve_gate_bwd(m->grad_x_norm, G(m->i_gate[i]), m->grad_gate, b->saved_gate, b->saved_xn_attn,
                            P(m->i_gate[i]), BT, H, VE_GATE_CHANNELS, C);
        orc_rmsnorm_bwd(m->grad_x_norm, m->grad_x_norm, b->saved_x, b->saved_rms_attn, BT, C);
        orc_add_residual_fwd(m->grad_x, m->grad_x, m->grad_x_norm, BT * C);
        /* Q8: post-scaled-add saved_x; Q9: grad_x0 assigned, never consumed */
        orc_scalar_grad_reduce(G(m->i_res), m->grad_x, b->saved_x, i, BT * C);
        orc_scalar_grad_reduce(G(m->i_x0), m->grad_x, m->x0, i, BT * C);
        {
            double a1 = 0.0, a2 = 0.0;
            for (int64_t j = 0; j < BT * C; ++j) {
                a1 += fabs((double)m->grad_x[j] * (double)b->saved_x[j]);
                a2 += fabs((double)m->grad_x[j] * (double)m->x0[j]);
            }
            m->l1_res[i] = a1;
            m->l1_x0[i] = a2;
        }
        orc_scaled_add_bwd(m->grad_x, m->grad_x0, m->grad_x, P(m->i_res), P(m->i_x0), i, BT * C);
    }
    /* Q10: embedding norm backward skipped */
    orc_embedding_bwd(G(m->i_wte), m->grad_x, inputs, BT, C);
}

/* train.mojo:25-33 */
static double lr_multiplier(double progress) {
    const double WARMUP = 0.0, WARMDOWN = 0.5, FINAL = 0.0; /* config.mojo:81-83 */
    if (progress < WARMUP) return WARMUP > 0 ? progress / WARMUP : 1.0;
    if (progress < 1.0 - WARMDOWN) return 1.0;
    double cd = (1.0 - progress) / WARMDOWN;
    return cd + (1.0 - cd) * FINAL;
}

/* optimizer.mojo:103-127 (step_group) */
static void adam_group(orc_model* m, int64_t ti, double lr_g, double b1d, double lrm) {
    float lr = (float)(lr_g * lrm);
    float b1 = (float)b1d, b2 = (float)0.95; /* config.mojo:73 */
    float bc1 = 1.0f, bc2 = 1.0f;
    for (int64_t s = 0; s < m->adam_step; ++s) {
        bc1 *= b1;
        bc2 *= b2;
    }
    int64_t off = m->t[ti].offset;
    orc_adamw(m->params + off, m->grads + off, m->adam_m + off, m->adam_v + off, lr, b1, b2,
              (float)1e-10, 0.0f, 1.0f - bc1, 1.0f - bc2, m->t[ti].size);
}

/* train.mojo:246-281 */
void orc_model_optimizer_step(orc_model* m, double progress) {
    const orc_config* c = &m->c;
    if (progress > 1.0) progress = 1.0;
    double lrm = lr_multiplier(progress);
    double lr_scale = pow((double)c->n_embd / 768.0, -0.5); /* train.mojo:167 */
    m->adam_step += 1;
    adam_group(m, m->i_lm, 0.004 * lr_scale, 0.8, lrm);
    adam_group(m, m->i_wte, 0.6 * lr_scale, 0.8, lrm);
    adam_group(m, m->i_res, 0.5 * 0.01, 0.8, lrm);
    adam_group(m, m->i_x0, 0.5, 0.96, lrm);
    for (int64_t i = 0; i < c->n_layer; ++i)
        if (has_ve(c, i)) {
            adam_group(m, m->i_ve[i], 0.6 * lr_scale, 0.8, lrm);
            adam_group(m, m->i_gate[i], 0.04, 0.8, lrm);
        }
    double frac = (double)m->adam_step / 300.0;
    if (frac > 1.0) frac = 1.0;
    double mu = (1.0 - frac) * 0.85 + frac * 0.95;
    double wd = 0.2 * (1.0 - progress);
    for (int64_t i = 0; i < c->n_layer; ++i) {
        int64_t ids[6] = {m->i_q[i], m->i_k[i], m->i_v[i], m->i_proj[i], m->i_fc[i], m->i_mlpp[i]};
        for (int j = 0; j < 6; ++j) {
            orc_tensor* t = &m->t[ids[j]];
            orc_muon_step(m->params + t->offset, m->grads + t->offset, m->muon_buf + t->offset, t->rows,
                          t->cols, 0.04, lrm, mu, wd);
        }
    }
}

float orc_model_train_step(orc_model* m, const int64_t* inputs, const int64_t* targets, double progress) {
    orc_model_zero_grads(m);
    float loss = orc_model_forward(m, inputs, targets);
    orc_model_backward(m, inputs, targets, 1.0f);
    orc_model_optimizer_step(m, progress);
    return loss;
}
