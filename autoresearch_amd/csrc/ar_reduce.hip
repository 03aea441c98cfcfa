// ar_reduce.hip -- row-reduction kernels: RMSNorm fwd/bwd, softmax, cross
// entropy fwd/bwd, mean, the value-embedding gate kernels, the learned-scalar
// gradient reduction, the Frobenius normalisation and the deterministic
// embedding scatter.
//
// Reductions never use float atomics: multi-block sums write per-block
// partials in a fixed assignment and a second kernel adds them in a fixed
// order, so every result is run-to-run deterministic (the reference's float
// atomics, ops.mojo:1160-1164 / 1267-1274 / 1307-1308, are not).
#include "ar_internal.hpp"

using namespace ar;

namespace {

constexpr int kBlock = 256;
__host__ __device__ inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------- K2 rmsnorm_fwd (ops.mojo:61-104): one wave per row ----------------
template <bool VEC>
__global__ void rmsnorm_fwd_k(float* out, float* rms_out, const float* in, int64_t rows, int64_t dim) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
    for (int64_t r = wave; r < rows; r += nwaves) {
        const float* x = in + r * dim;
        float* y = out + r * dim;
        float ss = 0.f;
        if (VEC) {
            for (int64_t i = lane; i < dim / 4; i += kWave) {
                float4 v = reinterpret_cast<const float4*>(x)[i];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        } else {
            for (int64_t i = lane; i < dim; i += kWave) ss += x[i] * x[i];
        }
        ss = wave_sum(ss);
        const float rms = sqrtf(ss / (float)dim + 1e-5f);
        if (lane == 0 && rms_out) rms_out[r] = rms;
        if (VEC) {
            for (int64_t i = lane; i < dim / 4; i += kWave) {
                float4 v = reinterpret_cast<const float4*>(x)[i];
                reinterpret_cast<float4*>(y)[i] = make_float4(v.x / rms, v.y / rms, v.z / rms, v.w / rms);
            }
        } else {
            for (int64_t i = lane; i < dim; i += kWave) y[i] = x[i] / rms;
        }
    }
}

// ---------------- K21 rmsnorm_bwd (ops.mojo:1039-1085) ----------------
template <bool VEC>
__global__ void rmsnorm_bwd_k(float* dx, const float* dy, const float* x, const float* rms, int64_t rows,
                              int64_t dim) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
    for (int64_t r = wave; r < rows; r += nwaves) {
        const float* xr = x + r * dim;
        const float* gr = dy + r * dim;
        float* o = dx + r * dim;
        float dot = 0.f;
        if (VEC) {
            for (int64_t i = lane; i < dim / 4; i += kWave) {
                float4 a = reinterpret_cast<const float4*>(xr)[i];
                float4 g = reinterpret_cast<const float4*>(gr)[i];
                dot += a.x * g.x + a.y * g.y + a.z * g.z + a.w * g.w;
            }
        } else {
            for (int64_t i = lane; i < dim; i += kWave) dot += gr[i] * xr[i];
        }
        dot = wave_sum(dot);
        const float rr = rms[r];
        const float coef = dot / ((float)dim * (rr * rr));
        if (VEC) {
            for (int64_t i = lane; i < dim / 4; i += kWave) {
                float4 a = reinterpret_cast<const float4*>(xr)[i];
                float4 g = reinterpret_cast<const float4*>(gr)[i];
                reinterpret_cast<float4*>(o)[i] = make_float4((g.x - a.x * coef) / rr, (g.y - a.y * coef) / rr,
                                                              (g.z - a.z * coef) / rr, (g.w - a.w * coef) / rr);
            }
        } else {
            for (int64_t i = lane; i < dim; i += kWave) o[i] = (gr[i] - xr[i] * coef) / rr;
        }
    }
}

// Online (max, sum-exp) over one row by a block; every thread gets (m, s).
__device__ __forceinline__ void row_max_sumexp(const float* row, int64_t n, float* red, float& m_out, float& s_out) {
    float m = -INFINITY, s = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        float v = row[i];
        if (v > m) {
            s = s * __expf(m - v) + 1.f;
            m = v;
        } else {
            s += __expf(v - m);
        }
    }
    const float bm = block_max(m, red);
    s = (m == -INFINITY) ? 0.f : s * __expf(m - bm);
    const float bs = block_sum(s, red + 32);
    m_out = bm;
    s_out = bs;
}

// ---------------- K16 cross_entropy_fwd (ops.mojo:672-740) ----------------
__global__ void ce_fwd_k(float* loss, const float* logits, const int64_t* targets, int64_t V) {
    __shared__ float red[64];
    const int64_t t = blockIdx.x;
    const float* row = logits + t * V;
    float m, s;
    row_max_sumexp(row, V, red, m, s);
    if (threadIdx.x == 0) {
        const int64_t tg = targets[t];
        const float lse = m + logf(s);
        loss[t] = (tg >= 0 && tg < V) ? -row[tg] + lse : 0.f;  // out-of-range targets are ignored rows
    }
}

// ---------------- K18 cross_entropy_softcap_bwd (ops.mojo:778-864) ----------------
__global__ void ce_bwd_k(float* grad, const float* logits, const int64_t* targets, int64_t V, float loss_scale) {
    __shared__ float red[64];
    const int64_t t = blockIdx.x;
    const int64_t tg = targets[t];
    float* g = grad + t * V;
    if (tg < 0 || tg >= V) {
        for (int64_t i = threadIdx.x; i < V; i += blockDim.x) g[i] = 0.f;
        return;
    }
    const float* row = logits + t * V;
    float m, s;
    row_max_sumexp(row, V, red, m, s);
    for (int64_t i = threadIdx.x; i < V; i += blockDim.x) {
        const float sm = __expf(row[i] - m) / s;
        g[i] = (i == tg ? sm - 1.0f : sm) * loss_scale;
    }
}

// ---------------- K15 softmax_fwd (ops.mojo:600-666) ----------------
__global__ void softmax_k(float* out, const float* in, int64_t cols) {
    __shared__ float red[64];
    const int64_t r = blockIdx.x;
    float m, s;
    row_max_sumexp(in + r * cols, cols, red, m, s);
    for (int64_t i = threadIdx.x; i < cols; i += blockDim.x) out[r * cols + i] = __expf(in[r * cols + i] - m) / s;
}

// ---------------- fixed-order multi-block sums ----------------
// kSumBlocks (ar_internal.hpp) is fixed: the partial assignment never depends
// on the device.

// partial[b] = sum over i in block b's grid-stride set of a[i]*(b? b[i] : a[i]) or a[i]
__global__ void dot_partial_k(float* partial, const float* a, const float* b, int64_t n, int mode) {
    __shared__ float red[16];
    float s = 0.f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float x = a[i];
        s += mode == 0 ? x : (mode == 1 ? x * x : x * b[i]);
    }
    s = block_sum(s, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

// mode 0: out[idx] = total / n (mean); mode 1: out[idx] += total;
// mode 2: out[0] = 1 / (sqrt(total) * 1.02 + 1e-6) (Frobenius scale, optimizer.mojo:178)
__global__ void finish_sum_k(float* out, const float* partial, int np, int64_t idx, int64_t n, int mode) {
    __shared__ float red[16];
    float s = 0.f;
    for (int i = threadIdx.x; i < np; i += blockDim.x) s += partial[i];
    s = block_sum(s, red);
    if (threadIdx.x == 0) {
        if (mode == 0) out[idx] = s / (float)n;
        else if (mode == 1) out[idx] += s;
        else out[0] = 1.0f / (sqrtf(s) * 1.02f + 1e-6f);
    }
}

__global__ void scale_by_device_scalar_k(float* x, const float* scale, int64_t n) {
    const float sc = scale[0];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        x[i] = x[i] * sc;
}

// ---------------- K6 flash_attn_bwd_precompute_d (ops.mojo:329-346) ----------------
// ROUND_DO: dO is rounded to bf16 first, as the bf16 backward rounds it for
// dP = dO V^T.  D must equal sum_j P_j dP_j for dS_j = P_j (dP_j - D) to be
// unbiased; a D from the unrounded dO differs from that sum by the same amount
// for every key of the row, which the attention-weighted mean key amplifies.
template <bool ROUND_DO>
__global__ void precompute_d_k(float* d, const float* o, const float* g, int64_t rows, int64_t hd) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
    for (int64_t r = wave; r < rows; r += nwaves) {
        float s = 0.f;
        for (int64_t i = lane; i < hd; i += kWave) {
            const float gv = ROUND_DO ? (float)(bf16)g[r * hd + i] : g[r * hd + i];
            s += o[r * hd + i] * gv;
        }
        s = wave_sum(s);
        if (lane == 0) d[r] = s;
    }
}

// ---------------- K11 ve_gate_fwd (ops.mojo:516-541) ----------------
__global__ void ve_gate_fwd_k(float* gate, const float* xn, const float* w, int64_t nt, int64_t nkv, int64_t gc,
                              int64_t C) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nt * nkv;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = i / nkv, h = i % nkv;
        float acc = 0.f;
        for (int64_t c = 0; c < gc; ++c) acc += w[h * gc + c] * xn[t * C + c];
        gate[i] = 2.0f * (1.0f / (1.0f + __expf(-acc)));
    }
}

// ---------------- K26 ve_apply_bwd (ops.mojo:1193-1237): one wave per (t,h) ----------------
__global__ void ve_apply_bwd_k(float* gve, float* ggate, const float* gv, const float* gate, const float* ve,
                               int64_t rows, int64_t hd) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) / kWave;
    for (int64_t r = wave; r < rows; r += nwaves) {
        const float g = gate[r];
        float dg = 0.f;
        for (int64_t d = lane; d < hd; d += kWave) {
            const float x = gv[r * hd + d];
            gve[r * hd + d] = g * x;
            dg += ve[r * hd + d] * x;
        }
        dg = wave_sum(dg);
        if (lane == 0) ggate[r] = dg;
    }
}

// ---------------- K27 ve_gate_bwd (ops.mojo:1240-1274), deterministic ----------------
// Block b owns a fixed token range.  Thread (c = tid % CW, j = tid / CW),
// CW = 32 or 64 channel lanes (gc <= CW), walks tokens t0 + j + NJ i with
// U tokens' loads issued together: gx[t,c] += sum_h dz[t,h] W[h,c] for its
// tokens (no conflicts), and a per-block partial of
// gW[h,c] = sum_t dz[t,h] x[t,c], reduced over j in LDS in j order.  The
// gate factors dz[t,h] = ggate g (1 - g/2) of kGateTok tokens at a time are
// staged in LDS by one coalesced pass, so a token step waits for one round
// of loads (x and gx together), not one per head.
constexpr int kGateTok = 256;
template <int CW, typename TG>
__global__ __launch_bounds__(256) void ve_gate_bwd_partial_k(TG* __restrict__ gx, float* __restrict__ partial,
                                                             const float* __restrict__ ggate,
                                                             const float* __restrict__ gate,
                                                             const float* __restrict__ xn,
                                                             const float* __restrict__ w, int64_t nt, int64_t nkv,
                                                             int64_t gc, int64_t C, int64_t ldx) {
    constexpr int NJ = 256 / CW, U = 8;
    __shared__ float acc_s[NJ][kGateMaxH][CW];
    __shared__ float dz_s[kGateTok * kGateMaxH];
    const int c = threadIdx.x % CW, j = threadIdx.x / CW;
    const int64_t per = (nt + gridDim.x - 1) / gridDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * per;
    const int64_t t1 = t0 + per < nt ? t0 + per : nt;
    float accw[kGateMaxH], wv[kGateMaxH];
#pragma unroll
    for (int h = 0; h < kGateMaxH; ++h) {
        accw[h] = 0.f;
        wv[h] = (h < nkv && c < gc) ? w[h * gc + c] : 0.f;
    }
    for (int64_t base = t0; base < t1; base += kGateTok) {
        const int64_t end = base + kGateTok < t1 ? base + kGateTok : t1;
        __syncthreads();  // the previous tokens' factors are no longer read
        for (int64_t i = threadIdx.x; i < (end - base) * nkv; i += 256) {
            const float g = gate[base * nkv + i];
            dz_s[i] = ggate[base * nkv + i] * g * (1.0f - g / 2.0f);
        }
        __syncthreads();
        if (c >= gc) continue;
        for (int64_t t = base + j; t < end; t += U * NJ) {
            float x[U], gv[U], ax[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t tt = t + u * NJ;
                const bool ok = tt < end;
                x[u] = ok ? xn[tt * ldx + c] : 0.f;
                gv[u] = ok ? (float)gx[tt * C + c] : 0.f;
                ax[u] = 0.f;
            }
#pragma unroll
            for (int h = 0; h < kGateMaxH; ++h) {
                if (h >= nkv) break;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int64_t tt = t + u * NJ;
                    if (tt >= end) break;
                    const float dz = dz_s[(tt - base) * nkv + h];
                    ax[u] += dz * wv[h];
                    accw[h] += dz * x[u];
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t tt = t + u * NJ;
                if (tt < end) gx[tt * C + c] = (TG)(gv[u] + ax[u]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < kGateMaxH; ++h) acc_s[j][h][c] = accw[h];
    __syncthreads();
    if (j == 0 && c < gc) {
        for (int64_t h = 0; h < nkv; ++h) {
            float s = acc_s[0][h][c];
#pragma unroll
            for (int jj = 1; jj < NJ; ++jj) s += acc_s[jj][h][c];
            partial[(int64_t)blockIdx.x * nkv * gc + h * gc + c] = s;
        }
    }
}

// Partials summed in block order; 16 loads issued ahead of their adds.
__global__ void ve_gate_bwd_finish_k(float* gw, const float* partial, int nblocks, int64_t n) {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        float s = 0.f;
        int b = 0;
        for (; b + 16 <= nblocks; b += 16) {
            float x[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) x[u] = partial[(int64_t)(b + u) * n + i];
#pragma unroll
            for (int u = 0; u < 16; ++u) s += x[u];
        }
        for (; b < nblocks; ++b) s += partial[(int64_t)b * n + i];
        gw[i] += s;
    }
}

// ---------------- K24 embedding_bwd: deterministic sorted scatter ----------------
// Tokens are stably sorted by id.  The sorted list is cut into chunks: a chunk
// starts at every position p with p % kEmbChunk == 0 or id[p] != id[p-1].
// A chunk's rows are summed in token order (starting from its first row);
// then each id's row is G[v] = ((G[v] + chunk_0) + chunk_1) + ... in order.
constexpr int kEmbChunk = 64;

// Stable LSD counting sort of the token ids (pairs id -> token position).
// Each pass sorts by one digit of at most kSortMaxBits bits:
//   sort_hist_k     per tile of kSortTile positions, the count of each digit
//                   (LDS integer atomics: the counts do not depend on order),
//                   stored digit-major: hist[d * ntiles + tile];
//   sort_scan_k     one workgroup turns hist into exclusive offsets in that
//                   order (all of digit 0 over the tiles in order, then digit
//                   1, ...), i.e. the first output slot of (digit, tile);
//   sort_scatter_k  one wave per tile walks its positions in order, 64 at a
//                   time: the lanes holding the same digit are found with one
//                   ballot per digit bit, ranked by lane, and placed after the
//                   (digit, tile) offset advanced by the earlier rounds.
// Tiles, rounds and lanes are visited in position order, so equal digits keep
// their input order (stable), and the result is the same on every run.
constexpr int kSortTile = 2048;
constexpr int kSortMaxBits = 11;

__global__ __launch_bounds__(256) void sort_hist_k(int32_t* hist, const int64_t* ids, const uint32_t* keys, int64_t n,
                                                    int shift, int bits, int64_t ntiles) {
    __shared__ int32_t cnt[1 << kSortMaxBits];
    const int bins = 1 << bits;
    for (int d = threadIdx.x; d < bins; d += 256) cnt[d] = 0;
    __syncthreads();
    const int64_t t0 = (int64_t)blockIdx.x * kSortTile;
    for (int i = threadIdx.x; i < kSortTile; i += 256) {
        const int64_t p = t0 + i;
        if (p < n) {
            const uint32_t k = ids ? (uint32_t)ids[p] : keys[p];
            atomicAdd(&cnt[(k >> shift) & (uint32_t)(bins - 1)], 1);
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < bins; d += 256) hist[(int64_t)d * ntiles + blockIdx.x] = cnt[d];
}

// Exclusive scan of total int32 values in place by one 1024-thread
// workgroup: thread t owns a contiguous run, the runs' sums are scanned in
// LDS, then each run is rewritten from its offset.
__global__ __launch_bounds__(1024) void sort_scan_k(int32_t* v, int64_t total) {
    __shared__ int32_t part[1024];
    const int t = threadIdx.x;
    const int64_t per = (total + 1023) / 1024;
    const int64_t a = (int64_t)t * per, b = a + per < total ? a + per : total;
    int32_t s = 0;
    for (int64_t i = a; i < b; ++i) s += v[i];
    part[t] = s;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // inclusive Hillis-Steele scan of the run sums
        const int32_t x = t >= o ? part[t - o] : 0;
        __syncthreads();
        part[t] += x;
        __syncthreads();
    }
    int32_t run = part[t] - s;
    for (int64_t i = a; i < b; ++i) {
        const int32_t c = v[i];
        v[i] = run;
        run += c;
    }
}

__global__ __launch_bounds__(64) void sort_scatter_k(uint32_t* keys_out, int32_t* vals_out, const int64_t* ids,
                                                     const uint32_t* keys_in, const int32_t* vals_in,
                                                     const int32_t* hist, int64_t n, int shift, int bits,
                                                     int64_t ntiles) {
    __shared__ int32_t base[1 << kSortMaxBits];
    const int lane = threadIdx.x;
    const int bins = 1 << bits;
    for (int d = lane; d < bins; d += 64) base[d] = hist[(int64_t)d * ntiles + blockIdx.x];
    __syncthreads();
    const int64_t t0 = (int64_t)blockIdx.x * kSortTile;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    for (int r = 0; r < kSortTile && t0 + r < n; r += 64) {  // wave-uniform bounds
        const int64_t p = t0 + r + lane;
        const bool valid = p < n;
        uint32_t k = 0;
        int32_t v = 0;
        if (valid) {
            k = ids ? (uint32_t)ids[p] : keys_in[p];
            v = ids ? (int32_t)p : vals_in[p];
        }
        const uint32_t d = (k >> shift) & (uint32_t)(bins - 1);
        uint64_t peers = __ballot(valid);
        for (int bit = 0; bit < bits; ++bit) {
            const bool on = (d >> bit) & 1u;
            const uint64_t bal = __ballot(on);
            peers &= on ? bal : ~bal;
        }
        // peers: the valid lanes holding digit d (this lane included when valid)
        const int leader = valid ? __ffsll((unsigned long long)peers) - 1 : lane;
        int32_t b0 = (valid && lane == leader) ? base[d] : 0;
        b0 = __shfl(b0, leader, 64);
        if (valid) {
            const int32_t pos = b0 + __popcll(peers & below);
            keys_out[pos] = k;
            vals_out[pos] = v;
            if (lane == leader) base[d] = b0 + __popcll(peers);
        }
        __syncthreads();  // the next round's leaders read the advanced offsets
    }
}

__device__ __forceinline__ bool emb_chunk_start(const uint32_t* k, int64_t p) {
    return p == 0 || (p % kEmbChunk) == 0 || k[p] != k[p - 1];
}

// First index in [lo, hi) whose key exceeds v (keys sorted ascending).
__device__ __forceinline__ int64_t emb_upper(const uint32_t* k, int64_t lo, int64_t hi, uint32_t v) {
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (k[mid] <= v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// The same for a whole wave (every lane calls it with the same arguments and
// gets the same result): 64 probes per step, each step narrowing the range to
// one probe interval, i.e. ceil(log64(hi - lo)) dependent loads instead of
// log2(hi - lo).  Invariant: the answer lies in [lo, hi], keys[lo - 1] <= v.
__device__ __forceinline__ int64_t emb_upper_wave(const uint32_t* k, int64_t lo, int64_t hi, uint32_t v, int lane) {
    while (lo < hi) {
        const int64_t step = (hi - lo + kWave - 1) / kWave;
        const int64_t q = lo + (int64_t)lane * step;
        const bool past = q >= hi || k[q] > v;
        const uint64_t m = __builtin_amdgcn_ballot_w64(past);
        const int f = m ? __builtin_ctzll(m) : kWave;  // first probe past the run of v
        if (f == 0) return lo;
        const int64_t a = lo + (int64_t)(f - 1) * step + 1;  // probe f - 1 is inside the run
        const int64_t b = lo + (int64_t)f * step;
        lo = a;
        hi = b < hi ? b : hi;
    }
    return lo;
}

// Chunk sums, one workgroup per 64-position window of the sorted ids (every
// chunk lies inside one window): the window's rows are walked in order, 8
// rows' loads issued ahead, and each chunk's sum (started from its first row,
// then += the next rows in token order) is written to partial[chunk start].
// Threads own float2 columns t + 256 j (dim % 2 == 0).
constexpr int kUnroll = 8;
// The window walk's loads are branch-free (clamped row and column, the
// clamped values never added or stored) so that kWinAhead rows' gathers are
// in flight together; a bound-checked load in a branch makes the compiler
// wait for each one before issuing the next.
constexpr int kWinAhead = 8;

template <int NJ>
__global__ __launch_bounds__(256) void emb_chunk_sum_win_k(float* partial, const uint32_t* keys, const int32_t* tok,
                                                           const float* dy, int64_t n, int64_t dim) {
    __shared__ uint32_t s_key[kEmbChunk];
    __shared__ int32_t s_tok[kEmbChunk];
    const int64_t w0 = (int64_t)blockIdx.x * kEmbChunk;
    const int len = (int)(n - w0 < kEmbChunk ? n - w0 : kEmbChunk);
    if (threadIdx.x < len) {
        s_key[threadIdx.x] = keys[w0 + threadIdx.x];
        s_tok[threadIdx.x] = tok[w0 + threadIdx.x];
    }
    __syncthreads();
    const int64_t d2 = dim / 2;
    float2 acc[NJ];
    int start = 0;
    int64_t cj[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) cj[j] = threadIdx.x + 256 * j < d2 ? threadIdx.x + 256 * j : 0;
    for (int r0 = 0; r0 < len; r0 += kWinAhead) {
        float2 x[kWinAhead][NJ];
#pragma unroll
        for (int u = 0; u < kWinAhead; ++u) {
            const int r = r0 + u < len ? r0 + u : len - 1;
            const float2* row = reinterpret_cast<const float2*>(dy + (int64_t)s_tok[r] * dim);
#pragma unroll
            for (int j = 0; j < NJ; ++j) x[u][j] = row[cj[j]];
        }
#pragma unroll
        for (int u = 0; u < kWinAhead; ++u) {
            const int r = r0 + u;
            if (r >= len) break;
            if (r == 0 || s_key[r] != s_key[r - 1]) {
                if (r > 0) {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int64_t c = threadIdx.x + 256 * j;
                        if (c < d2) reinterpret_cast<float2*>(partial + (w0 + start) * dim)[c] = acc[j];
                    }
                }
                start = r;
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[j] = x[u][j];
            } else {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    acc[j].x += x[u][j].x;
                    acc[j].y += x[u][j].y;
                }
            }
        }
    }
    if (len > 0) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int64_t c = threadIdx.x + 256 * j;
            if (c < d2) reinterpret_cast<float2*>(partial + (w0 + start) * dim)[c] = acc[j];
        }
    }
}

__global__ void emb_chunk_sum_k(float* partial, const uint32_t* keys, const int32_t* tok, const float* dy, int64_t n,
                                int64_t dim) {
    const int lane = threadIdx.x % kWave;
    const int64_t p = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (p >= n || !emb_chunk_start(keys, p)) return;
    int64_t q = (p / kEmbChunk + 1) * kEmbChunk;
    if (q > n) q = n;
    q = emb_upper(keys, p, q, keys[p]);
    for (int64_t d = lane; d < dim; d += kWave) {
        float s = dy[(int64_t)tok[p] * dim + d];
        for (int64_t r = p + 1; r < q; ++r) s += dy[(int64_t)tok[r] * dim + d];
        partial[p * dim + d] = s;
    }
}

// One wave per id segment: G[v] = ((G[v] + chunk_0) + chunk_1) + ..., where
// chunk_0 starts at the segment start p and chunk_j (j >= 1) at the j-th
// multiple of kEmbChunk after it.  Lane l owns the float4 columns l + 64 j
// (j < NC); the chunk rows' loads are issued kUnroll at a time ahead of their
// in-order adds (8 x NC float4 registers: the 256-thread bound keeps NC = 4
// out of scratch).
template <int NC>
__global__ __launch_bounds__(256) void emb_segment_apply_v_k(float* gw, const float* partial, const uint32_t* keys, int64_t n, int64_t dim) {
    const int lane = threadIdx.x % kWave;
    const int64_t p = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (p >= n || !(p == 0 || keys[p] != keys[p - 1])) return;
    const uint32_t v = keys[p];
    const int64_t end = emb_upper_wave(keys, p + 1, n, v, lane);
    const int64_t d4 = dim / 4;
    float4* row = reinterpret_cast<float4*>(gw + (int64_t)v * dim);
    float4 acc[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = lane + 64 * j < d4 ? row[lane + 64 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
    // chunk starts: p, then (p / kEmbChunk + j) * kEmbChunk for j >= 1, below end
    const int64_t nch = 1 + (end - 1) / kEmbChunk - p / kEmbChunk;
    for (int64_t c0 = 0; c0 < nch; c0 += kUnroll) {
        float4 x[kUnroll][NC];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t ci = c0 + u;
            const bool ok = ci < nch;
            const int64_t c = !ok ? p : (ci == 0 ? p : (p / kEmbChunk + ci) * kEmbChunk);
            const float4* src = reinterpret_cast<const float4*>(partial + c * dim);
#pragma unroll
            for (int j = 0; j < NC; ++j)
                x[u][j] = ok && lane + 64 * j < d4 ? src[lane + 64 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (c0 + u >= nch) break;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                acc[j].x += x[u][j].x; acc[j].y += x[u][j].y; acc[j].z += x[u][j].z; acc[j].w += x[u][j].w;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j)
        if (lane + 64 * j < d4) row[lane + 64 * j] = acc[j];
}

__global__ void emb_segment_apply_k(float* gw, const float* partial, const uint32_t* keys, int64_t n, int64_t dim) {
    const int lane = threadIdx.x % kWave;
    const int64_t p = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (p >= n || !(p == 0 || keys[p] != keys[p - 1])) return;
    const uint32_t v = keys[p];
    const int64_t end = emb_upper(keys, p + 1, n, v);
    float* row = gw + (int64_t)v * dim;
    for (int64_t d = lane; d < dim; d += kWave) {
        float acc = row[d];
        for (int64_t c = p; c < end; c = (c / kEmbChunk + 1) * kEmbChunk) acc += partial[c * dim + d];
        row[d] = acc;
    }
}

}  // namespace

// =====================================================================
// C ABI
// =====================================================================

static unsigned wave_grid(int64_t rows) { return flat_grid(rows, kBlock / kWave); }

extern "C" int32_t ar_rmsnorm_fwd(ar_stream_t stream, float* output, float* rms_out, const float* input,
                                  int64_t num_rows, int64_t dim) {
    AR_CHECK_ARG(output && input, "rmsnorm_fwd: null pointer");
    AR_CHECK_ARG(num_rows >= 0 && dim > 0, "rmsnorm_fwd: bad shape");
    if (num_rows == 0) return AR_OK;
    if (dim % 4 == 0 && al16(output) && al16(input))
        rmsnorm_fwd_k<true><<<wave_grid(num_rows), kBlock, 0, S(stream)>>>(output, rms_out, input, num_rows, dim);
    else
        rmsnorm_fwd_k<false><<<wave_grid(num_rows), kBlock, 0, S(stream)>>>(output, rms_out, input, num_rows, dim);
    return AR_LAUNCH_CHECK("rmsnorm_fwd");
}

extern "C" int32_t ar_rmsnorm_bwd(ar_stream_t stream, float* grad_input, const float* grad_output,
                                  const float* input, const float* rms_saved, int64_t num_rows, int64_t dim) {
    AR_CHECK_ARG(grad_input && grad_output && input && rms_saved, "rmsnorm_bwd: null pointer");
    AR_CHECK_ARG(num_rows >= 0 && dim > 0, "rmsnorm_bwd: bad shape");
    if (num_rows == 0) return AR_OK;
    if (dim % 4 == 0 && al16(grad_input) && al16(grad_output) && al16(input))
        rmsnorm_bwd_k<true><<<wave_grid(num_rows), kBlock, 0, S(stream)>>>(grad_input, grad_output, input,
                                                                         rms_saved, num_rows, dim);
    else
        rmsnorm_bwd_k<false><<<wave_grid(num_rows), kBlock, 0, S(stream)>>>(grad_input, grad_output, input,
                                                                          rms_saved, num_rows, dim);
    return AR_LAUNCH_CHECK("rmsnorm_bwd");
}

extern "C" int32_t ar_cross_entropy_fwd(ar_stream_t stream, float* loss_out, const float* logits,
                                        const int64_t* targets, int64_t num_tokens, int64_t vocab_size) {
    AR_CHECK_ARG(loss_out && logits && targets, "cross_entropy_fwd: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && vocab_size > 0, "cross_entropy_fwd: bad shape");
    if (num_tokens == 0) return AR_OK;
    ce_fwd_k<<<(unsigned)num_tokens, kBlock, 0, S(stream)>>>(loss_out, logits, targets, vocab_size);
    return AR_LAUNCH_CHECK("cross_entropy_fwd");
}

extern "C" int32_t ar_cross_entropy_softcap_bwd(ar_stream_t stream, float* grad_logits, const float* logits,
                                                const int64_t* targets, float cap, int64_t num_tokens,
                                                int64_t vocab_size, float loss_scale) {
    (void)cap;  // the softcap derivative is not applied (ops.mojo:854-858)
    AR_CHECK_ARG(grad_logits && logits && targets, "cross_entropy_softcap_bwd: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && vocab_size > 0, "cross_entropy_softcap_bwd: bad shape");
    if (num_tokens == 0) return AR_OK;
    ce_bwd_k<<<(unsigned)num_tokens, kBlock, 0, S(stream)>>>(grad_logits, logits, targets, vocab_size, loss_scale);
    return AR_LAUNCH_CHECK("cross_entropy_softcap_bwd");
}

extern "C" int32_t ar_softmax_fwd(ar_stream_t stream, float* output, const float* input, int64_t num_rows,
                                  int64_t cols) {
    AR_CHECK_ARG(output && input, "softmax_fwd: null pointer");
    AR_CHECK_ARG(num_rows >= 0 && cols > 0, "softmax_fwd: bad shape");
    if (num_rows == 0) return AR_OK;
    softmax_k<<<(unsigned)num_rows, kBlock, 0, S(stream)>>>(output, input, cols);
    return AR_LAUNCH_CHECK("softmax_fwd");
}

namespace ar {
int32_t fixed_sum(hipStream_t st, float* out, const float* a, const float* b, int64_t n, int mode_in, int mode_out,
                  int64_t idx, float* partial) {
    dot_partial_k<<<kSumBlocks, kBlock, 0, st>>>(partial, a, b, n, mode_in);
    finish_sum_k<<<1, 1024, 0, st>>>(out, partial, kSumBlocks, idx, n, mode_out);
    return check_launch("fixed_sum");
}

int32_t frob_normalize(hipStream_t st, float* data, int64_t n, float* scratch) {
    if (n == 0) return AR_OK;
    float* scale = scratch + kSumBlocks;
    dot_partial_k<<<kSumBlocks, kBlock, 0, st>>>(scratch, data, nullptr, n, 1);
    finish_sum_k<<<1, 1024, 0, st>>>(scale, scratch, kSumBlocks, 0, n, 2);
    scale_by_device_scalar_k<<<flat_grid(n, kBlock * 4), kBlock, 0, st>>>(data, scale, n);
    return check_launch("normalize_frobenius");
}

template <typename TG>
static int32_t ve_gate_bwd_t(hipStream_t st, TG* gx, float* gw, const float* ggate, const float* gate,
                             const float* xn, const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C,
                             int64_t ldx, float* partial) {
    if (nt == 0) return AR_OK;
    if (gc <= 32)
        ve_gate_bwd_partial_k<32, TG>
            <<<kGateBlocks, 256, 0, st>>>(gx, partial, ggate, gate, xn, w, nt, nkv, gc, C, ldx);
    else
        ve_gate_bwd_partial_k<64, TG>
            <<<kGateBlocks, 256, 0, st>>>(gx, partial, ggate, gate, xn, w, nt, nkv, gc, C, ldx);
    ve_gate_bwd_finish_k<<<1, 256, 0, st>>>(gw, partial, kGateBlocks, nkv * gc);
    return check_launch("ve_gate_bwd");
}
int32_t ve_gate_bwd(hipStream_t st, float* gx, float* gw, const float* ggate, const float* gate, const float* xn,
                    const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C, int64_t ldx, float* partial) {
    return ve_gate_bwd_t(st, gx, gw, ggate, gate, xn, w, nt, nkv, gc, C, ldx, partial);
}
int32_t ve_gate_bwd(hipStream_t st, bf16* gx, float* gw, const float* ggate, const float* gate, const float* xn,
                    const float* w, int64_t nt, int64_t nkv, int64_t gc, int64_t C, int64_t ldx, float* partial) {
    return ve_gate_bwd_t(st, gx, gw, ggate, gate, xn, w, nt, nkv, gc, C, ldx, partial);
}
}  // namespace ar

static int32_t ws_sum(ar_stream_t stream, float* out, const float* a, const float* b, int64_t n, int mi, int mo,
                      int64_t idx) {
    int32_t st;
    float* partial = (float*)workspace(S(stream), kSumBlocks * sizeof(float), &st);
    if (!partial) return st;
    return ar::fixed_sum(S(stream), out, a, b, n, mi, mo, idx, partial);
}

extern "C" int32_t ar_mean_reduce(ar_stream_t stream, float* output, const float* input, int64_t size) {
    AR_CHECK_ARG(output && input && size > 0, "mean_reduce: bad argument");
    return ws_sum(stream, output, input, nullptr, size, 0, 0, 0);
}

extern "C" int32_t ar_scalar_grad_reduce(ar_stream_t stream, float* grad_scalar, const float* grad_output,
                                         const float* input, int64_t idx, int64_t size) {
    AR_CHECK_ARG(grad_scalar && grad_output && input && size >= 0 && idx >= 0, "scalar_grad_reduce: bad argument");
    return ws_sum(stream, grad_scalar, grad_output, input, size, 2, 1, idx);
}

extern "C" int32_t ar_normalize_frobenius(ar_stream_t stream, float* data, int64_t size) {
    AR_CHECK_ARG(data && size >= 0, "normalize_frobenius: bad argument");
    if (size == 0) return AR_OK;
    int32_t st;
    float* ws = (float*)workspace(S(stream), (kSumBlocks + 64) * sizeof(float), &st);
    if (!ws) return st;
    return ar::frob_normalize(S(stream), data, size, ws);
}

static int32_t precompute_d(ar_stream_t stream, float* d_out, const float* output, const float* grad_output,
                            int64_t B, int64_t T, int64_t num_heads, int64_t head_dim, bool round_do) {
    AR_CHECK_ARG(d_out && output && grad_output, "flash_attn_bwd_precompute_d: null pointer");
    AR_CHECK_ARG(B >= 0 && T >= 0 && num_heads > 0 && head_dim > 0, "flash_attn_bwd_precompute_d: bad shape");
    const int64_t rows = B * T * num_heads;
    if (rows == 0) return AR_OK;
    if (round_do)
        precompute_d_k<true><<<wave_grid(rows), kBlock, 0, S(stream)>>>(d_out, output, grad_output, rows, head_dim);
    else
        precompute_d_k<false><<<wave_grid(rows), kBlock, 0, S(stream)>>>(d_out, output, grad_output, rows, head_dim);
    return AR_LAUNCH_CHECK("flash_attn_bwd_precompute_d");
}

extern "C" int32_t ar_flash_attn_bwd_precompute_d(ar_stream_t stream, float* d_out, const float* output,
                                                  const float* grad_output, int64_t B, int64_t T,
                                                  int64_t num_heads, int64_t head_dim) {
    return precompute_d(stream, d_out, output, grad_output, B, T, num_heads, head_dim, false);
}

extern "C" int32_t ar_flash_attn_bwd_precompute_d_bf16(ar_stream_t stream, float* d_out, const float* output,
                                                       const float* grad_output, int64_t B, int64_t T,
                                                       int64_t num_heads, int64_t head_dim) {
    return precompute_d(stream, d_out, output, grad_output, B, T, num_heads, head_dim, true);
}

extern "C" int32_t ar_ve_gate_fwd(ar_stream_t stream, float* gate_out, const float* x_norm, const float* gate_weight,
                                  int64_t num_tokens, int64_t n_kv_head, int64_t gate_channels, int64_t embd_dim) {
    AR_CHECK_ARG(gate_out && x_norm && gate_weight, "ve_gate_fwd: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && n_kv_head > 0 && gate_channels > 0 && gate_channels <= embd_dim,
                 "ve_gate_fwd: bad shape");
    if (num_tokens == 0) return AR_OK;
    ve_gate_fwd_k<<<flat_grid(num_tokens * n_kv_head, kBlock), kBlock, 0, S(stream)>>>(
        gate_out, x_norm, gate_weight, num_tokens, n_kv_head, gate_channels, embd_dim);
    return AR_LAUNCH_CHECK("ve_gate_fwd");
}

extern "C" int32_t ar_ve_apply_bwd(ar_stream_t stream, float* grad_ve, float* grad_gate, const float* grad_v,
                                   const float* gate, const float* ve, int64_t num_tokens, int64_t n_kv_head,
                                   int64_t head_dim) {
    AR_CHECK_ARG(grad_ve && grad_gate && grad_v && gate && ve, "ve_apply_bwd: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && n_kv_head > 0 && head_dim > 0, "ve_apply_bwd: bad shape");
    const int64_t rows = num_tokens * n_kv_head;
    if (rows == 0) return AR_OK;
    ve_apply_bwd_k<<<wave_grid(rows), kBlock, 0, S(stream)>>>(grad_ve, grad_gate, grad_v, gate, ve, rows, head_dim);
    return AR_LAUNCH_CHECK("ve_apply_bwd");
}

extern "C" int32_t ar_ve_gate_bwd(ar_stream_t stream, float* grad_x_norm_out, float* grad_gate_weight,
                                  const float* grad_gate, const float* gate, const float* x_norm,
                                  const float* gate_weight, int64_t num_tokens, int64_t n_kv_head,
                                  int64_t gate_channels, int64_t embd_dim) {
    AR_CHECK_ARG(grad_x_norm_out && grad_gate_weight && grad_gate && gate && x_norm && gate_weight,
                 "ve_gate_bwd: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && n_kv_head > 0 && n_kv_head <= kGateMaxH && gate_channels > 0 &&
                     gate_channels <= 64 && gate_channels <= embd_dim,
                 "ve_gate_bwd: unsupported shape (n_kv_head <= 16, gate_channels <= 64)");
    if (num_tokens == 0) return AR_OK;
    int32_t st;
    const int64_t n = n_kv_head * gate_channels;
    float* partial = (float*)workspace(S(stream), (size_t)kGateBlocks * n * sizeof(float), &st);
    if (!partial) return st;
    return ar::ve_gate_bwd(S(stream), grad_x_norm_out, grad_gate_weight, grad_gate, gate, x_norm, gate_weight,
                           num_tokens, n_kv_head, gate_channels, embd_dim, embd_dim, partial);
}

// Sort workspace layout: keys, keys_sorted, vals, vals_sorted (n each), flag,
// cub temp, then partial sums [n, dim].
extern "C" int32_t ar_embedding_bwd_sorted(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                           const uint32_t* sorted_ids, const int32_t* sorted_tokens,
                                           int64_t num_tokens, int64_t embd_dim, float* partial) {
    const int64_t n = num_tokens;
    if (n <= 0 || embd_dim <= 0) return AR_OK;
    const unsigned grid = (unsigned)cdiv(n, kBlock / kWave);
    const int64_t nc = cdiv(embd_dim, 256), nj = cdiv(embd_dim, 512);
    if (embd_dim % 4 == 0 && al16(grad_output) && al16(partial) && al16(grad_weight) && nc <= 4) {
        const unsigned wins = (unsigned)cdiv(n, kEmbChunk);
        if (nj <= 1) emb_chunk_sum_win_k<1><<<wins, 256, 0, S(stream)>>>(partial, sorted_ids, sorted_tokens, grad_output, n, embd_dim);
        else emb_chunk_sum_win_k<2><<<wins, 256, 0, S(stream)>>>(partial, sorted_ids, sorted_tokens, grad_output, n, embd_dim);
        if (nc <= 1) emb_segment_apply_v_k<1><<<grid, kBlock, 0, S(stream)>>>(grad_weight, partial, sorted_ids, n, embd_dim);
        else if (nc <= 2) emb_segment_apply_v_k<2><<<grid, kBlock, 0, S(stream)>>>(grad_weight, partial, sorted_ids, n, embd_dim);
        else emb_segment_apply_v_k<4><<<grid, kBlock, 0, S(stream)>>>(grad_weight, partial, sorted_ids, n, embd_dim);
    } else {
        emb_chunk_sum_k<<<grid, kBlock, 0, S(stream)>>>(partial, sorted_ids, sorted_tokens, grad_output, n, embd_dim);
        emb_segment_apply_k<<<grid, kBlock, 0, S(stream)>>>(grad_weight, partial, sorted_ids, n, embd_dim);
    }
    return AR_LAUNCH_CHECK("embedding_bwd");
}

// Stable sort of token ids: sorted_ids/sorted_tokens (n each), ids taken
// as their low end_bit bits (32 when the vocabulary size is unknown).  The
// passes ping-pong between the outputs and a scratch pair, ordered so that
// the last pass writes the outputs.
static void sort_plan(int32_t end_bit, int& npass, int& bits) {
    if (end_bit < 1) end_bit = 1;
    npass = (end_bit + kSortMaxBits - 1) / kSortMaxBits;
    bits = (end_bit + npass - 1) / npass;
}

extern "C" int32_t ar_embedding_sort(ar_stream_t stream, uint32_t* sorted_ids, int32_t* sorted_tokens,
                                     const int64_t* indices, int64_t num_tokens, int32_t end_bit, void* scratch,
                                     size_t scratch_bytes, size_t* scratch_needed) {
    const int64_t n = num_tokens;
    AR_CHECK_ARG(n >= 0 && n < ((int64_t)1 << 31) && end_bit >= 1 && end_bit <= 32, "embedding_sort: bad arguments");
    int npass, bits;
    sort_plan(end_bit, npass, bits);
    const int64_t ntiles = cdiv(n, kSortTile) > 0 ? cdiv(n, kSortTile) : 1;
    const size_t keys_bytes = ((size_t)n * 4 + 255) & ~size_t(255);
    const size_t hist_bytes = ((size_t)(1 << bits) * ntiles * 4 + 255) & ~size_t(255);
    const size_t need = 2 * keys_bytes + hist_bytes;
    if (scratch_needed) *scratch_needed = need;
    if (!scratch) return AR_OK;
    if (scratch_bytes < need) return set_error(AR_EINVAL, "embedding_sort: scratch too small");
    AR_CHECK_ARG(sorted_ids && sorted_tokens && indices, "embedding_sort: null pointer");
    if (n == 0) return AR_OK;
    char* base = (char*)scratch;
    uint32_t* tk = (uint32_t*)base;
    int32_t* tv = (int32_t*)(base + keys_bytes);
    int32_t* hist = (int32_t*)(base + 2 * keys_bytes);
    const hipStream_t st = S(stream);
    const uint32_t* kin = nullptr;
    const int32_t* vin = nullptr;
    for (int p = 0; p < npass; ++p) {
        const int shift = p * bits;
        const int pb = end_bit - shift < bits ? end_bit - shift : bits;
        const bool to_out = ((npass - 1 - p) % 2) == 0;
        uint32_t* kout = to_out ? sorted_ids : tk;
        int32_t* vout = to_out ? sorted_tokens : tv;
        const int64_t* ids = p == 0 ? indices : nullptr;
        sort_hist_k<<<(unsigned)ntiles, 256, 0, st>>>(hist, ids, kin, n, shift, pb, ntiles);
        sort_scan_k<<<1, 1024, 0, st>>>(hist, (int64_t)(1 << pb) * ntiles);
        sort_scatter_k<<<(unsigned)ntiles, 64, 0, st>>>(kout, vout, ids, kin, vin, hist, n, shift, pb, ntiles);
        kin = kout;
        vin = vout;
    }
    return AR_LAUNCH_CHECK("embedding_sort");
}

extern "C" int32_t ar_embedding_bwd(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                    const int64_t* indices, int64_t num_tokens, int64_t embd_dim) {
    AR_CHECK_ARG(grad_weight && grad_output && indices, "embedding_bwd: null pointer");
    AR_CHECK_ARG(num_tokens >= 0 && num_tokens < (int64_t)1 << 31 && embd_dim > 0, "embedding_bwd: bad shape");
    if (num_tokens == 0) return AR_OK;
    size_t sort_bytes = 0;
    int32_t st = ar_embedding_sort(stream, nullptr, nullptr, indices, num_tokens, 32, nullptr, 0, &sort_bytes);
    if (st) return st;
    const size_t ids_bytes = ((size_t)num_tokens * 4 + 255) & ~size_t(255);
    const size_t part_bytes = (size_t)num_tokens * embd_dim * sizeof(float);
    char* ws = (char*)workspace(S(stream), 2 * ids_bytes + sort_bytes + part_bytes, &st);
    if (!ws) return st;
    uint32_t* sids = (uint32_t*)ws;
    int32_t* stok = (int32_t*)(ws + ids_bytes);
    char* sort_scratch = ws + 2 * ids_bytes;
    float* partial = (float*)(sort_scratch + sort_bytes);
    st = ar_embedding_sort(stream, sids, stok, indices, num_tokens, 32, sort_scratch, sort_bytes, nullptr);
    if (st) return st;
    return ar_embedding_bwd_sorted(stream, grad_weight, grad_output, sids, stok, num_tokens, embd_dim, partial);
}
