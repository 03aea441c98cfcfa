// ar_attention.hip -- flash attention forward and backward on the gfx950
// matrix cores, for the reference's flash_attn_fwd (ops.mojo:244-323),
// flash_attn_bwd_dq (ops.mojo:349-411) and flash_attn_bwd_dkv
// (ops.mojo:414-480).
//
// Layout: q, k, v, O, dO are [B, T, H, hd] (token-major, heads interleaved:
// row stride H*hd), LSE and D are [B, T, H].  Key kp is visible from query qp
// iff kp <= qp and (window <= 0 or kp >= qp - window).
//
// Work decomposition (all three kernels): a workgroup of 4 wave64s owns 128
// rows of one (b, h) -- queries for fwd / dQ, keys for dK/dV -- 32 per wave,
// and streams 64-row tiles of the other side through LDS, skipping tiles that
// the causal / sliding-window mask removes entirely.
//
// MFMA mapping.  Products are formed transposed so the 32 rows a wave owns
// are the MFMA *columns*: e.g. the forward computes S^T = K Q^T, where lane l
// holds query l%32 and 16 keys.  Softmax statistics are then per-lane values
// (two lanes, l and l^32, share a query).  The P (or dS) tile is fed straight
// back as the B operand of the next product (O^T += V^T P^T) without leaving
// registers: the MFMA accumulator layout hands each lane a permuted subset of
// keys, and the A operand (V^T, K^T, dO^T, Q^T) is read from LDS in that same
// permuted key order.  bf16 compute (v_mfma_f32_32x32x16_bf16) reads the
// permuted operand from a transposed [d][row] LDS copy; fp32 compute
// (v_mfma_f32_32x32x2_f32) reads it straight from the [row][d] tile.
//
// dK/dV are accumulated by key-block ownership and dQ by query-block
// ownership (two kernels, no atomics: deterministic).  Softmax runs in the
// exp2 domain with the 1/sqrt(hd) scale and log2(e) folded into one multiply.
#include "ar_internal.hpp"

using namespace ar;

namespace {

constexpr int kThreads = 256;
constexpr int kOwn = 128;  // rows owned by a workgroup (4 waves x 32)
constexpr int kTile = 64;  // rows per streamed LDS tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ int acc_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

// 2^x with the hardware's v_exp_f32 (1 ulp): results below 2^-126
// (probabilities that change no fp32 sum they enter) flush to zero, and
// 2^-inf = 0.  The library exp2f spends several instructions and registers per
// element on denormal results.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

template <bool BF16> struct AT;

template <> struct AT<true> {
    using LT = bf16;
    using Frag = bf16x8;
    static constexpr int KS = 16, CW = 8, PADN = 8, LDT = kTile + 8, STEPS32 = 2;
    static constexpr bool TRANS = true;
    __device__ static f32x16 mma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    // Operand fragment of a row stored d-contiguous: k-step ks.
    __device__ static Frag rowfrag(const LT* row, int ks, int lane) {
        return *reinterpret_cast<const bf16x8*>(row + ks * KS + (lane >> 5) * 8);
    }
    // A operand in permuted row order for k-step s of 32-row block kb:
    // rows {32kb + 16s + 4g + 0..3, 32kb + 16s + 8 + 4g + 0..3}, g = lane/32.
    // `tr` is the transposed LDS tile, [d][row] with row stride LDT.
    __device__ static Frag permfrag(const LT* natural, int ldn, const LT* tr, int d, int kb, int s, int lane) {
        (void)natural;
        (void)ldn;
        const int g = lane >> 5;
        const LT* p = tr + d * LDT + kb * 32 + 16 * s + 4 * g;
        bf16x4 lo = *reinterpret_cast<const bf16x4*>(p);
        bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + 8);
        Frag f;
        f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
        f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
        return f;
    }
    // B operand from the lane's own accumulator values, k-step s.
    __device__ static Frag accfrag(const f32x16& a, int s) {
        Frag f;
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (bf16)a[8 * s + e];
        return f;
    }
    // The bf16 rounding residual of accfrag: accfrag + accfrag_lo carries
    // ~16 significant bits of the fp32 value.
    __device__ static Frag accfrag_lo(const f32x16& a, int s) {
        Frag f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = a[8 * s + e];
            f[e] = (bf16)(x - (float)(bf16)x);
        }
        return f;
    }
};

template <> struct AT<false> {
    using LT = float;
    using Frag = float;
    static constexpr int KS = 2, CW = 4, PADN = 4, LDT = 4, STEPS32 = 16;
    static constexpr bool TRANS = false;
    __device__ static f32x16 mma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __device__ static Frag rowfrag(const LT* row, int ks, int lane) { return row[ks * KS + (lane >> 5)]; }
    // row {32kb + 8(s/4) + 4g + s%4}, read from the natural [row][d] tile.
    __device__ static Frag permfrag(const LT* natural, int ldn, const LT* tr, int d, int kb, int s, int lane) {
        (void)tr;
        const int r = kb * 32 + (s >> 2) * 8 + (lane >> 5) * 4 + (s & 3);
        return natural[r * ldn + d];
    }
    __device__ static Frag accfrag(const f32x16& a, int s) { return a[s]; }
    __device__ static Frag accfrag_lo(const f32x16& a, int s) { (void)a; (void)s; return 0.0f; }
};

// One 64-row tile of a [T, rs]-strided operand (columns [0, HD)) on its way to
// LDS (natural [row][HD + PADN] layout), in two halves so that its global
// loads can be issued before the MFMAs of the previous tile and written to LDS
// after them: TileVals holds this thread's items of the tile (4 rows x 4
// columns each).  Rows at or beyond T load row T - 1 and are zeroed by a
// select, so no load sits in a branch.
template <bool BF16, int HD, typename TIN>
struct TileVals {
    using A = AT<BF16>;
    using LT = typename A::LT;
    static constexpr int CW = A::CW, ITEMS = (kTile / 4) * (HD / CW), NIT = (ITEMS + kThreads - 1) / kThreads;
    static_assert(!BF16 && sizeof(TIN) == 4, "fp32 operands, fp32 compute");
    static_assert(ITEMS % kWave == 0, "whole waves per item pass");
    LT v[NIT][4][CW];
    __device__ __forceinline__ void load(const TIN* base, int64_t rs, int row0, int T) {
#pragma unroll
        for (int n = 0; n < NIT; ++n) {
            const int it = n * kThreads + threadIdx.x;
            if (ITEMS % kThreads != 0 && it >= ITEMS) break;  // whole waves (ITEMS is a multiple of 64)
            const int r4 = it % (kTile / 4), dc = (it / (kTile / 4)) * CW;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + r4 * 4 + i;
                const TIN* src = base + (int64_t)(row < T ? row : T - 1) * rs + dc;
#pragma unroll
                for (int j = 0; j < CW; j += 4) *reinterpret_cast<float4*>(&v[n][i][j]) =
                    *reinterpret_cast<const float4*>(src + j);
            }
        }
    }
    __device__ __forceinline__ void write(LT* nat, int row0, int T) const {
        constexpr int LDN = HD + A::PADN;
#pragma unroll
        for (int n = 0; n < NIT; ++n) {
            const int it = n * kThreads + threadIdx.x;
            if (ITEMS % kThreads != 0 && it >= ITEMS) break;
            const int r4 = it % (kTile / 4), dc = (it / (kTile / 4)) * CW;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool in = row0 + r4 * 4 + i < T;
                float4 x = *reinterpret_cast<const float4*>(&v[n][i][0]);
                if (!in) x = make_float4(0.f, 0.f, 0.f, 0.f);
                *reinterpret_cast<float4*>(nat + (r4 * 4 + i) * LDN + dc) = x;
            }
        }
    }
};

// Load the 32 rows [r0, r0+32) of an operand as B fragments (lane row r0 + l%32).
template <bool BF16, int HD, typename TIN>
__device__ __forceinline__ void load_bfrags(typename AT<BF16>::Frag (&f)[HD / AT<BF16>::KS], const TIN* base,
                                            int64_t rs, int row, int T, int lane) {
    using A = AT<BF16>;
#pragma unroll
    for (int ks = 0; ks < HD / A::KS; ++ks) {
        if constexpr (BF16) {
            typename A::Frag fr;
            if (row < T) {
                const TIN* src = base + (int64_t)row * rs + ks * A::KS + (lane >> 5) * 8;
                if constexpr (sizeof(TIN) == 4) {
                    float4 a = *reinterpret_cast<const float4*>(src);
                    float4 b = *reinterpret_cast<const float4*>(src + 4);
                    fr[0] = (bf16)a.x; fr[1] = (bf16)a.y; fr[2] = (bf16)a.z; fr[3] = (bf16)a.w;
                    fr[4] = (bf16)b.x; fr[5] = (bf16)b.y; fr[6] = (bf16)b.z; fr[7] = (bf16)b.w;
                } else {
                    fr = *reinterpret_cast<const bf16x8*>(src);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) fr[e] = (bf16)0.0f;
            }
            f[ks] = fr;
        } else {
            f[ks] = row < T ? (float)base[(int64_t)row * rs + ks * A::KS + (lane >> 5)] : 0.0f;
        }
    }
}

// Write a wave's transposed accumulator tiles (rows d, columns = the wave's 32
// rows) as [row][d] output rows, scaled, through a wave-private LDS scratch.
template <int HD, typename TOUT>
__device__ __forceinline__ void store_rows_T(TOUT* out, int64_t rs, int row_base, int T, const f32x16 (&acc)[HD / 32],
                                             float scale, float* scratch, int lane) {
    // scratch: 32 x 36 floats per wave
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
#pragma unroll
        for (int v = 0; v < 16; ++v) scratch[(lane & 31) * 36 + acc_row(v, lane)] = acc[dt][v] * scale;
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int r = pass * 8 + lane / 8, c4 = (lane % 8) * 4;
            const int row = row_base + r;
            if (row < T) {
                float4 x = *reinterpret_cast<const float4*>(scratch + r * 36 + c4);
                TOUT* dst = out + (int64_t)row * rs + dt * 32 + c4;
                if constexpr (sizeof(TOUT) == 4) {
                    *reinterpret_cast<float4*>(dst) = x;
                } else {
                    dst[0] = (TOUT)x.x; dst[1] = (TOUT)x.y; dst[2] = (TOUT)x.z; dst[3] = (TOUT)x.w;
                }
            }
        }
        __syncthreads();
    }
}

template <bool BF16, int HD>
constexpr int lds_tile_elems() {
    using A = AT<BF16>;
    return kTile * (HD + A::PADN) + (A::TRANS ? HD * A::LDT : 0);
}

// ============================ forward ============================
// Occupancy: two workgroups per CU (<= 256 registers; the tiles take 67.6 KB
// of LDS at hd 128).  Unbounded, the compiler took 264 registers at hd 128 and
// the kernel ran one wave per SIMD, with every tile load exposed.  The
// backward kernels get the same bound up to hd 64; at hd 128 their own-row
// fragments alone (2 x 64 registers) leave no room for it without spills.
template <bool BF16, int HD, typename TIN>
__global__ __launch_bounds__(kThreads, 2) void fa_fwd_k(float* out, float* lse, const TIN* q, const TIN* k, const TIN* v,
                                                     int B, int T, int H, int window, float scale_log2) {
    using A = AT<BF16>;
    using LT = typename A::LT;
    constexpr int LDN = HD + A::PADN;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LT* sK = reinterpret_cast<LT*>(smem_raw);
    LT* sV = sK + kTile * LDN;                                  // natural V (fp32 path)
    LT* sVT = sK + kTile * LDN;                                 // transposed V (bf16 path)
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int q0 = blockIdx.x * kOwn, qw = q0 + wave * 32, my_q = qw + (lane & 31);
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;

    typename A::Frag qf[HD / A::KS];
    load_bfrags<BF16, HD>(qf, q + boff, rs, my_q, T, lane);

    f32x16 o[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    float m = -INFINITY, l = 0.f;

    int kstart = 0;
    if (window > 0) kstart = q0 - window > 0 ? q0 - window : 0;
    kstart = (kstart / kTile) * kTile;
    const int kend = (q0 + kOwn < T) ? q0 + kOwn : T;
    // the next tile's K / V rows are loaded into registers while this tile's
    // MFMAs run, and written to LDS after the barrier that ends them
    TileVals<BF16, HD, TIN> nk, nv;
    if (kstart < kend) {
        nk.load(k + boff, rs, kstart, T);
        nv.load(v + boff, rs, kstart, T);
    }
    for (int kv0 = kstart; kv0 < kend; kv0 += kTile) {
        nk.write(sK, kv0, T);
        nv.write(sV, kv0, T);
        __syncthreads();
        if (kv0 + kTile < kend) {
            nk.load(k + boff, rs, kv0 + kTile, T);
            nv.load(v + boff, rs, kv0 + kTile, T);
        }
        const bool skip = kv0 > qw + 31 || (window > 0 && kv0 + kTile - 1 < qw - window) || qw >= T;
        if (!skip) {
            f32x16 s[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
                const LT* krow = sK + (kb * 32 + (lane & 31)) * LDN;
#pragma unroll
                for (int ks = 0; ks < HD / A::KS; ++ks) s[kb] = A::mma(A::rowfrag(krow, ks, lane), qf[ks], s[kb]);
            }
            float mt = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = kv0 + kb * 32 + acc_row(e, lane);
                    const bool ok = key <= my_q && key < T && (window <= 0 || key >= my_q - window);
                    const float x = ok ? s[kb][e] * scale_log2 : -INFINITY;
                    s[kb][e] = x;
                    mt = fmaxf(mt, x);
                }
            mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
            const float m_new = fmaxf(m, mt);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = exp2_hw(m - m_use);
            float rsum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = exp2_hw(s[kb][e] - m_use);
                    s[kb][e] = p;
                    rsum += p;
                }
            rsum += __shfl_xor(rsum, 32, kWave);
            l = l * alpha + rsum;
            m = m_new;
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
            // O^T += V^T P^T.  With bf16 operands P goes in as a two-term bf16
            // split (hi + lo), so O keeps fp32-level accuracy in P: the
            // backward's D = rowsum(dO * O) must equal sum_j P_j dP_j, and a
            // bf16-rounded P would bias every dS_j = P_j (dP_j - D) by the same
            // amount, which the attention-weighted mean key then multiplies.
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int st = 0; st < A::STEPS32; ++st) {
                    const typename A::Frag pb = A::accfrag(s[kb], st);
                    typename A::Frag pl{};
                    if constexpr (BF16) pl = A::accfrag_lo(s[kb], st);
#pragma unroll
                    for (int dt = 0; dt < HD / 32; ++dt) {
                        const int d = dt * 32 + (lane & 31);
                        const typename A::Frag va = A::permfrag(sV, LDN, sVT, d, kb, st, lane);
                        o[dt] = A::mma(va, pb, o[dt]);
                        if constexpr (BF16) o[dt] = A::mma(va, pl, o[dt]);
                    }
                }
        }
        __syncthreads();
    }
    const float inv_l = l > 0.f ? 1.0f / l : 0.f;
    if (lane < 32 && my_q < T)
        lse[((int64_t)b * T + my_q) * H + h] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 36;
    // Output scale is per query (per lane); fold it before staging.
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= inv_l;
    store_rows_T<HD>(out + boff, rs, qw, T, o, 1.0f, scratch, lane);
}

// ============================ backward: dQ ============================
// The next K / V tile is prefetched into registers as in the forward; at hd 128
// that takes ~380 registers, one wave per SIMD (fp32 step: dQ 21.55 -> 21.33 ms
// against the 256-register form that loaded each tile when it started).
template <bool BF16, int HD, typename TIN>
__global__ __launch_bounds__(kThreads, HD <= 64 ? 2 : 1) void fa_bwd_dq_k(float* dq, const TIN* q, const TIN* k, const TIN* v,
                                                        const TIN* dout, const float* lse, const float* dbuf, int B,
                                                        int T, int H, int window, float scale_log2, float scale) {
    using A = AT<BF16>;
    using LT = typename A::LT;
    constexpr int LDN = HD + A::PADN;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LT* sK = reinterpret_cast<LT*>(smem_raw);
    LT* sKT = sK + kTile * LDN;
    LT* sV = sKT + (A::TRANS ? HD * A::LDT : 0);
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int q0 = blockIdx.x * kOwn, qw = q0 + wave * 32, my_q = qw + (lane & 31);
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;

    typename A::Frag qf[HD / A::KS], df[HD / A::KS];
    load_bfrags<BF16, HD>(qf, q + boff, rs, my_q, T, lane);
    load_bfrags<BF16, HD>(df, dout + boff, rs, my_q, T, lane);
    const int64_t bth = ((int64_t)b * T + (my_q < T ? my_q : 0)) * H + h;
    const float my_lse2 = lse[bth] * kLog2e;
    const float my_D = dbuf[bth];

    f32x16 acc[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;

    int kstart = 0;
    if (window > 0) kstart = q0 - window > 0 ? q0 - window : 0;
    kstart = (kstart / kTile) * kTile;
    const int kend = (q0 + kOwn < T) ? q0 + kOwn : T;
    // the next tile's K / V rows are loaded into registers while this tile's
    // MFMAs run, and written to LDS after the barrier that ends them
    TileVals<BF16, HD, TIN> nk, nv;
    if (kstart < kend) {
        nk.load(k + boff, rs, kstart, T);
        nv.load(v + boff, rs, kstart, T);
    }
    for (int kv0 = kstart; kv0 < kend; kv0 += kTile) {
        nk.write(sK, kv0, T);
        nv.write(sV, kv0, T);
        __syncthreads();
        if (kv0 + kTile < kend) {
            nk.load(k + boff, rs, kv0 + kTile, T);
            nv.load(v + boff, rs, kv0 + kTile, T);
        }
        const bool skip = kv0 > qw + 31 || (window > 0 && kv0 + kTile - 1 < qw - window) || qw >= T;
        if (!skip) {
            // one 32-key half at a time (not unrolled): only one S / dP pair is
            // live beside the own-row Q and dO fragments, the dQ accumulators
            // and the prefetched tile
#pragma unroll 1
            for (int kb = 0; kb < 2; ++kb) {
                f32x16 s, dp;
#pragma unroll
                for (int e = 0; e < 16; ++e) s[e] = dp[e] = 0.f;
                const LT* krow = sK + (kb * 32 + (lane & 31)) * LDN;
                const LT* vrow = sV + (kb * 32 + (lane & 31)) * LDN;
#pragma unroll
                for (int ks = 0; ks < HD / A::KS; ++ks) {
                    s = A::mma(A::rowfrag(krow, ks, lane), qf[ks], s);
                    dp = A::mma(A::rowfrag(vrow, ks, lane), df[ks], dp);
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = kv0 + kb * 32 + acc_row(e, lane);
                    const bool ok = key <= my_q && key < T && my_q < T && (window <= 0 || key >= my_q - window);
                    const float p = ok ? exp2_hw(s[e] * scale_log2 - my_lse2) : 0.f;
                    s[e] = p * (dp[e] - my_D);
                }
#pragma unroll
                for (int st = 0; st < A::STEPS32; ++st) {
                    const typename A::Frag db = A::accfrag(s, st);
#pragma unroll
                    for (int dt = 0; dt < HD / 32; ++dt) {
                        const int d = dt * 32 + (lane & 31);
                        acc[dt] = A::mma(A::permfrag(sK, LDN, sKT, d, kb, st, lane), db, acc[dt]);
                    }
                }
            }
        }
        __syncthreads();
    }
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 36;
    store_rows_T<HD>(dq + boff, rs, qw, T, acc, scale, scratch, lane);
}

// ============================ backward: dK, dV ============================
// dK and dV in one pass from one S / P / dS per tile.  At hd 128 the own K and
// V fragments, both accumulator sets (4 x 64 registers) and the next tile's
// Q / dO rows take ~440 registers, so that launch runs one wave per SIMD (one
// workgroup per CU).  That measured faster than a dV launch and a dK launch of
// 256 registers each, which recomputed S twice and left the dK launch no room
// for the prefetch: fp32 step, dK + dV 37.4 -> 28.6 ms.
template <bool BF16, int HD, typename TIN>
__global__ __launch_bounds__(kThreads, HD <= 64 ? 2 : 1) void fa_bwd_dkv_k(float* dk, float* dv, const TIN* q, const TIN* k,
                                                         const TIN* v, const TIN* dout, const float* lse,
                                                         const float* dbuf, int B, int T, int H, int window,
                                                         float scale_log2, float scale) {
    using A = AT<BF16>;
    using LT = typename A::LT;
    constexpr int LDN = HD + A::PADN;
    constexpr int TE = lds_tile_elems<BF16, HD>();
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LT* sQ = reinterpret_cast<LT*>(smem_raw);
    LT* sQT = sQ + kTile * LDN;
    LT* sD = sQ + TE;
    LT* sDT = sD + kTile * LDN;
    float* sL = reinterpret_cast<float*>(sQ + 2 * TE);
    float* sDl = sL + kTile;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int k0 = blockIdx.x * kOwn, kw = k0 + wave * 32, my_k = kw + (lane & 31);
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;

    typename A::Frag kf[HD / A::KS], vf[HD / A::KS];
    load_bfrags<BF16, HD>(kf, k + boff, rs, my_k, T, lane);
    load_bfrags<BF16, HD>(vf, v + boff, rs, my_k, T, lane);

    f32x16 dka[HD / 32], dva[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) dka[dt][e] = dva[dt][e] = 0.f;

    const int qstart = (k0 / kTile) * kTile;
    int qend = T;
    if (window > 0 && k0 + kOwn - 1 + window + 1 < T) qend = k0 + kOwn - 1 + window + 1;
    // The next Q / dO tile and its LSE / D values are loaded into registers
    // while this tile's MFMAs run, and written to LDS after the barrier.
    TileVals<BF16, HD, TIN> nq, nd;
    float nl = 0.f, ndl = 0.f;
    auto ld_load = [&](int qt0) {  // LSE / D of query qt0 + tid (row 0 past T: masked)
        if (threadIdx.x < kTile) {
            const int qq = qt0 + threadIdx.x;
            const int64_t bth = ((int64_t)b * T + (qq < T ? qq : 0)) * H + h;
            nl = lse[bth];
            ndl = dbuf[bth];
        }
    };
    if (qstart < qend) {
        nq.load(q + boff, rs, qstart, T);
        nd.load(dout + boff, rs, qstart, T);
        ld_load(qstart);
    }
    for (int qt0 = qstart; qt0 < qend; qt0 += kTile) {
        nq.write(sQ, qt0, T);
        nd.write(sD, qt0, T);
        if (threadIdx.x < kTile) {
            sL[threadIdx.x] = nl * kLog2e;
            sDl[threadIdx.x] = ndl;
        }
        __syncthreads();
        if (qt0 + kTile < qend) {
            nq.load(q + boff, rs, qt0 + kTile, T);
            nd.load(dout + boff, rs, qt0 + kTile, T);
            ld_load(qt0 + kTile);
        }
        const bool skip = qt0 + kTile - 1 < kw || (window > 0 && qt0 > kw + 31 + window) || kw >= T;
        if (!skip) {
            // the two 32-query halves one after the other (not unrolled: at
            // hd 128 two halves in flight would spill)
#pragma unroll 1
            for (int qb = 0; qb < 2; ++qb) {
                f32x16 s, dp;
#pragma unroll
                for (int e = 0; e < 16; ++e) s[e] = dp[e] = 0.f;
                const LT* qrow = sQ + (qb * 32 + (lane & 31)) * LDN;
                const LT* drow = sD + (qb * 32 + (lane & 31)) * LDN;
#pragma unroll
                for (int ks = 0; ks < HD / A::KS; ++ks) {
                    s = A::mma(A::rowfrag(qrow, ks, lane), kf[ks], s);
                    dp = A::mma(A::rowfrag(drow, ks, lane), vf[ks], dp);
                }
                // s, dp: lane holds key my_k, queries qt0 + 32qb + acc_row(e)
                f32x16 p, ds;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int qr = qb * 32 + acc_row(e, lane);
                    const int qq = qt0 + qr;
                    const bool ok = my_k <= qq && qq < T && my_k < T && (window <= 0 || my_k >= qq - window);
                    const float pv = ok ? exp2_hw(s[e] * scale_log2 - sL[qr]) : 0.f;
                    p[e] = pv;
                    ds[e] = pv * (dp[e] - sDl[qr]);
                }
#pragma unroll
                for (int st = 0; st < A::STEPS32; ++st) {
                    const typename A::Frag pb = A::accfrag(p, st);
                    const typename A::Frag db = A::accfrag(ds, st);
#pragma unroll
                    for (int dt = 0; dt < HD / 32; ++dt) {
                        const int d = dt * 32 + (lane & 31);
                        dva[dt] = A::mma(A::permfrag(sD, LDN, sDT, d, qb, st, lane), pb, dva[dt]);
                        dka[dt] = A::mma(A::permfrag(sQ, LDN, sQT, d, qb, st, lane), db, dka[dt]);
                    }
                }
            }
        }
        __syncthreads();
    }
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 36;
    store_rows_T<HD>(dk + boff, rs, kw, T, dka, scale, scratch, lane);
    store_rows_T<HD>(dv + boff, rs, kw, T, dva, 1.0f, scratch, lane);
}

template <bool BF16, int HD>
size_t fwd_lds() {
    using A = AT<BF16>;
    size_t tiles = (size_t)(kTile * (HD + A::PADN) + (A::TRANS ? HD * A::LDT : kTile * (HD + A::PADN))) *
                   sizeof(typename A::LT);
    size_t stage = 4 * 32 * 36 * sizeof(float);
    return tiles > stage ? tiles : stage;
}
template <bool BF16, int HD>
size_t dq_lds() {
    using A = AT<BF16>;
    size_t tiles = (size_t)(2 * kTile * (HD + A::PADN) + (A::TRANS ? HD * A::LDT : 0)) * sizeof(typename A::LT);
    size_t stage = 4 * 32 * 36 * sizeof(float);
    return tiles > stage ? tiles : stage;
}
template <bool BF16, int HD>
size_t dkv_lds() {
    size_t tiles = (size_t)2 * lds_tile_elems<BF16, HD>() * sizeof(typename AT<BF16>::LT) + 2 * kTile * sizeof(float);
    size_t stage = 4 * 32 * 36 * sizeof(float);
    return tiles > stage ? tiles : stage;
}

}  // namespace

namespace ar {

template <bool BF16, int HD, typename TIN>
static int32_t attn_dispatch_hd(hipStream_t st, AttnOp op, float* o1, float* o2, const TIN* q, const TIN* k,
                                const TIN* v, const TIN* dout, const float* lse, const float* dbuf, int B, int T, int H,
                                int window, float sc) {
    const float scale = sc > 0.f ? sc : 1.0f / sqrtf((float)HD);
    const float scale_log2 = scale * kLog2e;
    dim3 grid((unsigned)((T + kOwn - 1) / kOwn), (unsigned)(B * H));
    if (op == AttnOp::FWD) {
        const size_t lds = fwd_lds<BF16, HD>();
        fa_fwd_k<BF16, HD, TIN><<<grid, kThreads, lds, st>>>(o1, o2, q, k, v, B, T, H, window, scale_log2);
        return check_launch("flash_attn_fwd");
    }
    if (op == AttnOp::DQ) {
        const size_t lds = dq_lds<BF16, HD>();
        fa_bwd_dq_k<BF16, HD, TIN><<<grid, kThreads, lds, st>>>(o1, q, k, v, dout, lse, dbuf, B, T, H, window,
                                                                scale_log2, scale);
        return check_launch("flash_attn_bwd_dq");
    }
    const size_t lds = dkv_lds<BF16, HD>();
    fa_bwd_dkv_k<BF16, HD, TIN><<<grid, kThreads, lds, st>>>(o1, o2, q, k, v, dout, lse, dbuf, B, T, H, window,
                                                             scale_log2, scale);
    return check_launch("flash_attn_bwd_dkv");
}

template <bool BF16, typename TIN>
int32_t attn_dispatch(hipStream_t st, AttnOp op, float* o1, float* o2, const TIN* q, const TIN* k, const TIN* v,
                      const TIN* dout, const float* lse, const float* dbuf, int64_t B, int64_t T, int64_t H,
                      int64_t HD, int64_t window, float scale) {
    if (HD > 128) return set_error(AR_EUNSUPPORTED, "flash attention: head_dim %lld > 128", (long long)HD);
    if (B <= 0 || T <= 0 || H <= 0) return B == 0 || T == 0 ? AR_OK : set_error(AR_EINVAL, "flash attention: bad shape");
    if (B * H > 65535 || T > (1 << 30)) return set_error(AR_EINVAL, "flash attention: shape too large");
    const int w = window > (int64_t)T ? (int)T : (int)window;  // a window >= T is full causal
    switch (HD) {
        case 32: return attn_dispatch_hd<BF16, 32, TIN>(st, op, o1, o2, q, k, v, dout, lse, dbuf, (int)B, (int)T, (int)H, w, scale);
        case 64: return attn_dispatch_hd<BF16, 64, TIN>(st, op, o1, o2, q, k, v, dout, lse, dbuf, (int)B, (int)T, (int)H, w, scale);
        case 128: return attn_dispatch_hd<BF16, 128, TIN>(st, op, o1, o2, q, k, v, dout, lse, dbuf, (int)B, (int)T, (int)H, w, scale);
        default: return set_error(AR_EUNSUPPORTED, "flash attention: head_dim %lld not in {32, 64, 128}", (long long)HD);
    }
}

}  // namespace ar

static __host__ __device__ inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

#define AR_ATTN_PTRS(...)                                                                   \
    do {                                                                                    \
        const void* ps[] = {__VA_ARGS__};                                                   \
        for (const void* p : ps)                                                            \
            if (!p || !al16(p)) return ar::set_error(AR_EINVAL, "%s: null or unaligned pointer", __func__); \
    } while (0)

// ---- any head_dim <= 128 (ops.mojo:267 accepts every head_dim up to 128) ----
// The tiled kernels exist for head_dim 32, 64 and 128.  Another head_dim runs
// them at the next of those sizes on copies of q, k, v (and dO) whose rows are
// zero past head_dim, with the softmax scale of the real head_dim: the zero
// columns add nothing to any score or to D, and the output columns past
// head_dim (O, dQ, dK, dV) are exact zeros that the copy back drops.
namespace {

bool native_hd(int64_t hd) { return hd == 32 || hd == 64 || hd == 128; }
int64_t padded_hd(int64_t hd) { return hd <= 32 ? 32 : (hd <= 64 ? 64 : 128); }
size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

template <typename TO>
__global__ void pad_rows_k(TO* dst, const float* src, int64_t rows, int hd, int hdp) {
    const int64_t n = rows * hdp;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / hdp;
        const int d = (int)(i - r * hdp);
        dst[i] = (TO)(d < hd ? src[r * hd + d] : 0.0f);
    }
}
__global__ void unpad_rows_k(float* dst, const float* src, int64_t rows, int hd, int hdp) {
    const int64_t n = rows * hd;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / hd;
        dst[i] = src[r * hdp + (i - r * hd)];
    }
}

// One attention op at a head_dim outside {32, 64, 128}: fp32 operands (bf = false)
// or bf16-rounded copies (bf = true).  in = {q, k, v[, dO]}.
int32_t attn_padded(ar_stream_t stream, bool bf, ar::AttnOp op, float* o1, float* o2, const float* const* in,
                    const float* lse, const float* dbuf, int64_t B, int64_t T, int64_t H, int64_t hd,
                    int64_t window) {
    if (hd <= 0 || B < 0 || T < 0 || H < 0)
        return ar::set_error(AR_EINVAL, "flash attention: bad shape (B %lld, T %lld, H %lld, head_dim %lld)",
                             (long long)B, (long long)T, (long long)H, (long long)hd);
    if (hd > 128)
        return ar::set_error(AR_EUNSUPPORTED, "flash attention: head_dim %lld not in [1, 128]", (long long)hd);
    if (B == 0 || T == 0 || H == 0) return AR_OK;
    const int64_t hdp = padded_hd(hd), rows = B * T * H, n = rows * hdp;
    const int nin = op == ar::AttnOp::FWD ? 3 : 4;
    const int nout = op == ar::AttnOp::DKV ? 2 : 1;
    const size_t in_b = align256((size_t)n * (bf ? sizeof(ar::bf16) : sizeof(float)));
    const size_t out_b = align256((size_t)n * sizeof(float));
    int32_t st;
    char* w = (char*)ar::workspace(ar::S(stream), nin * in_b + nout * out_b, &st);
    if (!w) return st;
    const unsigned g = ar::flat_grid(n, 256);
    void* pin[4] = {nullptr, nullptr, nullptr, nullptr};
    for (int i = 0; i < nin; ++i) {
        pin[i] = w + i * in_b;
        if (bf) pad_rows_k<ar::bf16><<<g, 256, 0, ar::S(stream)>>>((ar::bf16*)pin[i], in[i], rows, (int)hd, (int)hdp);
        else pad_rows_k<float><<<g, 256, 0, ar::S(stream)>>>((float*)pin[i], in[i], rows, (int)hd, (int)hdp);
    }
    int32_t r = ar::check_launch("flash attention: pad head_dim");
    if (r) return r;
    float* p1 = (float*)(w + nin * in_b);
    float* p2 = op == ar::AttnOp::DKV ? (float*)(w + nin * in_b + out_b) : o2;  // FWD: o2 = LSE, unpadded
    const float scale = 1.0f / sqrtf((float)hd);
    if (bf)
        r = ar::flash_attn_bf16(ar::S(stream), op, p1, p2, ar::FlashOut{}, (const ar::bf16*)pin[0],
                                (const ar::bf16*)pin[1], (const ar::bf16*)pin[2], (const ar::bf16*)pin[3], lse, dbuf,
                                B, T, H, hdp, window, scale);
    else
        r = ar::attn_dispatch<false, float>(ar::S(stream), op, p1, p2, (const float*)pin[0], (const float*)pin[1],
                                            (const float*)pin[2], (const float*)pin[3], lse, dbuf, B, T, H, hdp,
                                            window, scale);
    if (r) return r;
    const unsigned go = ar::flat_grid(rows * hd, 256);
    unpad_rows_k<<<go, 256, 0, ar::S(stream)>>>(o1, p1, rows, (int)hd, (int)hdp);
    if (op == ar::AttnOp::DKV) unpad_rows_k<<<go, 256, 0, ar::S(stream)>>>(o2, p2, rows, (int)hd, (int)hdp);
    return ar::check_launch("flash attention: unpad head_dim");
}

// bf16 compute at head_dim 32 / 64 / 128: operands rounded to bf16 once (into
// the library workspace), then the bf16-operand kernels of ar_flash.hip.
int32_t to_bf16_ws(ar_stream_t stream, const float* const* src, int n, int64_t elems, ar::bf16** dst) {
    int32_t st;
    const size_t each = align256((size_t)elems * sizeof(ar::bf16));
    char* w = (char*)ar::workspace(S(stream), (size_t)n * each, &st);
    if (!w) return st;
    for (int i = 0; i < n; ++i) {
        dst[i] = (ar::bf16*)(w + i * each);
        const int32_t r = ar::to_bf16(S(stream), dst[i], src[i], elems);
        if (r) return r;
    }
    return AR_OK;
}
}  // namespace

extern "C" int32_t ar_flash_attn_fwd(ar_stream_t stream, float* output, float* lse_out, const float* q, const float* k,
                                     const float* v, int64_t B, int64_t T, int64_t num_heads, int64_t head_dim,
                                     int64_t window_size) {
    AR_ATTN_PTRS(output, q, k, v);
    AR_CHECK_ARG(lse_out != nullptr, "flash_attn_fwd: null lse");
    if (!native_hd(head_dim)) {
        const float* in[3] = {q, k, v};
        return attn_padded(stream, false, ar::AttnOp::FWD, output, lse_out, in, nullptr, nullptr, B, T, num_heads,
                           head_dim, window_size);
    }
    return ar::attn_dispatch<false, float>(S(stream), ar::AttnOp::FWD, output, lse_out, q, k, v, nullptr, nullptr,
                                           nullptr, B, T, num_heads, head_dim, window_size);
}

extern "C" int32_t ar_flash_attn_fwd_bf16(ar_stream_t stream, float* output, float* lse_out, const float* q,
                                          const float* k, const float* v, int64_t B, int64_t T, int64_t num_heads,
                                          int64_t head_dim, int64_t window_size) {
    AR_ATTN_PTRS(output, q, k, v);
    AR_CHECK_ARG(lse_out != nullptr, "flash_attn_fwd_bf16: null lse");
    AR_CHECK_ARG(B >= 0 && T >= 0 && num_heads >= 0, "flash_attn_fwd_bf16: bad shape");
    if (native_hd(head_dim) && (B == 0 || T == 0 || num_heads == 0)) return AR_OK;  // nothing to do
    const float* src[3] = {q, k, v};
    if (!native_hd(head_dim))
        return attn_padded(stream, true, ar::AttnOp::FWD, output, lse_out, src, nullptr, nullptr, B, T, num_heads,
                           head_dim, window_size);
    ar::bf16* b[3];
    int32_t r = to_bf16_ws(stream, src, 3, B * T * num_heads * head_dim, b);
    if (r) return r;
    return ar::flash_attn_bf16(S(stream), ar::AttnOp::FWD, output, lse_out, ar::FlashOut{}, b[0], b[1], b[2], nullptr,
                               nullptr, nullptr, B, T, num_heads, head_dim, window_size);
}
extern "C" int32_t ar_flash_attn_bwd_dq(ar_stream_t stream, float* grad_q, const float* q, const float* k,
                                        const float* v, const float* grad_output, const float* lse, const float* d_buf,
                                        int64_t B, int64_t T, int64_t num_heads, int64_t head_dim,
                                        int64_t window_size) {
    AR_ATTN_PTRS(grad_q, q, k, v, grad_output);
    AR_CHECK_ARG(lse && d_buf, "flash_attn_bwd_dq: null lse / d_buf");
    if (!native_hd(head_dim)) {
        const float* in[4] = {q, k, v, grad_output};
        return attn_padded(stream, false, ar::AttnOp::DQ, grad_q, nullptr, in, lse, d_buf, B, T, num_heads, head_dim,
                           window_size);
    }
    return ar::attn_dispatch<false, float>(S(stream), ar::AttnOp::DQ, grad_q, nullptr, q, k, v, grad_output, lse,
                                           d_buf, B, T, num_heads, head_dim, window_size);
}
extern "C" int32_t ar_flash_attn_bwd_dq_bf16(ar_stream_t stream, float* grad_q, const float* q, const float* k,
                                             const float* v, const float* grad_output, const float* lse,
                                             const float* d_buf, int64_t B, int64_t T, int64_t num_heads,
                                             int64_t head_dim, int64_t window_size) {
    AR_ATTN_PTRS(grad_q, q, k, v, grad_output);
    AR_CHECK_ARG(lse && d_buf, "flash_attn_bwd_dq_bf16: null lse / d_buf");
    AR_CHECK_ARG(B >= 0 && T >= 0 && num_heads >= 0, "flash_attn_bwd_dq_bf16: bad shape");
    if (native_hd(head_dim) && (B == 0 || T == 0 || num_heads == 0)) return AR_OK;  // nothing to do
    const float* src[4] = {q, k, v, grad_output};
    if (!native_hd(head_dim))
        return attn_padded(stream, true, ar::AttnOp::DQ, grad_q, nullptr, src, lse, d_buf, B, T, num_heads, head_dim,
                           window_size);
    ar::bf16* b[4];
    int32_t r = to_bf16_ws(stream, src, 4, B * T * num_heads * head_dim, b);
    if (r) return r;
    return ar::flash_attn_bf16(S(stream), ar::AttnOp::DQ, grad_q, nullptr, ar::FlashOut{}, b[0], b[1], b[2], b[3], lse,
                               d_buf, B, T, num_heads, head_dim, window_size);
}
extern "C" int32_t ar_flash_attn_bwd_dkv(ar_stream_t stream, float* grad_k, float* grad_v, const float* q,
                                         const float* k, const float* v, const float* grad_output, const float* lse,
                                         const float* d_buf, int64_t B, int64_t T, int64_t num_heads,
                                         int64_t head_dim, int64_t window_size) {
    AR_ATTN_PTRS(grad_k, grad_v, q, k, v, grad_output);
    AR_CHECK_ARG(lse && d_buf, "flash_attn_bwd_dkv: null lse / d_buf");
    if (!native_hd(head_dim)) {
        const float* in[4] = {q, k, v, grad_output};
        return attn_padded(stream, false, ar::AttnOp::DKV, grad_k, grad_v, in, lse, d_buf, B, T, num_heads, head_dim,
                           window_size);
    }
    return ar::attn_dispatch<false, float>(S(stream), ar::AttnOp::DKV, grad_k, grad_v, q, k, v, grad_output, lse,
                                           d_buf, B, T, num_heads, head_dim, window_size);
}
extern "C" int32_t ar_flash_attn_bwd_dkv_bf16(ar_stream_t stream, float* grad_k, float* grad_v, const float* q,
                                              const float* k, const float* v, const float* grad_output,
                                              const float* lse, const float* d_buf, int64_t B, int64_t T,
                                              int64_t num_heads, int64_t head_dim, int64_t window_size) {
    AR_ATTN_PTRS(grad_k, grad_v, q, k, v, grad_output);
    AR_CHECK_ARG(lse && d_buf, "flash_attn_bwd_dkv_bf16: null lse / d_buf");
    AR_CHECK_ARG(B >= 0 && T >= 0 && num_heads >= 0, "flash_attn_bwd_dkv_bf16: bad shape");
    if (native_hd(head_dim) && (B == 0 || T == 0 || num_heads == 0)) return AR_OK;  // nothing to do
    const float* src[4] = {q, k, v, grad_output};
    if (!native_hd(head_dim))
        return attn_padded(stream, true, ar::AttnOp::DKV, grad_k, grad_v, src, lse, d_buf, B, T, num_heads, head_dim,
                           window_size);
    ar::bf16* b[4];
    int32_t r = to_bf16_ws(stream, src, 4, B * T * num_heads * head_dim, b);
    if (r) return r;
    return ar::flash_attn_bf16(S(stream), ar::AttnOp::DKV, grad_k, grad_v, ar::FlashOut{}, b[0], b[1], b[2], b[3], lse,
                               d_buf, B, T, num_heads, head_dim, window_size);
}

template int32_t ar::attn_dispatch<false, float>(hipStream_t, ar::AttnOp, float*, float*, const float*, const float*,
                                                 const float*, const float*, const float*, const float*, int64_t,
                                                 int64_t, int64_t, int64_t, int64_t, float);
