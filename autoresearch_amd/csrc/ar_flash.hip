// ar_flash.hip -- flash attention for bf16-stored operands (the bf16 step):
// forward (ops.mojo:244-323), dQ (ops.mojo:349-411) and dK/dV
// (ops.mojo:414-480), same math and work split as ar_attention.hip, with the
// data movement rebuilt around two gfx950 features:
//
//   * Natural tiles only.  Every streamed 64-row tile (K, V, Q, dO) sits in
//     LDS in its natural [row][d] layout, 16-byte chunks XOR-swizzled per row
//     (physical chunk = logical chunk ^ swz(row)).  Operands that the MFMA
//     needs with the row index contiguous (V^T for O^T += V^T P^T, K^T for
//     dQ, Q^T / dO^T for dK / dV) are read with ds_read_b64_tr_b16: inside
//     each group of 16 lanes, lane 4k+q supplies the address of row k,
//     columns 4q..4q+3, and lane i receives rows 0..3 of column i.  Two such
//     reads give a lane the 8 rows {16s + 4g + 0..3, 16s + 8 + 4g + 0..3}
//     (g = lane / 32) that the accumulator-fed B operand holds, so no
//     transposed LDS copy is ever written.
//   * swz(r) = 4 (r mod 4) + (r / 4) mod 4 (mod chunks per row) keeps both
//     access patterns spread over the banks: 16 consecutive rows read at one
//     logical chunk hit 16 different chunks (row fragments), and 4
//     consecutive rows x 4 consecutive chunks hit 16 different chunks
//     (transposed reads).
//   * Double-buffered tiles: the next tile goes from global memory straight
//     into the other LDS stage (16-byte global_load_lds, no registers) while
//     the current tile's MFMAs run; one wait + barrier per tile.
//   * Blocks of one (batch, head) run on one XCD (K / V stay in its L2), and
//     the causal work is issued heavy-first.
//
// Layout: q, k, v, dO [B, T, H, hd] bf16 (row stride H*hd); LSE, D
// [B, T, H] fp32; outputs O, dQ, dK, dV in fp32 and / or bf16 (any row
// stride: the bf16 step writes dQ | dK | dV into one [B*T, 3C] buffer, dQ and
// dK already rotated back by the inverse rope).
#include <type_traits>

#include "ar_internal.hpp"

namespace ar {
namespace {

constexpr int kThreads = 256;
constexpr int kOwn = 128;  // rows owned by a workgroup (4 waves x 32)
constexpr int kTile = 64;  // rows per streamed tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ int acc_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

template <int HD>
struct Geo {
    static constexpr int NCH = HD / 8;            // 16-byte chunks per row
    static constexpr int TILE = kTile * HD;       // bf16 elements per tile
    static constexpr int PER = TILE / 8 / kThreads;  // chunks per thread per tile
    static constexpr int KSTEPS = HD / 16;
    static constexpr int DT = HD / 32;
    __device__ static int swz(int r) { return (4 * (r & 3) + ((r >> 2) & 3)) & (NCH - 1); }
    // element offset of logical (row, chunk) + e (e < 8) in a tile
    __device__ static int off(int r, int c) { return r * HD + ((c ^ swz(r)) << 3); }
};

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row fragment: row r, k-step ks (lane holds d = 16 ks + 8 (lane / 32) .. +8).
template <int HD>
__device__ __forceinline__ bf16x8 rowfrag(const bf16* tile, int r, int ks, int lane) {
    return *reinterpret_cast<const bf16x8*>(tile + Geo<HD>::off(r, 2 * ks + (lane >> 5)));
}

// The same fragment as rowfrag(tile + 32 kb HD, lane % 32, ks, lane), from
// base = rowbase(lane): chunk 2 ks + lane / 32 of a row sits at
// ((2 ks + lane / 32) ^ swz) * 16 = (((lane / 32) ^ swz) * 16) ^ (ks * 32)
// bytes into the row (2 ks is even, and the row's 2 HD bytes are a power of
// two above every chunk offset), so each k-step's address is one XOR.
template <int HD>
__device__ __forceinline__ unsigned rowbase(int lane) {
    return 2u * (unsigned)Geo<HD>::off(lane & 31, lane >> 5);
}
template <int HD>
__device__ __forceinline__ bf16x8 rowfrag_x(const bf16* tile, unsigned base, int ks) {
    return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(tile) + (base ^ (unsigned)(ks << 5)));
}

// Transposed fragment of a natural tile for 32-row block rb, k-step s and
// column block ct: lane l gets column 32 ct + l % 32, rows
// {32 rb + 16 s + 4 g + 0..3, 32 rb + 16 s + 8 + 4 g + 0..3}, g = l / 32.
template <int HD>
__device__ __forceinline__ bf16x8 trfrag(const bf16* tile, int rb, int s, int ct, int lane) {
    const int g = lane >> 4, src = lane & 15;
    const int row = 32 * rb + 16 * s + 4 * (g >> 1) + (src >> 2);
    const int col = 32 * ct + 16 * (g & 1) + 4 * (src & 3);
    const bf16* p0 = tile + Geo<HD>::off(row, col >> 3) + (col & 7);
    const bf16* p1 = tile + Geo<HD>::off(row + 8, col >> 3) + (col & 7);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
    const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, both);
}

// trfrag's two reads from per-lane byte bases tb0 / tb1 (those of rb = s =
// ct = 0): a lane's row swizzle depends only on its row within the 16-row
// group, rb and s move the reads by whole rows, and column block ct enters the
// chunk index as 4 ct, which the swizzle's XOR carries to 64 ct bytes.
template <int HD>
__device__ __forceinline__ void trbase(int lane, unsigned& tb0, unsigned& tb1) {
    const int g = lane >> 4, src = lane & 15;
    const int row = 4 * (g >> 1) + (src >> 2);
    const int col = 16 * (g & 1) + 4 * (src & 3);
    tb0 = 2u * (unsigned)(Geo<HD>::off(row, col >> 3) + (col & 7));
    tb1 = 2u * (unsigned)(Geo<HD>::off(row + 8, col >> 3) + (col & 7));
}
template <int HD>
__device__ __forceinline__ bf16x8 trfrag_x(const bf16* tile, unsigned tb0, unsigned tb1, int rb, int s, int ct) {
    const char* t = reinterpret_cast<const char*>(tile + (32 * rb + 16 * s) * HD);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (tb0 ^ (unsigned)(64 * ct))));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (tb1 ^ (unsigned)(64 * ct))));
    const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, both);
}

// 2^x with the hardware's v_exp_f32: results below 2^-126 (probabilities
// that change no fp32 sum they enter) flush to zero, and 2^-inf = 0.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt vmcnt(0) (lgkmcnt / expcnt left open).  Issued once before a tile
// loop: the loop body then starts with no vector-memory load outstanding on
// any path, so the compiler does not make the first MFMAs of every tile wait
// for the next tile's prefetch.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The lane index, made opaque to the optimiser once per tile: the swizzled
// LDS addresses derived from it are then recomputed inside the tile loop
// (a few VALU ops) instead of being hoisted out of it, where dozens of them
// would stay live for the whole loop and push the kernel into spills.
__device__ __forceinline__ int opaque_lane(int lane) {
    asm volatile("" : "+v"(lane));
    return lane;
}

// B fragment (bf16x8) of the lane's own accumulator values, k-step s.
__device__ __forceinline__ bf16x8 accfrag(const f32x16& a, int s) {
    bf16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (bf16)a[8 * s + e];
    return f;
}

// Direct-to-LDS load of one ROWS-row tile into the swizzled natural layout
// (16-byte slot id = i * kThreads + tid holds logical chunk
// (id % NCH) ^ swz(row) of row id / NCH; a wave's 64 slots are one 1 KB
// global_load_lds).  Rows past T repeat row T - 1: callers mask every score
// of such a row to probability 0.
template <int HD, int ROWS, int NTH = kThreads>
struct TileU {  // 16-byte chunks per thread of a ROWS-row tile (NTH threads per workgroup)
    static constexpr int N = (ROWS * Geo<HD>::NCH + NTH - 1) / NTH;
};

// This thread's chunk byte offsets from a tile's first row (row stride rs
// elements), fixed for the kernel: a whole tile's DMA is then a wave-uniform
// base address plus these offsets (no per-copy address arithmetic).
template <int HD, int ROWS = kTile, int N, int NTH = kThreads>
__device__ __forceinline__ void tile_offsets(unsigned (&off)[N], int64_t rs) {
    using G = Geo<HD>;
    static_assert(N == TileU<HD, ROWS, NTH>::N, "offset count");
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int id = i * NTH + threadIdx.x;
        const int r = id / G::NCH, c = (id % G::NCH) ^ G::swz(r);
        off[i] = (unsigned)(r * (int)rs + c * 8) * 2u;
    }
}

template <int HD, int ROWS = kTile, int N, int NTH = kThreads>
__device__ __forceinline__ void dma_tile(bf16* dst, const bf16* base, int64_t rs, int row0, int T,
                                         const unsigned (&off)[N]) {
    using G = Geo<HD>;
    static_assert(N == TileU<HD, ROWS, NTH>::N, "offset count");
    constexpr int UNITS = ROWS * G::NCH;  // a multiple of 64: the guards below are wave-uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (row0 + ROWS <= T) {
        const bf16* tb = base + (int64_t)row0 * rs;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (UNITS % NTH != 0 && i * NTH + wave * kWave >= UNITS) break;
            dma16s(tb, off[i], lds_addr(dst + (i * NTH + wave * kWave) * 8));
        }
        return;
    }
    // the sequence's last, partial tile: rows clamped per chunk.  The thread
    // index is made opaque so that this rarely taken path's address math is
    // not hoisted into registers for the whole kernel.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int id = i * NTH + tid;
        if (UNITS % NTH != 0 && i * NTH + wave * kWave >= UNITS) break;
        const int r = id / G::NCH, c = (id % G::NCH) ^ G::swz(r);
        const int row = row0 + r < T ? row0 + r : T - 1;
        dma16(base + (int64_t)row * rs + c * 8, lds_addr(dst + (i * NTH + wave * kWave) * 8));
    }
}

// B fragments of 32 own rows (row = row0 + lane % 32), read from global.
template <int HD>
__device__ __forceinline__ void own_frags(bf16x8 (&f)[HD / 16], const bf16* base, int64_t rs, int row, int T,
                                          int lane) {
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
        if (row < T) {
            f[ks] = *reinterpret_cast<const bf16x8*>(base + (int64_t)row * rs + ks * 16 + (lane >> 5) * 8);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) f[ks][e] = (bf16)0.0f;
        }
    }
}

// Block -> (bh, row block): the nrb blocks of one (b, h) are contiguous in a
// per-XCD run (workgroups are dispatched round-robin over the 8 XCDs), and
// with heavy_first the block index runs from the last row block down.
__device__ __forceinline__ void block_coords(int nrb, int nbh, bool heavy_first, int& bh, int& rb) {
    const int total = nrb * nbh;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    bh = id / nrb;
    rb = id % nrb;
    if (heavy_first) rb = nrb - 1 - rb;
}

// Write a wave's transposed accumulators (rows d, columns = its 32 rows r)
// as [r][d] rows, scaled per column (colscale: one value per lane column):
// fp32 to `of` (row stride rsf) and / or bf16 to `ob` (row stride rsb), the
// bf16 copy optionally rotated by the inverse rope of its token
// (tok = tok0 + r, table row tok % period; rope_bwd, ops.mojo:1088-1123).
// Pairs (d, d + HD/2) are staged together through wave-private LDS (32 x 68
// floats per wave).
struct RowOut {
    float* of;
    bf16* ob;
    int64_t rsf, rsb;
    const float *cos_t, *sin_t;
    int64_t tok0, period;
};

// Output rows are stored with the nontemporal hint: they are not read again
// by this kernel, and streaming them past L2 keeps the K / V (or Q / dO)
// tiles that other workgroups of the same head still read resident there.
__device__ __forceinline__ void st_nt(float* p, float4 x) {
    __builtin_nontemporal_store(x.x, p);
    __builtin_nontemporal_store(x.y, p + 1);
    __builtin_nontemporal_store(x.z, p + 2);
    __builtin_nontemporal_store(x.w, p + 3);
}
__device__ __forceinline__ void st_nt(bf16* p, bf16x4 v) {
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned long long, v), reinterpret_cast<unsigned long long*>(p));
}

template <int HD>
__device__ __forceinline__ void store_rows(const RowOut& o, int row_base, int T, const f32x16 (&acc)[HD / 32],
                                           float colscale, float* scratch, int lane) {
    constexpr int DT = HD / 32, HALF = HD / 2;
    constexpr int NPAIR = DT >= 2 ? DT / 2 : 1;  // staged (block, block + DT/2) pairs
    constexpr int PW = DT >= 2 ? 32 : 16;        // pair columns per staged block
    constexpr int LDS_ = 68;
#pragma unroll
    for (int p = 0; p < NPAIR; ++p) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            scratch[(lane & 31) * LDS_ + acc_row(v, lane)] = acc[p][v] * colscale;
            if constexpr (DT >= 2) scratch[(lane & 31) * LDS_ + 32 + acc_row(v, lane)] = acc[p + DT / 2][v] * colscale;
        }
        __syncthreads();
        // items: 32 rows x (PW / 4) groups of 4 columns
#pragma unroll
        for (int it = 0; it < 32 * (PW / 4) / kWave; ++it) {
            const int item = it * kWave + lane;
            const int r = item / (PW / 4), c4 = (item % (PW / 4)) * 4;
            const int row = row_base + r;
            if (row >= T) continue;
            float4 x1 = *reinterpret_cast<const float4*>(scratch + r * LDS_ + c4);
            float4 x2 = *reinterpret_cast<const float4*>(scratch + r * LDS_ + (DT >= 2 ? 32 : 16) + c4);
            const int d1 = (DT >= 2 ? p * 32 : 0) + c4, d2 = d1 + HALF;
            if (o.of) {
                st_nt(o.of + (int64_t)row * o.rsf + d1, x1);
                st_nt(o.of + (int64_t)row * o.rsf + d2, x2);
            }
            if (o.ob) {
                if (o.cos_t) {
                    const int64_t tr = ((o.tok0 + row) % o.period) * HALF + d1;
                    const float4 c = *reinterpret_cast<const float4*>(o.cos_t + tr);
                    const float4 sn = *reinterpret_cast<const float4*>(o.sin_t + tr);
                    // inverse rotation: s' = -sin; y1 = x1 c + x2 s', y2 = -x1 s' + x2 c
                    const float4 y1 = make_float4(x1.x * c.x - x2.x * sn.x, x1.y * c.y - x2.y * sn.y,
                                                  x1.z * c.z - x2.z * sn.z, x1.w * c.w - x2.w * sn.w);
                    const float4 y2 = make_float4(x1.x * sn.x + x2.x * c.x, x1.y * sn.y + x2.y * c.y,
                                                  x1.z * sn.z + x2.z * c.z, x1.w * sn.w + x2.w * c.w);
                    x1 = y1;
                    x2 = y2;
                }
                bf16x4 b1, b2;
                b1[0] = (bf16)x1.x; b1[1] = (bf16)x1.y; b1[2] = (bf16)x1.z; b1[3] = (bf16)x1.w;
                b2[0] = (bf16)x2.x; b2[1] = (bf16)x2.y; b2[2] = (bf16)x2.z; b2[3] = (bf16)x2.w;
                st_nt(o.ob + (int64_t)row * o.rsb + d1, b1);
                st_nt(o.ob + (int64_t)row * o.rsb + d2, b2);
            }
        }
        __syncthreads();
    }
}

// RowOut advanced to sequence b, head h (rows = tokens of sequence b).
__device__ __forceinline__ RowOut at_head(RowOut o, int b, int h, int T, int HD) {
    if (o.of) o.of += (int64_t)b * T * o.rsf + (int64_t)h * HD;
    if (o.ob) o.ob += (int64_t)b * T * o.rsb + (int64_t)h * HD;
    o.tok0 = (int64_t)b * T;
    return o;
}

// visibility of key kp from query qp
// (bitwise, not short-circuit: per-element masks compile to compares and
// selects, not to exec-mask branches)
__device__ __forceinline__ bool visible(int kp, int qp, int T, int window) {
    return (kp <= qp) & (qp < T) & ((window <= 0) | (kp >= qp - window));
}

// ============================ forward ============================
// Two workgroups per CU (2 waves per SIMD): registers are capped at 256.
template <int HD>
__global__ __launch_bounds__(kThreads, 2) void fa2_fwd_k(RowOut out, float* lse, const bf16* q, const bf16* k,
                                                         const bf16* v, int B, int T, int H, int window,
                                                         float scale_log2) {
    using G = Geo<HD>;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16* const lds = reinterpret_cast<bf16*>(smem_raw);  // stage s: K at 2 s TILE, V at (2 s + 1) TILE
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int nqb = (T + kOwn - 1) / kOwn;
    int bh, qb;
    block_coords(nqb, B * H, true, bh, qb);
    const int b = bh / H, h = bh % H;
    const int q0 = qb * kOwn, qw = q0 + wave * 32, my_q = qw + (lane & 31);
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;

    bf16x8 qf[G::KSTEPS];
    own_frags<HD>(qf, q + boff, rs, my_q, T, lane);
    f32x16 o[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    float m = -INFINITY, l = 0.f;

    int kstart = 0;
    if (window > 0) kstart = q0 - window > 0 ? q0 - window : 0;
    kstart = (kstart / kTile) * kTile;
    const int kend = (q0 + kOwn < T) ? q0 + kOwn : T;
    const int ntiles = kend > kstart ? (kend - kstart + kTile - 1) / kTile : 0;

    // Software pipeline: K runs one tile ahead of V, so iteration `it` holds
    // K(it + 1) and V(it) and issues the score MFMAs of tile it + 1 in the
    // same basic block as tile it's softmax (VALU), which the scheduler
    // interleaves.  Buffers: K(t) in stage t & 1 slot 0, V(t) in stage t & 1
    // slot 1; iteration it refills K(it + 2) and V(it + 1), whose previous
    // contents were last read in iteration it - 1.
    auto kbuf = [&](int t) { return lds + (2 * (t & 1)) * G::TILE; };
    auto vbuf = [&](int t) { return lds + (2 * (t & 1) + 1) * G::TILE; };
    // a tile is active for this wave unless the causal / window mask removes all of it
    auto active = [&](int t) {
        const int kv0 = kstart + t * kTile;
        return !(kv0 > qw + 31 || (window > 0 && kv0 + kTile - 1 < qw - window) || qw >= T);
    };
    auto scores = [&](const bf16* sK, f32x16 (&sc)[2]) {
        const unsigned rb = rowbase<HD>(opaque_lane(threadIdx.x % kWave));
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) sc[kb][e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) sc[kb] = mma(rowfrag_x<HD>(sK + kb * 32 * HD, rb, ks), qf[ks], sc[kb]);
    };
    auto mask = [&](f32x16 (&sc)[2], int kv0) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                sc[kb][e] = visible(kv0 + kb * 32 + acc_row(e, lane), my_q, T, window) ? sc[kb][e] : -INFINITY;
    };
    auto is_full = [&](int kv0) {
        return kv0 + kTile - 1 <= qw && qw + 31 < T && (window <= 0 || kv0 >= qw + 31 - window);
    };
    // softmax of tile scores sc (in place: p) with the running max / sum
    // update, in three parts: the new reference max (m_use; m itself is
    // moved by softmax_sum), the exponentials, the sum update
    auto softmax_max = [&](const f32x16 (&sc)[2]) {
        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) mt = fmaxf(mt, sc[kb][e]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave)) * scale_log2;
        const float m_new = fmaxf(m, mt);
        return m_new == -INFINITY ? 0.f : m_new;
    };
    auto softmax_sum = [&](float rsum, float alpha, float m_use) {
        rsum += __shfl_xor(rsum, 32, kWave);
        l = l * alpha + rsum;
        // m_use is 0 only while every score seen so far is masked (l = 0)
        m = l > 0.f ? m_use : -INFINITY;
    };
    auto softmax = [&](f32x16 (&sc)[2]) {
        const float m_use = softmax_max(sc);
        const float alpha = exp2_fast(m - m_use);
        float rsum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float pp = exp2_fast(fmaf(sc[kb][e], scale_log2, -m_use));
                sc[kb][e] = pp;
                rsum += pp;
            }
        softmax_sum(rsum, alpha, m_use);
        return alpha;
    };
    auto pv = [&](const f32x16 (&sc)[2], const bf16* sV, float alpha) {
        // skip the rescale (a multiply by 1) when the max moved for no row of the wave
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
        }
        // O^T += V^T P^T, P rounded to bf16 once (l keeps the fp32 sums)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const bf16x8 ph = accfrag(sc[kb], st);
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) o[dt] = mma(trfrag<HD>(sV, kb, st, dt, lane), ph, o[dt]);
            }
    };

    unsigned toff[TileU<HD, kTile>::N];
    tile_offsets<HD>(toff, rs);
    if (ntiles > 0) {
        dma_tile<HD>(kbuf(0), k + boff, rs, kstart, T, toff);
        dma_tile<HD>(vbuf(0), v + boff, rs, kstart, T, toff);
        if (ntiles > 1) dma_tile<HD>(kbuf(1), k + boff, rs, kstart + kTile, T, toff);
    }
    wait_vmem();
    __syncthreads();
    f32x16 sa[2], sb[2];  // scores of the current / next tile (the loop body runs twice per trip, roles swapped)
    if (ntiles > 0 && active(0)) scores(kbuf(0), sa);
    __syncthreads();  // every wave is done with K(0) before step 0 refills its buffer with K(2)
    auto step = [&](int it, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
        const int kv0 = kstart + it * kTile;
        if (it + 2 < ntiles) dma_tile<HD>(kbuf(it + 2), k + boff, rs, kv0 + 2 * kTile, T, toff);
        if (it + 1 < ntiles) dma_tile<HD>(vbuf(it + 1), v + boff, rs, kv0 + kTile, T, toff);
        const bool a_cur = active(it), a_nxt = it + 1 < ntiles && active(it + 1);
        if (a_cur && !is_full(kv0)) mask(cur, kv0);
        if (a_cur && a_nxt) {
            // the next tile's score MFMAs interleaved in program order with
            // this tile's softmax (exponentials two elements per MFMA)
            const float m_use = softmax_max(cur);
            const float alpha = exp2_fast(m - m_use);
            const bf16* sK = kbuf(it + 1);
            const unsigned rb = rowbase<HD>(opaque_lane(threadIdx.x % kWave));
            float rsum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e) nxt[kb][e] = 0.f;
            constexpr int EPM = 16 / G::KSTEPS;  // exponentials per MFMA: 32 per lane over 2 KSTEPS MFMAs
#pragma unroll
            for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    nxt[kb] = mma(rowfrag_x<HD>(sK + kb * 32 * HD, rb, ks), qf[ks], nxt[kb]);
#pragma unroll
                    for (int j = 0; j < EPM; ++j) {
                        const int flat = (ks * 2 + kb) * EPM + j, ckb = flat >> 4, ce = flat & 15;
                        const float pp = exp2_fast(fmaf(cur[ckb][ce], scale_log2, -m_use));
                        cur[ckb][ce] = pp;
                        rsum += pp;
                    }
                }
            softmax_sum(rsum, alpha, m_use);
            pv(cur, vbuf(it), alpha);
        } else {
            if (a_nxt) scores(kbuf(it + 1), nxt);
            if (a_cur) pv(cur, vbuf(it), softmax(cur));
        }
        wait_vmem();  // this thread's part of K(it + 2) / V(it + 1) has landed
        __syncthreads();
    };
    int it = 0;
    for (; it + 1 < ntiles; it += 2) {
        step(it, sa, sb);
        step(it + 1, sb, sa);
    }
    if (it < ntiles) step(it, sa, sb);
    const float inv_l = l > 0.f ? 1.0f / l : 0.f;
    if (lane < 32 && my_q < T) lse[((int64_t)b * T + my_q) * H + h] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 68;
    store_rows<HD>(at_head(out, b, h, T, HD), qw, T, o, inv_l, scratch, lane);
}

// ============================ backward: dQ ============================
template <int HD>
__global__ __launch_bounds__(kThreads, 2) void fa2_dq_k(RowOut dq, const bf16* q, const bf16* k, const bf16* v,
                                                     const bf16* dout, const float* lse, const float* dbuf,
                                                     int B, int T, int H, int window, float scale_log2,
                                                     float scale) {
    using G = Geo<HD>;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16* const lds = reinterpret_cast<bf16*>(smem_raw);  // stage s: K at 2 s TILE, V at (2 s + 1) TILE
    const int lane = threadIdx.x % kWave, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nqb = (T + kOwn - 1) / kOwn;
    int bh, qb;
    block_coords(nqb, B * H, true, bh, qb);
    const int b = bh / H, h = bh % H;
    const int q0 = qb * kOwn, qw = q0 + wave * 32, my_q = qw + (lane & 31);
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;

    bf16x8 qf[G::KSTEPS], df[G::KSTEPS];
    own_frags<HD>(qf, q + boff, rs, my_q, T, lane);
    own_frags<HD>(df, dout + boff, rs, my_q, T, lane);
    const int64_t bth = ((int64_t)b * T + (my_q < T ? my_q : 0)) * H + h;
    const float my_lse2 = lse[bth] * kLog2e;
    const float my_D = dbuf[bth];

    f32x16 acc[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;

    int kstart = 0;
    if (window > 0) kstart = q0 - window > 0 ? q0 - window : 0;
    kstart = (kstart / kTile) * kTile;
    const int kend = (q0 + kOwn < T) ? q0 + kOwn : T;
    const int ntiles = kend > kstart ? (kend - kstart + kTile - 1) / kTile : 0;

    unsigned toff[TileU<HD, kTile>::N];
    tile_offsets<HD>(toff, rs);
    if (ntiles > 0) {
        dma_tile<HD>(lds, k + boff, rs, kstart, T, toff);
        dma_tile<HD>(lds + G::TILE, v + boff, rs, kstart, T, toff);
    }
    wait_vmem();
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int kv0 = kstart + it * kTile;
        const int cur = it & 1;
        const bool more = it + 1 < ntiles;
        if (more) {
            dma_tile<HD>(lds + (2 * (cur ^ 1)) * G::TILE, k + boff, rs, kv0 + kTile, T, toff);
            dma_tile<HD>(lds + (2 * (cur ^ 1) + 1) * G::TILE, v + boff, rs, kv0 + kTile, T, toff);
        }
        const bf16* sK = lds + (2 * cur) * G::TILE;
        const bf16* sV = lds + (2 * cur + 1) * G::TILE;
        const bool skip = kv0 > qw + 31 || (window > 0 && kv0 + kTile - 1 < qw - window) || qw >= T;
        if (!skip) {
            const int lane = opaque_lane(threadIdx.x % kWave);
            const unsigned rb = rowbase<HD>(lane);
            unsigned tb0, tb1;
            trbase<HD>(lane, tb0, tb1);
            const bool full = kv0 + kTile - 1 <= qw && qw + 31 < T && (window <= 0 || kv0 >= qw + 31 - window);
            // one 32-key half at a time keeps only one S / dP pair live
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                f32x16 s, dp;
#pragma unroll
                for (int e = 0; e < 16; ++e) s[e] = dp[e] = 0.f;
#pragma unroll
                for (int ks = 0; ks < G::KSTEPS; ++ks) {
                    s = mma(rowfrag_x<HD>(sK + kb * 32 * HD, rb, ks), qf[ks], s);
                    dp = mma(rowfrag_x<HD>(sV + kb * 32 * HD, rb, ks), df[ks], dp);
                }
                // full tiles skip the per-element mask (a wave-uniform branch)
                auto ds = [&](auto masked) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const bool ok = !decltype(masked)::value ||
                                        visible(kv0 + kb * 32 + acc_row(e, lane), my_q, T, window);
                        const float p = ok ? exp2_fast(fmaf(s[e], scale_log2, -my_lse2)) : 0.f;
                        s[e] = p * (dp[e] - my_D);
                    }
                };
                if (full)
                    ds(std::false_type{});
                else
                    ds(std::true_type{});
                // dQ^T += K^T dS^T
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const bf16x8 db = accfrag(s, st);
#pragma unroll
                    for (int dt = 0; dt < G::DT; ++dt) acc[dt] = mma(trfrag_x<HD>(sK, tb0, tb1, kb, st, dt), db, acc[dt]);
                }
            }
        }
        wait_vmem();  // this thread's part of the next K / V tile has landed
        __syncthreads();
    }
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 68;
    store_rows<HD>(at_head(dq, b, h, T, HD), qw, T, acc, scale, scratch, lane);
}

// ============================ backward: dK, dV ============================
// dK and dV in one pass: S and dP are computed once per (key, query) tile,
// P feeds dV^T += dO^T P and dS = P (dP - D) feeds dK^T += Q^T dS.  Both
// accumulator sets (2 x 64 registers at hd 128) and the own K fragments stay
// in registers; the own V rows live in LDS (read as row fragments for dP), so
// two workgroups still share a CU without spills.  Q / dO stream in 32-row
// tiles (double-buffered, direct-to-LDS).
//
// With WDS the bf16 dS that feeds the dK product is also stored, for the dQ
// product to read instead of recomputing S and dP (fa2_dq_ds_k), in the
// layout that product's B operand takes: per (b, h), 32-query block q32 and
// 32-key block k32, 1024 bf16 at ds + ((bh * n32 + q32) * n32 + k32) * 1024
// (n32 = ceil(T / 32)), fragment s (keys 16 s..16 s+15) at s * 512, lane l
// (query l % 32) at 8 l: keys 16 s + 4 (l / 32) + {0..3, 8..11}.  A wave turns
// its 32 x 32 dS^T block (lane = key) around through 2.3 KB of wave-private
// LDS and stores the two fragments as two 1 KB rows of 16-byte pieces.  Only
// blocks that block_hidden keeps are written (masked scores as zeros), and
// only those are used by the dQ product.
constexpr int kDkvTile = 32;
constexpr int kDsBlock = 32 * 32;  // bf16 elements per stored dS block
constexpr int kStgLd = 36;         // staging row stride (bf16): 8-byte writes and transposed reads conflict-free

// The 32 x 32 score block of keys kb0..kb0+31 and queries q0..q0+31 (both
// 32-aligned) holds no visible score: the dK / dV kernel skips it and writes
// no dS for it, and the dQ-from-dS kernel skips it too.
__device__ __forceinline__ bool block_hidden(int kb0, int q0, int T, int window) {
    return q0 + 31 < kb0 || (window > 0 && q0 > kb0 + 31 + window) || kb0 >= T || q0 >= T;
}

// s_waitcnt vmcnt(N) (lgkmcnt / expcnt left open).
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
    static_assert(N >= 0 && N < 16, "vmcnt");
    __builtin_amdgcn_s_waitcnt(N | 0x0F70);
}

// Transposed fragment of an unswizzled 32-row tile with row stride ld (bf16):
// lane l gets column l % 32, rows 16 s + 4 (l / 32) + {0..3, 8..11}.
__device__ __forceinline__ bf16x8 trfrag_plain(const bf16* t, int ld, int s, int lane) {
    const int g = lane >> 4, src = lane & 15;
    const int row = 16 * s + 4 * (g >> 1) + (src >> 2), col = 16 * (g & 1) + 4 * (src & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + row * ld + col));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (row + 8) * ld + col));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int HD, bool WDS>
constexpr size_t dkv_fused_lds() {
    const size_t tiles = 4 * (size_t)kDkvTile * HD * sizeof(bf16);  // Q, dO x 2 stages
    const size_t own_v = (size_t)kOwn * HD * sizeof(bf16);
    const size_t ld = 4 * kDkvTile * sizeof(float);                 // LSE, D x 2 stages
    const size_t stg = WDS ? 4 * 32 * kStgLd * sizeof(bf16) : 0;   // dS transpose staging, per wave
    const size_t loop = tiles + own_v + ld + stg;
    const size_t stage = 4 * 32 * 68 * sizeof(float);               // store_rows staging
    return loop > stage ? loop : stage;
}

template <int HD, bool WDS>
__global__ __launch_bounds__(kThreads, 2) void fa2_dkv_fused_k(RowOut out_k, RowOut out_v, const bf16* q,
                                                               const bf16* k, const bf16* v, const bf16* dout,
                                                               const float* lse, const float* dbuf, bf16* ds_out,
                                                               int B, int T, int H, int window, float scale_log2,
                                                               float scale) {
    using G = Geo<HD>;
    constexpr int KT = kDkvTile, TT = KT * HD;  // rows, bf16 elements per streamed tile
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16* const lds = reinterpret_cast<bf16*>(smem_raw);  // stage s: Q at 2 s TT, dO at (2 s + 1) TT
    bf16* const sV = lds + 4 * TT;                        // the workgroup's own 128 V rows
    float* const sLD = reinterpret_cast<float*>(sV + kOwn * HD);
    const int lane = threadIdx.x % kWave, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    bf16* const stg = reinterpret_cast<bf16*>(sLD + 4 * KT) + wave * 32 * kStgLd;
    const int nkb = (T + kOwn - 1) / kOwn;
    int bh, kblk;
    block_coords(nkb, B * H, false, bh, kblk);
    const int b = bh / H, h = bh % H;
    const int k0 = kblk * kOwn, kw = k0 + wave * 32, my_k = kw + (lane & 31);
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;

    bf16x8 kf[G::KSTEPS];
    own_frags<HD>(kf, k + boff, rs, my_k, T, lane);

    f32x16 adk[G::DT], adv[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) adk[dt][e] = adv[dt][e] = 0.f;

    const int qstart = (k0 / KT) * KT;
    int qend = T;
    if (window > 0 && k0 + kOwn - 1 + window + 1 < T) qend = k0 + kOwn - 1 + window + 1;
    const int ntiles = qend > qstart ? (qend - qstart + KT - 1) / KT : 0;

    // LSE / D of a query tile straight into LDS: wave 0, lanes 0..KT-1 the
    // LSE values, lanes KT..2 KT-1 the D values (4-byte copies, rows past T
    // repeat row 0; their scores are masked)
    auto dma_ld = [&](int qt0, int stage) {
        if (wave == 0) {
            const int j = lane % KT, qq = qt0 + j;
            const int64_t i = ((int64_t)b * T + (qq < T ? qq : 0)) * H + h;
            dma4(lane < KT ? lse + i : dbuf + i, lds_addr(sLD + stage * 2 * KT));
        }
    };
    {
        unsigned voff[TileU<HD, kOwn>::N];
        tile_offsets<HD, kOwn>(voff, rs);
        dma_tile<HD, kOwn>(sV, v + boff, rs, k0, T, voff);
    }
    unsigned toff[TileU<HD, KT>::N];
    tile_offsets<HD, KT>(toff, rs);
    if (ntiles > 0) {
        dma_tile<HD, KT>(lds, q + boff, rs, qstart, T, toff);
        dma_tile<HD, KT>(lds + TT, dout + boff, rs, qstart, T, toff);
        dma_ld(qstart, 0);
    }
    wait_vmem();
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int qt0 = qstart + it * KT;
        const int cur = it & 1;
        const bool more = it + 1 < ntiles;
        if (more) {
            dma_tile<HD, KT>(lds + (2 * (cur ^ 1)) * TT, q + boff, rs, qt0 + KT, T, toff);
            dma_tile<HD, KT>(lds + (2 * (cur ^ 1) + 1) * TT, dout + boff, rs, qt0 + KT, T, toff);
            dma_ld(qt0 + KT, cur ^ 1);
        }
        const bf16* sQ = lds + (2 * cur) * TT;
        const bf16* sD = lds + (2 * cur + 1) * TT;
        const float* sL = sLD + cur * 2 * KT;
        const float* sDl = sL + KT;
        if (!block_hidden(kw, qt0, T, window)) {
            const int lane = opaque_lane(threadIdx.x % kWave);
            const unsigned rb = rowbase<HD>(lane);
            unsigned tb0, tb1;
            trbase<HD>(lane, tb0, tb1);
            const bool full = qt0 >= kw + 31 && qt0 + KT <= T && kw + 31 < T &&
                              (window <= 0 || kw >= qt0 + KT - 1 - window);
            f32x16 s, dp;
#pragma unroll
            for (int e = 0; e < 16; ++e) s[e] = dp[e] = 0.f;
#pragma unroll
            for (int ks = 0; ks < G::KSTEPS; ++ks) {
                s = mma(rowfrag_x<HD>(sQ, rb, ks), kf[ks], s);
                dp = mma(rowfrag_x<HD>(sD, rb, ks), rowfrag_x<HD>(sV + wave * 32 * HD, rb, ks), dp);
            }
            // lane: key my_k; rows: queries qt0 + acc_row(e); s becomes P, dp becomes dS.
            // Full tiles skip the per-element mask (a wave-uniform branch).
            auto ds = [&](auto masked) {
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int q4 = 8 * a + 4 * (lane >> 5);
                    const float4 l4 = *reinterpret_cast<const float4*>(sL + q4);
                    const float4 d4 = *reinterpret_cast<const float4*>(sDl + q4);
                    const float lvv[4] = {l4.x * kLog2e, l4.y * kLog2e, l4.z * kLog2e, l4.w * kLog2e};
                    const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int e = 4 * a + j;
                        const bool ok = !decltype(masked)::value ||
                                        ((my_k < T) & visible(my_k, qt0 + q4 + j, T, window));
                        const float pv = ok ? exp2_fast(fmaf(s[e], scale_log2, -lvv[j])) : 0.f;
                        s[e] = pv;
                        dp[e] = pv * (dp[e] - dv4[j]);
                    }
                }
            };
            if (full)
                ds(std::false_type{});
            else
                ds(std::true_type{});
            if constexpr (WDS) {
                // dS^T block (lane = key; queries 16 st + 4 g + {0..3, 8..11}, g =
                // lane / 32) into the staging rows, read back transposed (lane =
                // query) and stored as the block's two B fragments
                const int g = lane >> 5;
                bf16* const srow = stg + (lane & 31) * kStgLd + 4 * g;
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const bf16x8 f = accfrag(dp, st);
                    *reinterpret_cast<bf16x4*>(srow + 16 * st) = __builtin_shufflevector(f, f, 0, 1, 2, 3);
                    *reinterpret_cast<bf16x4*>(srow + 16 * st + 8) = __builtin_shufflevector(f, f, 4, 5, 6, 7);
                }
                const int n32 = (T + 31) / 32;
                bf16* const blk = ds_out + (((int64_t)bh * n32 + qt0 / 32) * n32 + kw / 32) * kDsBlock + lane * 8;
                // nontemporal: 1 KB of whole lines per store, streamed past L2
                // (allocated there, they evicted the Q / dO tiles the other
                // workgroups of the head still read)
#pragma unroll
                for (int st = 0; st < 2; ++st)
                    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, trfrag_plain(stg, kStgLd, st, lane)),
                                                reinterpret_cast<u32x4*>(blk + st * 512));
            }
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const bf16x8 fp = accfrag(s, st), fs = accfrag(dp, st);
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) {
                    adv[dt] = mma(trfrag_x<HD>(sD, tb0, tb1, 0, st, dt), fp, adv[dt]);
                    adk[dt] = mma(trfrag_x<HD>(sQ, tb0, tb1, 0, st, dt), fs, adk[dt]);
                }
            }
        }
        // this thread's part of the next Q / dO tile (and its LSE / D) has
        // landed; the tile's two dS stores, issued after those loads, may
        // still be in flight (vmcnt counts in issue order)
        if (WDS && !block_hidden(kw, qt0, T, window))
            wait_vmem_n<2>();
        else
            wait_vmem();
        __syncthreads();
    }
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 68;
    store_rows<HD>(at_head(out_v, b, h, T, HD), kw, T, adv, 1.0f, scratch, lane);
    store_rows<HD>(at_head(out_k, b, h, T, HD), kw, T, adk, scale, scratch, lane);
}

// ============================ backward: dQ from stored dS ============================
// dQ^T += K^T dS^T over the key tiles of the query block, from the dS blocks
// the dK / dV kernel stored (the same bf16 values the dQ kernel above forms
// for its product, so this is that kernel's result without the S / dP
// recompute).  One 512-thread workgroup per CU owns 256 queries (8 waves x
// 32) and streams 64-key tiles through three LDS stages, loads two tiles
// ahead: the K rows (natural, swizzled; K^T read transposed as in fa2_dq_k)
// and each wave's four dS fragments of the tile (4 KB contiguous in global
// memory and in LDS, read back as 16 bytes per lane).  Every load is a
// direct-to-LDS copy, so all vector-memory waits are the explicit ones below.
constexpr int kDqThreads = 512, kDqOwn = 256, kDqStages = 3;

template <int HD>
constexpr size_t dq_ds_lds() {
    const size_t stage = ((size_t)Geo<HD>::TILE + (kDqThreads / kWave) * 2 * kDsBlock) * sizeof(bf16);
    const size_t tiles = kDqStages * stage;
    const size_t out = (kDqThreads / kWave) * 32 * 68 * sizeof(float);  // store_rows staging
    return tiles > out ? tiles : out;
}

template <int HD>
__global__ __launch_bounds__(kDqThreads) void fa2_dq_ds_k(RowOut dq, const bf16* k, const bf16* ds, int B, int T,
                                                         int H, int window, float scale) {
    using G = Geo<HD>;
    constexpr int NK = TileU<HD, kTile, kDqThreads>::N;
    constexpr bool K_ALL = kTile * G::NCH % kDqThreads == 0;  // every wave copies part of each K tile
    constexpr int SDS = 2 * kDsBlock;              // bf16 elements of one wave's dS fragments per tile (4 KB)
    constexpr int STG = G::TILE + (kDqThreads / kWave) * SDS;  // bf16 elements per stage
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16* const lds = reinterpret_cast<bf16*>(smem_raw);
    const int lane = threadIdx.x % kWave, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nqb = (T + kDqOwn - 1) / kDqOwn, n32 = (T + 31) / 32;
    int bh, qb;
    block_coords(nqb, B * H, true, bh, qb);
    const int b = bh / H, h = bh % H;
    const int q0 = qb * kDqOwn, qw = q0 + wave * 32;
    const int64_t rs = (int64_t)H * HD;
    const int64_t boff = (int64_t)b * T * rs + (int64_t)h * HD;
    // this wave's row of dS blocks (a wave past T reads row n32 - 1, unused)
    const bf16* const dsw = ds + ((int64_t)bh * n32 + (qw / 32 < n32 ? qw / 32 : n32 - 1)) * n32 * kDsBlock;

    f32x16 acc[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;

    int kstart = 0;
    if (window > 0) kstart = q0 - window > 0 ? q0 - window : 0;
    kstart = (kstart / kTile) * kTile;
    const int kend = (q0 + kDqOwn < T) ? q0 + kDqOwn : T;
    const int ntiles = kend > kstart ? (kend - kstart + kTile - 1) / kTile : 0;

    unsigned toff[NK];
    tile_offsets<HD, kTile, NK, kDqThreads>(toff, rs);
    const unsigned lds0 = lds_addr(smem_raw);
    // tile t into stage t % 3: K rows, then this wave's 4 KB of dS fragments
    // (blocks k32, k32 + 1 of its row).  A block hidden from this wave is
    // never written and never read back: its copy is pointed at the row's
    // block kstart / 32 (already fetched by the first tile, so an L2 hit)
    // instead, which keeps the per-tile copy count the same for every wave.
    const int kdummy = kstart / 32;
    auto load = [&](int t) {
        const int kv0 = kstart + t * kTile, stage = t % kDqStages;
        dma_tile<HD, kTile, NK, kDqThreads>(lds + stage * STG, k + boff, rs, kv0, T, toff);
        const unsigned dl = lds0 + (unsigned)(stage * STG + G::TILE + wave * SDS) * 2u;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int blk = block_hidden(kv0 + 32 * kb, qw, T, window) ? kdummy : kv0 / 32 + kb;
#pragma unroll
            for (int s = 0; s < 2; ++s)
                dma16s(dsw + (int64_t)blk * kDsBlock, (unsigned)(s * 1024 + lane * 16), dl + (2 * kb + s) * 1024);
        }
    };
    // wait for the older of two tiles in flight: a wave's vector-memory
    // instructions per tile are its K copies (NK, or none for the waves that
    // a small K tile leaves out) and its 4 dS copies
    auto wait_older = [&]() {
        if (K_ALL || wave * kWave < kTile * G::NCH)
            wait_vmem_n<NK + 4>();
        else
            wait_vmem_n<4>();
    };
    if (ntiles > 0) load(0);
    if (ntiles > 1) load(1);
    if (ntiles > 1)
        wait_older();
    else
        wait_vmem();
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int kv0 = kstart + it * kTile;
        if (it + 2 < ntiles) load(it + 2);  // into the stage tile it - 1 used (retired by the last barrier)
        const bf16* sK = lds + (it % kDqStages) * STG;
        const bf16* sS = sK + G::TILE + wave * SDS;
        const int lane = opaque_lane(threadIdx.x % kWave);
        unsigned tb0, tb1;
        trbase<HD>(lane, tb0, tb1);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            if (block_hidden(kv0 + 32 * kb, qw, T, window)) continue;  // wave-uniform
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const bf16x8 db = *reinterpret_cast<const bf16x8*>(sS + (2 * kb + st) * 512 + lane * 8);
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) acc[dt] = mma(trfrag_x<HD>(sK, tb0, tb1, kb, st, dt), db, acc[dt]);
            }
        }
        // tile it + 1 has landed (this thread's part); tile it + 2's loads may
        // still be in flight
        if (it + 2 < ntiles)
            wait_older();
        else
            wait_vmem();
        __syncthreads();
    }
    float* scratch = reinterpret_cast<float*>(smem_raw) + wave * 32 * 68;
    store_rows<HD>(at_head(dq, b, h, T, HD), qw, T, acc, scale, scratch, lane);
}

// D = rowsum(dO * O) (ops.mojo:329-346) per (token, head) row: bf16 dO (the
// values the dP products read) against fp32 O, HD / 16 lanes per row, each
// 16 columns (all six 16-byte loads issued before the arithmetic), then a
// butterfly over those lanes.
template <int HD>
__global__ __launch_bounds__(kThreads) void fa2_d_k(float* d, const float* o, const bf16* dout, int64_t rows) {
    constexpr int LPR = HD / 16;
    const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t r = gid / LPR;
    const int c = (int)(gid % LPR);
    float sum = 0.f;
    if (r < rows) {
        const bf16* gp = dout + r * HD + c * 16;
        const float* op = o + r * HD + c * 16;
        const bf16x8 g0 = *reinterpret_cast<const bf16x8*>(gp), g1 = *reinterpret_cast<const bf16x8*>(gp + 8);
        const float4 a0 = *reinterpret_cast<const float4*>(op), a1 = *reinterpret_cast<const float4*>(op + 4);
        const float4 a2 = *reinterpret_cast<const float4*>(op + 8), a3 = *reinterpret_cast<const float4*>(op + 12);
        sum = a0.x * (float)g0[0] + a0.y * (float)g0[1] + a0.z * (float)g0[2] + a0.w * (float)g0[3] +
              a1.x * (float)g0[4] + a1.y * (float)g0[5] + a1.z * (float)g0[6] + a1.w * (float)g0[7];
        sum += a2.x * (float)g1[0] + a2.y * (float)g1[1] + a2.z * (float)g1[2] + a2.w * (float)g1[3] +
               a3.x * (float)g1[4] + a3.y * (float)g1[5] + a3.z * (float)g1[6] + a3.w * (float)g1[7];
    }
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, kWave);
    if (r < rows && c == 0) d[r] = sum;
}

template <int HD>
constexpr size_t fa2_lds(bool with_ld) {
    const size_t tiles = 4 * (size_t)Geo<HD>::TILE * sizeof(bf16) + (with_ld ? 4 * kTile * sizeof(float) : 0);
    const size_t stage = 4 * 32 * 68 * sizeof(float);
    return tiles > stage ? tiles : stage;
}

template <int HD>
int32_t flash_hd(hipStream_t st, AttnOp op, float* o1, float* o2, const FlashOut& fo, const bf16* q, const bf16* k,
                 const bf16* v, const bf16* dout, const float* lse, const float* dbuf, int B, int T, int H,
                 int window, float sc) {
    const float scale = sc > 0.f ? sc : 1.0f / sqrtf((float)HD);
    const float scale_log2 = scale * kLog2e;
    const unsigned grid = (unsigned)(((T + kOwn - 1) / kOwn) * B * H);
    const int64_t rs = (int64_t)H * HD, brs = fo.brs > 0 ? fo.brs : rs;
    if (op == AttnOp::FWD) {
        const RowOut out{o1, fo.b1, rs, brs, nullptr, nullptr, 0, 1};
        fa2_fwd_k<HD><<<grid, kThreads, fa2_lds<HD>(false), st>>>(out, o2, q, k, v, B, T, H, window, scale_log2);
        return check_launch("flash_attn_fwd (bf16 operands)");
    }
    const int64_t period = fo.period > 0 ? fo.period : (int64_t)B * T;
    if (op == AttnOp::DQ) {
        const RowOut out{o1, fo.b1, rs, brs, fo.cos_t, fo.sin_t, 0, period};
        fa2_dq_k<HD><<<grid, kThreads, fa2_lds<HD>(false), st>>>(out, q, k, v, dout, lse, dbuf, B, T, H, window,
                                                                 scale_log2, scale);
        return check_launch("flash_attn_bwd_dq (bf16 operands)");
    }
    const RowOut ov{o2, fo.b2, rs, brs, nullptr, nullptr, 0, 1};
    const RowOut ok{o1, fo.b1, rs, brs, fo.cos_t, fo.sin_t, 0, period};
    if (fo.ds)
        fa2_dkv_fused_k<HD, true><<<grid, kThreads, dkv_fused_lds<HD, true>(), st>>>(ok, ov, q, k, v, dout, lse, dbuf, fo.ds,
                                                                          B, T, H, window, scale_log2, scale);
    else
        fa2_dkv_fused_k<HD, false><<<grid, kThreads, dkv_fused_lds<HD, false>(), st>>>(ok, ov, q, k, v, dout, lse, dbuf,
                                                                           nullptr, B, T, H, window, scale_log2, scale);
    return check_launch("flash_attn_bwd_dkv (bf16 operands)");
}

template <int HD>
int32_t flash_dq_ds_hd(hipStream_t st, const FlashOut& fo, const bf16* k, const bf16* ds, int B, int T, int H,
                       int window) {
    const float scale = 1.0f / sqrtf((float)HD);
    const unsigned grid = (unsigned)(((T + kDqOwn - 1) / kDqOwn) * B * H);
    const int64_t rs = (int64_t)H * HD, brs = fo.brs > 0 ? fo.brs : rs;
    const int64_t period = fo.period > 0 ? fo.period : (int64_t)B * T;
    const RowOut out{nullptr, fo.b1, rs, brs, fo.cos_t, fo.sin_t, 0, period};
    fa2_dq_ds_k<HD><<<grid, kDqThreads, dq_ds_lds<HD>(), st>>>(out, k, ds, B, T, H, window, scale);
    return check_launch("flash_attn_bwd_dq from dS (bf16 operands)");
}

}  // namespace

int64_t flash_ds_elems(int64_t B, int64_t T, int64_t H) {
    return B * H * ((T + 31) / 32) * ((T + 31) / 32) * kDsBlock;
}

int32_t flash_d_bf16(hipStream_t st, float* d, const float* o, const bf16* dout, int64_t B, int64_t T, int64_t H,
                     int64_t HD) {
    const int64_t rows = B * T * H;
    if (rows <= 0) return AR_OK;
    if (HD != 32 && HD != 64 && HD != 128)
        return set_error(AR_EUNSUPPORTED, "flash attention D: head_dim %lld not in {32, 64, 128}", (long long)HD);
    const int64_t threads = rows * (HD / 16);
    const unsigned grid = (unsigned)((threads + kThreads - 1) / kThreads);
    if (HD == 128) fa2_d_k<128><<<grid, kThreads, 0, st>>>(d, o, dout, rows);
    else if (HD == 64) fa2_d_k<64><<<grid, kThreads, 0, st>>>(d, o, dout, rows);
    else fa2_d_k<32><<<grid, kThreads, 0, st>>>(d, o, dout, rows);
    return check_launch("flash attention D (bf16 dO)");
}

int32_t flash_dq_ds_bf16(hipStream_t st, const FlashOut& fo, const bf16* k, const bf16* ds, int64_t B, int64_t T,
                         int64_t H, int64_t HD, int64_t window) {
    if (B <= 0 || T <= 0 || H <= 0) return B == 0 || T == 0 ? AR_OK : set_error(AR_EINVAL, "flash attention: bad shape");
    if (((T + kOwn - 1) / kOwn) * B * H > 0x7fffffff || T > (1 << 30))
        return set_error(AR_EINVAL, "flash attention: shape too large");
    if (!fo.b1 || !ds) return set_error(AR_EINVAL, "flash attention dQ from dS: null output / dS");
    const int w = window > T ? (int)T : (int)window;
    switch (HD) {
        case 32: return flash_dq_ds_hd<32>(st, fo, k, ds, (int)B, (int)T, (int)H, w);
        case 64: return flash_dq_ds_hd<64>(st, fo, k, ds, (int)B, (int)T, (int)H, w);
        case 128: return flash_dq_ds_hd<128>(st, fo, k, ds, (int)B, (int)T, (int)H, w);
        default: return set_error(AR_EUNSUPPORTED, "flash attention: head_dim %lld not in {32, 64, 128}", (long long)HD);
    }
}

int32_t flash_attn_bf16(hipStream_t st, AttnOp op, float* o1, float* o2, const FlashOut& fo, const bf16* q,
                        const bf16* k, const bf16* v, const bf16* dout, const float* lse, const float* dbuf, int64_t B,
                        int64_t T, int64_t H, int64_t HD, int64_t window, float scale) {
    if (B <= 0 || T <= 0 || H <= 0) return B == 0 || T == 0 ? AR_OK : set_error(AR_EINVAL, "flash attention: bad shape");
    if (((T + kOwn - 1) / kOwn) * B * H > 0x7fffffff || T > (1 << 30))
        return set_error(AR_EINVAL, "flash attention: shape too large");
    const int w = window > T ? (int)T : (int)window;  // a window >= T is full causal
    switch (HD) {
        case 32: return flash_hd<32>(st, op, o1, o2, fo, q, k, v, dout, lse, dbuf, (int)B, (int)T, (int)H, w, scale);
        case 64: return flash_hd<64>(st, op, o1, o2, fo, q, k, v, dout, lse, dbuf, (int)B, (int)T, (int)H, w, scale);
        case 128: return flash_hd<128>(st, op, o1, o2, fo, q, k, v, dout, lse, dbuf, (int)B, (int)T, (int)H, w, scale);
        default: return set_error(AR_EUNSUPPORTED, "flash attention: head_dim %lld not in {32, 64, 128}", (long long)HD);
    }
}

}  // namespace ar
