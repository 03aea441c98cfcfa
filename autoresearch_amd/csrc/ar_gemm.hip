// ar_gemm.hip -- MFMA GEMMs for gfx950: the reference's three linear kernels
// linear_fwd (NT, ops.mojo:110-203), linear_bwd_dx (NN, ops.mojo:870-950) and
// linear_bwd_dw (TN, ops.mojo:953-1033), and the Muon Polar-Express products
// that reuse them (optimizer.mojo:288-336).
//
// One kernel template covers all three layouts.  In GEMM terms it computes
//   C[mo, no] (=, +=) sum_r A(mo, r) * B(no, r)
// where each operand is stored either "K-major" (r contiguous: X[M,K] of NT)
// or "MN-major" (mo/no contiguous: W[N,K] read as B of NN, dY and X of TN).
//   NT: A = X  [M,K] K-major,  B = W  [N,K] K-major
//   NN: A = dY [M,N] K-major,  B = W  [N,K] MN-major  (reduction over N)
//   TN: A = dY [M,N] MN-major, B = X  [M,K] MN-major  (reduction over M)
//
// Design (CDNA4):
//   * 256 threads = 4 wave64s, block tile 128x128, each wave a 64x64 quadrant
//     computed as 2x2 MFMA 32x32 tiles (v_mfma_f32_32x32x16_bf16 for bf16
//     compute, v_mfma_f32_32x32x2_f32 for exact fp32 compute).
//   * K-major operands are staged through LDS in [row][k] layout (k
//     contiguous, 16-byte padded rows) so every MFMA fragment is one
//     ds_read_b128 (bf16) or ds_read_b32 (fp32).  With bf16 compute an
//     MN-major operand stays in its natural [k][row] layout (16-byte loads
//     and stores, chunks XOR-swizzled by k) and each fragment is two
//     ds_read_b64_tr_b16 transpose reads; with fp32 compute it is transposed
//     in registers on the way in.
//   * The epilogue stages each wave's accumulators through LDS and writes C
//     (and reads the epilogue operand) as row-contiguous 4-wide vectors.
//   * Two LDS stages; the next k-tile's global loads are issued before the
//     current tile's MFMAs, one barrier per k-tile.
//   * 1-D grid, remapped so each XCD (8 per MI355X, workgroups dispatched
//     round-robin) owns a contiguous run of row-major tiles: the A row-panel
//     a tile reads stays in that XCD's L2.
//   * TN reduces over M = B*T (65536 at the benchmark size) into a small
//     output, so it is split over the reduction: each split writes an fp32
//     partial and a second kernel adds the partials in split order
//     (deterministic; the reference's single-block loop over M is serial).
#include "ar_internal.hpp"

#include <stdlib.h>

#include <mutex>
#include <type_traits>

using namespace ar;

namespace {

// Block tile BM x BN computed by NWM x NWN wave64s; each wave owns a
// (BM/NWM) x (BN/NWN) sub-tile made of 32x32 MFMA tiles.
template <int BM_, int BN_, int NWM_, int NWN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, NWM = NWM_, NWN = NWN_;
    static constexpr int THREADS = 64 * NWM * NWN;
    static constexpr int WM = BM / NWM, WN = BN / NWN;
    static constexpr int TM = WM / 32, TN = WN / 32;
};
// 128x128, 4 waves of 64x64: small problems (Muon, config 1) keep >= 1 tile per CU.
using TileS = Tile<128, 128, 2, 2>;
// 256x256, 8 waves of 128x64: the model GEMMs (M = B*T).  Per k-step a wave
// reads 4 A + 2 B fragments for 8 MFMAs, and a block re-reads each operand
// panel half as often as with 128x128 tiles.
using TileL = Tile<256, 256, 2, 4>;

// Epilogues.  STORE: C = acc.  ACCUM: C += acc.  PARTIAL: split-K partial.
// ADD: C = R + acc (R = aux, fp32, row stride ldc; may alias C).
// RELU2: C = relu(acc)^2, the activation only (c_fc + relu_squared_fwd,
//   ops.mojo:486-497, fused; the pre-activation is not kept).
// SOFTCAP: C = cap * tanh(acc / cap) (lm_head + softcap_fwd, ops.mojo:500-510).
// AXPBY: C = cap acc + beta aux (aux fp32, same batch stride / row stride as
//   C): the Polar Express combinations B = b A + c A^2 and X' = a X + B X
//   (optimizer.mojo:310-330) folded into the product that precedes them.
// RELU2_BWD: C = a > 0 ? 2 sqrt(a) acc : 0 with a = aux the stored activation
//   (TC, row stride ldc): relu(h)^2 = a gives h = sqrt(a) where h > 0, so
//   relu_squared_bwd's 2 h (ops.mojo:1126-1140) comes from the activation,
//   whose bf16 rounding perturbs sqrt(a) by at most 2^-10 relative.
// QKV (persistent kernel, head-aligned waves): the q | k | v product's
//   post-processing of qkv_post (ar_fused.hip) on the fp32 accumulators: q and
//   k rotated by rope_fwd (ops.mojo:209-238) and scaled by their per-head
//   RMSNorm (ops.mojo:61-104, model.mojo:680-691), v plus gate x value
//   embedding (ve_apply_fwd, ops.mojo:544-560), each written as bf16 into its
//   own [M, C] buffer.
// DOUT_D (persistent kernel, head-aligned waves): C = acc as bf16 (the
//   attention-output gradient dO of the c_proj dX product) and
//   D[row, head] = sum_d bf16(dO)[row, d] O[row, d] (flash_attn_bwd_precompute_d,
//   ops.mojo:329-346, on the bf16 dO the dP products read).
enum Epi { EPI_STORE = 0, EPI_ACCUM = 1, EPI_PARTIAL = 2, EPI_ADD = 3, EPI_RELU2 = 4, EPI_SOFTCAP = 5,
           EPI_RELU2_BWD = 6, EPI_AXPBY = 7, EPI_QKV = 8, EPI_DOUT_D = 9 };

template <bool BF16> struct Mfma;

template <> struct Mfma<true> {
    using LT = bf16;
    static constexpr int BK = 64, KS = 16, LDK = BK + 8, CW = 8;
    using Frag = bf16x8;
    __device__ static Frag frag(const LT* p) { return *reinterpret_cast<const bf16x8*>(p); }
    __device__ static f32x16 mma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static int lane_k(int lane) { return (lane >> 5) * 8; }
};

template <> struct Mfma<false> {
    using LT = float;
    static constexpr int BK = 32, KS = 2, LDK = BK + 4, CW = 4;
    using Frag = float;
    __device__ static Frag frag(const LT* p) { return *p; }
    __device__ static f32x16 mma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __device__ static int lane_k(int lane) { return lane >> 5; }
};

// Row of accumulator element v (0..15) of a 32x32 MFMA tile held by `lane`;
// its column is lane % 32.
__device__ __forceinline__ int acc_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

// 4-wide fp32 <-> storage-type vector access (16 B fp32, 8 B bf16).
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4(const bf16* p) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}
__device__ __forceinline__ void st4(float* p, float4 x) { *reinterpret_cast<float4*>(p) = x; }
__device__ __forceinline__ void st4(bf16* p, float4 x) {
    bf16x4 v;
    v[0] = (bf16)x.x;
    v[1] = (bf16)x.y;
    v[2] = (bf16)x.z;
    v[3] = (bf16)x.w;
    *reinterpret_cast<bf16x4*>(p) = v;
}
// The same stores with the nontemporal hint (global_store ... nt): the
// persistent GEMM's output streams to memory instead of being allocated in
// L2, where it would evict the operand panels the next tiles read (measured:
// 8-12 % faster on the step's K = 512 / 2048 products).
__device__ __forceinline__ void st4nt(float* p, float4 x) {
    __builtin_nontemporal_store(x.x, p);
    __builtin_nontemporal_store(x.y, p + 1);
    __builtin_nontemporal_store(x.z, p + 2);
    __builtin_nontemporal_store(x.w, p + 3);
}
__device__ __forceinline__ void st4nt(bf16* p, float4 x) {
    bf16x4 v;
    v[0] = (bf16)x.x;
    v[1] = (bf16)x.y;
    v[2] = (bf16)x.z;
    v[3] = (bf16)x.w;
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned long long, v), reinterpret_cast<unsigned long long*>(p));
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
// cap * tanh(x / cap) from the hardware exp2 and reciprocal:
// tanh(y) = sign(y) (1 - 2 / (2^(2 |y| log2 e) + 1)), absolute error ~1e-7
// (times cap); |y| large gives 2^inf = inf and exactly +-1.  The scale
// 2 log2(e) / cap does not depend on x, so its division is hoisted out of the
// epilogue loops: per element there is no IEEE division sequence (~10 VALU).
__device__ __forceinline__ float softcap(float x, float cap) {
    const float e = __builtin_amdgcn_exp2f(fabsf(x) * (2.8853900817779268f / cap));  // 2^(2 log2(e) |x| / cap)
    const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    return copysignf(cap * t, x);
}
__device__ __forceinline__ float4 softcap4(float4 x, float cap) {
    return make_float4(softcap(x.x, cap), softcap(x.y, cap), softcap(x.z, cap), softcap(x.w, cap));
}
// d/dh relu(h)^2 times g, from the activation a = relu(h)^2: 2 sqrt(a) g (0 where a == 0).
// The hardware square root (1 ulp) instead of sqrtf's correctly rounded
// sequence (~15 VALU): a is a rounded activation, far coarser than 1 ulp.
__device__ __forceinline__ float relu2_grad(float a, float g) {
    return a > 0.f ? 2.f * __builtin_amdgcn_sqrtf(a) * g : 0.f;
}

template <typename T, int N>
__device__ __forceinline__ void vload(T (&dst)[N], const T* src) {
    constexpr int BYTES = N * (int)sizeof(T);
    static_assert(BYTES == 8 || BYTES == 16 || BYTES == 32, "vector width");
    if constexpr (BYTES == 8) {
        *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
    } else if constexpr (BYTES == 16) {
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    } else {
        reinterpret_cast<uint4*>(dst)[0] = reinterpret_cast<const uint4*>(src)[0];
        reinterpret_cast<uint4*>(dst)[1] = reinterpret_cast<const uint4*>(src)[1];
    }
}

template <typename T, int N>
__device__ __forceinline__ void vzero(T (&dst)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) dst[i] = T(0.0f);
}

// Global -> register -> LDS tile loader for one operand (ROWS x BK tile).
//   K-major (KMAJ): LDS [row][k], rows padded to ldk, one 16-byte chunk of
//     CW k-values per item.
//   MN-major, bf16 compute (TR): LDS holds the natural [k][row] tile (ROWS
//     bf16 per k, 16-byte chunks XOR-swizzled by tr_swz(k)); the MFMA
//     fragments are read with ds_read_b64_tr_b16 (tr_frag).
//   MN-major, fp32 compute: (k x 4-row) blocks transposed in registers into
//     the [row][k] layout.
__device__ __forceinline__ int tr_swz(int k) { return 4 * (k & 3); }

template <typename TG, typename LT, bool KMAJ, int ROWS, int BK, int CW, int kThreads>
struct TileLoader {
    static constexpr bool TR = !KMAJ && sizeof(LT) == 2;
    static constexpr int MW = 4;  // rows per MN-major item (fp32 compute)
    static constexpr int NPASS = KMAJ ? (ROWS * BK / CW) / kThreads
                                      : (TR ? (BK * ROWS / 8) / kThreads : ((BK / CW) * (ROWS / MW)) / kThreads);
    static_assert(NPASS >= 1, "tile too small for the block");
    static constexpr int PER = KMAJ ? CW : (TR ? 8 : CW * MW);  // TG values per pass
    TG v[NPASS][PER];

    // g: operand base; ld: row stride of the stored matrix; rows: extent of
    // the output dimension; K: reduction extent.
    __device__ __forceinline__ void load(const TG* g, int64_t ld, int64_t row0, int64_t rows, int64_t k0,
                                         int64_t kend) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < NPASS; ++p) {
            if constexpr (KMAJ) {
                const int c = p * kThreads + tid;
                const int r = c / (BK / CW), kc = (c % (BK / CW)) * CW;
                const int64_t gr = row0 + r, gk = k0 + kc;
                if (gr < rows && gk < kend) {
                    TG tmp[CW];
                    vload(tmp, g + gr * ld + gk);
#pragma unroll
                    for (int i = 0; i < CW; ++i) v[p][i] = tmp[i];
                } else {
                    vzero(v[p]);
                }
            } else if constexpr (TR) {
                const int item = p * kThreads + tid;
                const int k = item / (ROWS / 8), c = item % (ROWS / 8);
                const int lc = c ^ tr_swz(k);
                const int64_t gk = k0 + k, gr = row0 + lc * 8;
                if (gr < rows && gk < kend) vload(v[p], g + gk * ld + gr);
                else vzero(v[p]);
            } else {
                const int item = p * kThreads + tid;
                const int mg = item % (ROWS / MW), kg = item / (ROWS / MW);
                const int64_t gr = row0 + mg * MW;
#pragma unroll
                for (int j = 0; j < CW; ++j) {
                    const int64_t gk = k0 + kg * CW + j;
                    TG tmp[MW];
                    if (gr < rows && gk < kend) vload(tmp, g + gk * ld + gr);
                    else vzero(tmp);
#pragma unroll
                    for (int i = 0; i < MW; ++i) v[p][j * MW + i] = tmp[i];
                }
            }
        }
    }

    __device__ __forceinline__ void store(LT* lds, int ldk) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int p = 0; p < NPASS; ++p) {
            if constexpr (KMAJ) {
                const int c = p * kThreads + tid;
                const int r = c / (BK / CW), kc = (c % (BK / CW)) * CW;
                LT out[CW];
#pragma unroll
                for (int i = 0; i < CW; ++i) out[i] = (LT)to_f32(v[p][i]);
                *reinterpret_cast<uint4*>(lds + r * ldk + kc) = *reinterpret_cast<const uint4*>(out);
            } else if constexpr (TR) {
                const int item = p * kThreads + tid;
                LT out[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) out[i] = (LT)to_f32(v[p][i]);
                *reinterpret_cast<uint4*>(lds + item * 8) = *reinterpret_cast<const uint4*>(out);
            } else {
                const int item = p * kThreads + tid;
                const int mg = item % (ROWS / MW), kg = item / (ROWS / MW);
#pragma unroll
                for (int i = 0; i < MW; ++i) {
                    LT out[CW];
#pragma unroll
                    for (int j = 0; j < CW; ++j) out[j] = (LT)to_f32(v[p][j * MW + i]);
                    *reinterpret_cast<uint4*>(lds + (mg * MW + i) * ldk + kg * CW) =
                        *reinterpret_cast<const uint4*>(out);
                }
            }
        }
    }
    // LDS elements of one stage of this operand.
    static constexpr int elems(int ldk) { return TR ? BK * ROWS : ROWS * ldk; }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// MFMA fragment (32 rows from mn0, k-step ks) of a TR tile with ROWS bf16 per
// k: inside each 16-lane group, lane 4k+q supplies the address of k-row k,
// columns 4q..4q+3, and lane i receives k-rows 0..3 of column i; two reads
// give lane l the k-values 16 ks + 8 (l / 32) + 0..7 of column mn0 + l % 32.
template <int ROWS>
__device__ __forceinline__ bf16x8 tr_frag(const bf16* tile, int mn0, int ks, int lane) {
    const int g = lane >> 4, src = lane & 15;
    const int k = 16 * ks + 8 * (g >> 1) + (src >> 2);
    const int col = mn0 + 16 * (g & 1) + 4 * (src & 3);
    const int co = (((col >> 3) ^ tr_swz(k)) << 3) + (col & 7);  // k and k + 4 share tr_swz
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + k * ROWS + co));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + (k + 4) * ROWS + co));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Linear block id -> (batch, split, tile_m, tile_n) with an XCD-contiguous
// order: each of the 8 XCDs owns a contiguous run of (batch, split, m, n).
__device__ __forceinline__ void tile_coords(int64_t tiles_n, int64_t tiles_mn, int64_t splits, int64_t total,
                                            int64_t& bt, int64_t& tm, int64_t& tn, int64_t& z) {
    int64_t id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    bt = id / (tiles_mn * splits);
    id %= tiles_mn * splits;
    z = id / tiles_mn;
    const int64_t r = id % tiles_mn;
    tm = r / tiles_n;
    tn = r % tiles_n;
}

template <typename TA, typename TB, typename TC, bool AK, bool BKM, bool BF16, int EPI, typename TL>
__global__ __launch_bounds__(TL::THREADS) void gemm_k(TC* C, const TA* A, const TB* B, int64_t M, int64_t N,
                                                      int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                                      int64_t k_per_split, float* partial, int64_t batch,
                                                      int64_t sA, int64_t sB, int64_t sC, const void* aux,
                                                      void* aux_out, float cap, float beta) {
    using MM = Mfma<BF16>;
    using LT = typename MM::LT;
    constexpr int BM = TL::BM, BN = TL::BN, TM = TL::TM, TN = TL::TN;
    constexpr int BK = MM::BK, LDK = MM::LDK, CW = MM::CW;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    // Stage s occupies [s*STAGE, (s+1)*STAGE): the A tile then the B tile.
    // Stage addresses are formed by arithmetic on the __shared__ base (never
    // through a pointer array), so every access stays a ds_read / ds_write.
    LT* const lds = reinterpret_cast<LT*>(smem_raw);
    using LA = TileLoader<TA, LT, AK, BM, BK, CW, TL::THREADS>;
    using LB = TileLoader<TB, LT, BKM, BN, BK, CW, TL::THREADS>;
    constexpr int AEL = LA::elems(LDK), STAGE = AEL + LB::elems(LDK);

    const int64_t tiles_n = (N + BN - 1) / BN, tiles_m = (M + BM - 1) / BM;
    const int64_t tiles_mn = tiles_m * tiles_n;
    const int64_t splits = (K + k_per_split - 1) / k_per_split;
    int64_t bt, tm, tn, z;
    tile_coords(tiles_n, tiles_mn, splits, tiles_mn * splits * batch, bt, tm, tn, z);
    // STORE / AXPBY may run without C when only the bf16 copy aux_out is
    // wanted (the batched Muon products whose fp32 result nothing reads)
    const bool has_c = C != nullptr;
    A += bt * sA;
    B += bt * sB;
    if (has_c) C += bt * sC;
    if constexpr (EPI == EPI_PARTIAL) partial += bt * splits * M * N;
    const int64_t m0 = tm * BM, n0 = tn * BN;
    const int64_t kbeg = z * k_per_split;
    const int64_t kend = (kbeg + k_per_split < K) ? kbeg + k_per_split : K;

    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int wm = wave / TL::NWN, wn = wave % TL::NWN;

    LA la;
    LB lb;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    const int64_t nk = (kend - kbeg + BK - 1) / BK;
    if (nk > 0) {
        la.load(A, lda, m0, M, kbeg, kend);
        lb.load(B, ldb, n0, N, kbeg, kend);
        la.store(lds, LDK);
        lb.store(lds + AEL, LDK);
    }
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(A, lda, m0, M, kbeg + (kt + 1) * BK, kend);
            lb.load(B, ldb, n0, N, kbeg + (kt + 1) * BK, kend);
        }
        const LT* sa = lds + cur * STAGE;
        const LT* sb = sa + AEL;
        const LT* a_base = sa + (wm * TL::WM + (lane & 31)) * LDK + MM::lane_k(lane);
        const LT* b_base = sb + (wn * TL::WN + (lane & 31)) * LDK + MM::lane_k(lane);
#pragma unroll
        for (int ks = 0; ks < BK / MM::KS; ++ks) {
            typename MM::Frag fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if constexpr (LA::TR) fa[i] = tr_frag<BM>(sa, wm * TL::WM + i * 32, ks, lane);
                else fa[i] = MM::frag(a_base + i * 32 * LDK + ks * MM::KS);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if constexpr (LB::TR) fb[j] = tr_frag<BN>(sb, wn * TL::WN + j * 32, ks, lane);
                else fb[j] = MM::frag(b_base + j * 32 * LDK + ks * MM::KS);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = MM::mma(fa[i], fb[j], acc[i][j]);
        }
        if (more) {
            la.store(lds + (cur ^ 1) * STAGE, LDK);
            lb.store(lds + (cur ^ 1) * STAGE + AEL, LDK);
        }
        __syncthreads();
    }

    // Epilogue through LDS: each wave stages a 32 x WN strip of its tile
    // (fp32, row stride SLD) and writes it back as row-contiguous 4-wide
    // vectors, so every global access (C, aux, partials) is coalesced.
    constexpr int WN = TL::WN, SLD = WN + 8, VPR = WN / 4, RPI = kWave / VPR, NR = 32 / RPI;
    // Epilogues that read memory (C for ACCUM, aux for ADD / RELU2_BWD) load
    // a strip's vectors before staging it, so the loads overlap each other
    // and the LDS round trip instead of queueing behind the stores.
    constexpr bool PRE = EPI == EPI_ACCUM || EPI == EPI_ADD || EPI == EPI_RELU2_BWD || EPI == EPI_AXPBY;
    float* const strip = reinterpret_cast<float*>(smem_raw) + wave * 32 * SLD;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        float4 pre[PRE ? NR : 1];
        if constexpr (PRE) {
#pragma unroll
            for (int t = 0; t < NR; ++t) {
                const int r = t * RPI + lane / VPR, c4 = (lane % VPR) * 4;
                const int64_t row = m0 + wm * TL::WM + i * 32 + r, col = n0 + wn * WN + c4;
                const int64_t o = row * ldc + col;
                if (row < M && col < N) {
                    if constexpr (EPI == EPI_ACCUM) pre[t] = ld4(C + o);
                    else if constexpr (EPI == EPI_ADD) pre[t] = ld4(static_cast<const float*>(aux) + o);
                    else if constexpr (EPI == EPI_AXPBY) pre[t] = ld4(static_cast<const float*>(aux) + bt * sC + o);
                    else pre[t] = ld4(static_cast<const TC*>(aux) + o);
                } else {
                    pre[t] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) strip[acc_row(v, lane) * SLD + j * 32 + (lane & 31)] = acc[i][j][v];
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NR; ++t) {
            const int r = t * RPI + lane / VPR, c4 = (lane % VPR) * 4;
            const int64_t row = m0 + wm * TL::WM + i * 32 + r, col = n0 + wn * WN + c4;
            if (row >= M || col >= N) continue;  // N % 4 == 0: col < N covers col + 3
            const float4 x = *reinterpret_cast<const float4*>(strip + r * SLD + c4);
            const int64_t o = row * ldc + col;
            if constexpr (EPI == EPI_PARTIAL) {
                *reinterpret_cast<float4*>(partial + (z * M + row) * N + col) = x;
            } else if constexpr (EPI == EPI_STORE) {
                if (has_c) st4(C + o, x);
                if (aux_out) st4(static_cast<bf16*>(aux_out) + bt * sC + o, x);  // bf16 copy (batched Muon)
            } else if constexpr (EPI == EPI_ACCUM || EPI == EPI_ADD) {
                st4(C + o, add4(pre[PRE ? t : 0], x));
            } else if constexpr (EPI == EPI_RELU2) {
                st4(C + o, make_float4(x.x > 0.f ? x.x * x.x : 0.f, x.y > 0.f ? x.y * x.y : 0.f,
                                       x.z > 0.f ? x.z * x.z : 0.f, x.w > 0.f ? x.w * x.w : 0.f));
            } else if constexpr (EPI == EPI_SOFTCAP) {
                st4(C + o, softcap4(x, cap));
            } else if constexpr (EPI == EPI_RELU2_BWD) {
                const float4 a = pre[PRE ? t : 0];
                st4(C + o, make_float4(relu2_grad(a.x, x.x), relu2_grad(a.y, x.y), relu2_grad(a.z, x.z),
                                       relu2_grad(a.w, x.w)));
            } else if constexpr (EPI == EPI_AXPBY) {
                const float4 y = pre[PRE ? t : 0];
                const float4 r = make_float4(cap * x.x + beta * y.x, cap * x.y + beta * y.y, cap * x.z + beta * y.z,
                                             cap * x.w + beta * y.w);
                if (has_c) st4(C + o, r);
                if (aux_out) st4(static_cast<bf16*>(aux_out) + bt * sC + o, r);  // bf16 copy (batched Muon)
            }
        }
        __syncthreads();
    }
}

// C[b][i] (+)= sum_z partial[b][z][i], z in order (row stride ldc for C).
template <typename TC>
__global__ void splitk_reduce_k(TC* C, const float* partial, int64_t M, int64_t N, int64_t ldc, int64_t splits,
                                int accumulate, int64_t batch, int64_t sC) {
    const int64_t mn = M * N;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < mn * batch;
         j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = j / mn, i = j % mn;
        const int64_t r = i / N, c = i % N;
        TC* Cb = C + b * sC;
        const float* pb = partial + b * splits * mn;
        float s = accumulate ? to_f32(Cb[r * ldc + c]) : 0.f;
        for (int64_t z = 0; z < splits; ++z) s += pb[z * mn + i];
        Cb[r * ldc + c] = from_f32<TC>(s);
    }
}

// ---------------------------------------------------------------------
// Persistent GEMM for bf16 operands in memory (the bf16 training step).
//
// One 512-thread workgroup per CU walks a strided list of 256x256 output
// tiles (x reduction splits).  Every k-tile (BK = 64) of A and B goes from
// global memory straight into LDS with 16-byte global_load_lds (no VGPR
// staging, no ds_write), two stages deep; the stream of k-tiles runs on
// across tile boundaries, so the next tile's first loads are in flight while
// the current tile's epilogue drains.  8 waves of 128 x 64 as in gemm_k.
//   K-major operand tile: 256 rows x 8 16-byte units, unit c of row r at
//     slot r*8 + (c ^ ((r >> 1) & 7)): each 16-lane phase of a fragment read
//     (rows r0..r0+15, one unit) covers all 64 banks once.
//   MN-major operand tile: 64 k-rows x 32 units, unit c of k-row k at slot
//     k*32 + (c ^ tr_swz(k)), read with tr_frag as in gemm_k.
// A lane's DMA slot is fixed (wave-instruction j of wave w fills slots
// (8j + w)*64 + lane), so the swizzle is applied to the global address the
// lane fetches: a per-lane 32-bit offset fixed for the whole kernel, added to
// a wave-uniform (SGPR) base that moves by one k-tile per copy and is set
// once per tile, so a copy costs a few scalar instructions.  The epilogue stages 16-row half strips (fp32) in a separate
// 32 KB region.  Shapes: M, N % 256, K (per split) % 64, lda/ldb % 8.
constexpr int kPkThreads = 512, kPkBK = 64, kPkStage = 2 * 256 * kPkBK * 2;  // bytes per stage (A + B)
constexpr int kPkLds = 2 * kPkStage + 8 * 16 * 64 * 4;                      // 160 KB

template <int N>
__device__ __forceinline__ void vm_wait() {
    // vmcnt(N) (6 bits: [3:0] and [15:14] of the encoding); expcnt / lgkmcnt not waited
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Per-lane byte offsets of the 4 DMA wave-instructions that fill one operand
// tile, relative to the tile's first element (row0, k0): slot (8j + w)*64 +
// lane of wave w, swizzled as the tile layout above says.  Constant for the
// whole kernel; the tile position goes into a wave-uniform base address.
template <bool KMAJ>
__device__ __forceinline__ void pk_offsets(unsigned (&off)[4], int ld, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int slot = (j * 8 + wave) * 64 + lane;
        if constexpr (KMAJ) {
            const int r = slot >> 3, c = (slot & 7) ^ ((r >> 1) & 7);
            off[j] = (unsigned)(r * ld + c * 8) * 2u;
        } else {
            const int k = slot >> 5, c = (slot & 31) ^ tr_swz(k);
            off[j] = (unsigned)(k * ld + c * 8) * 2u;
        }
    }
}

// Work item -> (split z, tile_m, tile_n); each XCD (workgroups are dispatched
// round-robin over 8) owns a contiguous run of items.
__device__ __forceinline__ void pk_item(int lin, int items, int tiles_n, int tiles_mn, int& z, int& tm, int& tn) {
    int id = lin;
    if (items % 8 == 0 && gridDim.x % 8 == 0) id = (lin % 8) * (items / 8) + lin / 8;
    z = id / tiles_mn;
    const int r = id - z * tiles_mn;
    tm = r / tiles_n;
    tn = r - tm * tiles_n;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Operands of the head-aligned epilogues (EPI_QKV, EPI_DOUT_D).
struct PkHead {
    bf16 *q, *k, *v;               // QKV: outputs, [M, cpart] bf16 each
    const float *cos_t, *sin_t;    // QKV: rope tables [period, HD / 2]
    int64_t period;                // QKV: table row = row % period
    const float* gate;             // QKV: [M, H] value-embedding gate (null: none)
    const float* table;            // QKV: value-embedding table [V, cpart]
    const int64_t* idx;            // QKV: token ids [M]
    const float* o;                // DOUT_D: attention output O, fp32 [M, N]
    float* d;                      // DOUT_D: D, [M, N / HD]
    int64_t cpart;                 // QKV: columns per part (C); a part starts on a 256-column tile
};

// HLD = 0: 8 waves of 128 x 64.  HLD = head_dim (32 / 64 / 128): 8 waves of
// 64 x 128 (4 x 2), so each wave's 128 output columns hold whole heads, for
// the head-wise epilogues.
template <bool AK, bool BKM, typename TC, int EPI, int HLD = 0>
__global__ __launch_bounds__(kPkThreads) void gemm_pk(TC* C, const bf16* A, const bf16* B, int64_t M, int64_t N,
                                                     int64_t lda, int64_t ldb, int64_t ldc, int64_t kps,
                                                     int64_t splits, float* partial, const void* aux, void* aux_out,
                                                     float cap, PkHead hx) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    constexpr int OPB = kPkStage / 2;
    constexpr bool HL = HLD > 0;
    constexpr int WTM = HL ? 2 : 4, WTN = HL ? 4 : 2;  // 32 x 32 MFMA blocks per wave (rows, columns)
    static_assert(!HL || (128 % HLD == 0 && HLD >= 32), "head-aligned waves hold whole heads");
    static_assert(HL == (EPI == EPI_QKV || EPI == EPI_DOUT_D), "head epilogues run on head-aligned waves");
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int wm = HL ? wave >> 1 : wave >> 2, wn = HL ? wave & 1 : wave & 3;
    const int wrow = wm * 32 * WTM, wcol = wn * 32 * WTN;  // the wave's block within the 256 x 256 tile
    // bf16 outputs whose epilogue is element-wise on the product alone: the
    // MFMA operands are swapped so that each accumulator holds a transposed
    // 32 x 32 block (lane l: row l % 32, four consecutive columns per group of
    // four values), and the epilogue stages bf16 instead of fp32 (see below)
    constexpr bool SW = std::is_same<TC, bf16>::value && (EPI == EPI_STORE || EPI == EPI_RELU2 || EPI == EPI_SOFTCAP ||
                                                          EPI == EPI_QKV || EPI == EPI_DOUT_D);
    const int tiles_n = (int)(N / 256), tiles_mn = (int)(M / 256) * tiles_n, items = tiles_mn * (int)splits;
    const int grid = (int)gridDim.x, b = (int)blockIdx.x;
    const int nk = (int)(kps / kPkBK);
    const int nmine = (items - b + grid - 1) / grid;
    const int G = nmine * nk;  // k-tiles this workgroup streams

    // DMA cursor: local item `di`, its k-tile `dkt`, and the byte addresses of
    // that k-tile's first A / B elements (wave-uniform, advanced per k-tile)
    unsigned aoffs[4], boffs[4];
    pk_offsets<AK>(aoffs, (int)lda, wave, lane);
    pk_offsets<BKM>(boffs, (int)ldb, wave, lane);
    const int64_t astep = AK ? 2 * kPkBK : 2 * kPkBK * lda, bstep = BKM ? 2 * kPkBK : 2 * kPkBK * ldb;
    const unsigned lds0 = lds_addr(smem_raw) + wave * 1024;
    int di = 0, dkt = 0;
    const char* pa = reinterpret_cast<const char*>(A);
    const char* pb = reinterpret_cast<const char*>(B);
    auto issue = [&](int g) {
        if (dkt == 0) {
            int z, tm, tn;
            pk_item(di * grid + b, items, tiles_n, tiles_mn, z, tm, tn);
            const int64_t k0 = (int64_t)z * kps;
            pa = reinterpret_cast<const char*>(A) + 2 * (AK ? (int64_t)tm * 256 * lda + k0 : k0 * lda + tm * 256);
            pb = reinterpret_cast<const char*>(B) + 2 * (BKM ? (int64_t)tn * 256 * ldb + k0 : k0 * ldb + tn * 256);
        }
        const unsigned st = lds0 + (g & 1) * kPkStage;
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16s(pa, aoffs[j], st + j * 8192);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16s(pb, boffs[j], st + OPB + j * 8192);
        pa += astep;
        pb += bstep;
        if (++dkt == nk) {
            dkt = 0;
            ++di;
        }
    };

    // K-major fragment byte offsets per k-step (row swizzle depends on the lane only)
    const int r32 = lane & 31, hi = lane >> 5;
    int aoff[4], boff[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int ra = wrow + r32, rb = wcol + r32;
        aoff[ks] = (ra * 8 + ((2 * ks + hi) ^ ((ra >> 1) & 7))) * 16;
        boff[ks] = (rb * 8 + ((2 * ks + hi) ^ ((rb >> 1) & 7))) * 16;
    }

    f32x16 acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    if (G > 0) issue(0);
    float* const strip = reinterpret_cast<float*>(smem_raw + 2 * kPkStage) + wave * 16 * 64;
    // epilogue lane offsets: lane (lane/16, lane%16) owns row t*4 + lane/16, columns 4*(lane%16)..+3
    const int lrow = lane >> 4, lcol = (lane & 15) * 4;
    int ckt = 0, ci = 0;  // compute cursor: k-tile within the current item, local item

    for (int g = 0; g < G; ++g) {
        // vmcnt(0): this wave's DMA of k-tile g (and anything older) has
        // landed; the barrier then publishes every wave's part and retires
        // all reads of the stage that the next DMA overwrites.
        vm_wait<0>();
        __builtin_amdgcn_s_barrier();
        if (g + 1 < G) issue(g + 1);
        const unsigned char* sa = smem_raw + (g & 1) * kPkStage;
        const unsigned char* sb = sa + OPB;
        auto frags = [&](int ks, bf16x8 (&fa)[WTM], bf16x8 (&fb)[WTN]) {
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                if constexpr (AK) fa[i] = *reinterpret_cast<const bf16x8*>(sa + aoff[ks] + i * 4096);
                else fa[i] = tr_frag<256>(reinterpret_cast<const bf16*>(sa), wrow + i * 32, ks, lane);
            }
#pragma unroll
            for (int j = 0; j < WTN; ++j) {
                if constexpr (BKM) fb[j] = *reinterpret_cast<const bf16x8*>(sb + boff[ks] + j * 4096);
                else fb[j] = tr_frag<256>(reinterpret_cast<const bf16*>(sb), wcol + j * 32, ks, lane);
            }
        };
        bf16x8 fa[2][WTM], fb[2][WTN];
        frags(0, fa[0], fb[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks < 3) frags(ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
            // keep the next k-step's fragment reads ahead of this k-step's
            // MFMAs: left alone, the scheduler sinks each read to just before
            // its first use and waits for it there (lgkmcnt(0) inside every
            // k-step), to save the second fragment set's registers
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j)
                    acc[i][j] = SW ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks & 1][j], fa[ks & 1][i], acc[i][j], 0, 0, 0)
                                   : __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ks & 1][i], fb[ks & 1][j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (++ckt != nk) continue;
        ckt = 0;
        const int it = ci++;

        // Epilogue of item `it`: per 32-row MFMA block i, two 16-row half
        // strips; lane (t, lane/16, lane%16) owns 4 consecutive columns.
        int z, tm, tn;
        pk_item(it * grid + b, items, tiles_n, tiles_mn, z, tm, tn);
        const int64_t row0 = (int64_t)tm * 256 + wrow, col0 = (int64_t)tn * 256 + wcol;
        // this wave's block: element (r, c) at base + r * ld + c
        const int64_t cbase = row0 * ldc + col0;
        const int clo = lrow * (int)ldc + lcol;
        if constexpr (SW) {
            // Per 32-row block i: the lane's 32 values (row m = lane % 32,
            // columns j * 32 + 8 g + 4 (lane / 32) + 0..3) go through the
            // element-wise op in fp32, are rounded to bf16 and written as 8-byte
            // pieces into a wave-private 32 x 64 bf16 strip; each lane then
            // reads 16 bytes (8 columns of one row) and stores them, 8 rows of
            // 128 bytes per store instruction.  Strip layout: row m at m * 128
            // bytes, logical 8-byte piece c (columns 4c..4c+3) in slot
            // ((c / 2) ^ (m % 8)) * 2 + ((c % 2) ^ (m / 8 % 2)): 16 rows of one
            // piece land in 16 different slots, and a 16-byte pair stays
            // adjacent (its halves swapped on rows with m / 8 odd).
            unsigned char* const bstrip = smem_raw + 2 * kPkStage + wave * 4096;
            const int m = lane & 31, hh = lane >> 5;
            const int rr = lane >> 3, c16 = lane & 7;
            // output rows: C, or for QKV the part (q / k / v) buffer this
            // tile's columns fall in (row stride cpart)
            TC* obase = C + cbase;
            int64_t ldo = ldc;
            int part = 0;
            int64_t pcol = col0;  // QKV: first column of the wave within its part
            if constexpr (EPI == EPI_QKV) {
                part = (int)(col0 / hx.cpart);
                pcol = col0 - (int64_t)part * hx.cpart;
                obase = (part == 0 ? hx.q : part == 1 ? hx.k : hx.v) + row0 * hx.cpart + pcol;
                ldo = hx.cpart;
            }
            TC* const lbase = obase + (int64_t)rr * ldo + c16 * 8;
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                if constexpr (HL) {
                    // the lane's values of row row0 + 32 i + m: column group cg = 4 j + g4
                    // (columns 8 cg + 4 hh + 0..3 of the wave's 128), acc[i][cg / 4][(cg % 4) * 4 + e]
                    const int64_t row = row0 + i * 32 + m;
                    constexpr int NH = 128 / HLD, HALF = HLD / 2;
                    if constexpr (EPI == EPI_QKV) {
                        if (part < 2) {
                            // rope_fwd: (x1, x2) -> (x1 c + x2 s, -x1 s + x2 c) on the head's
                            // halves (column d and d + HD/2: groups cg and cg + HALF / 8, same
                            // lane), then the head's RMSNorm over its HD values (half in the
                            // partner lane hh ^ 1)
                            const int64_t tok = row % hx.period;
                            const float* ct = hx.cos_t + tok * HALF;
                            const float* sn = hx.sin_t + tok * HALF;
                            float ss[NH];
#pragma unroll
                            for (int h = 0; h < NH; ++h) ss[h] = 0.f;
#pragma unroll
                            for (int cg = 0; cg < 16; ++cg) {
                                constexpr int GPH = HLD / 8;  // column groups per head
                                if ((cg % GPH) * 8 >= HALF) continue;
                                const int cgp = cg + HALF / 8, d = (cg % GPH) * 8 + 4 * hh;
                                const float4 cv = *reinterpret_cast<const float4*>(ct + d);
                                const float4 sv = *reinterpret_cast<const float4*>(sn + d);
                                const float cc[4] = {cv.x, cv.y, cv.z, cv.w}, sc[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    const float x1 = acc[i][cg / 4][(cg % 4) * 4 + e];
                                    const float x2 = acc[i][cgp / 4][(cgp % 4) * 4 + e];
                                    const float y1 = x1 * cc[e] + x2 * sc[e];
                                    const float y2 = x1 * (-sc[e]) + x2 * cc[e];
                                    acc[i][cg / 4][(cg % 4) * 4 + e] = y1;
                                    acc[i][cgp / 4][(cgp % 4) * 4 + e] = y2;
                                    ss[cg / GPH] += y1 * y1 + y2 * y2;
                                }
                            }
                            float inv[NH];
#pragma unroll
                            for (int h = 0; h < NH; ++h) {
                                const float t = ss[h] + __shfl_xor(ss[h], 32, kWave);
                                inv[h] = 1.0f / sqrtf(t / (float)HLD + 1e-5f);  // ops.mojo:61-104 eps
                            }
#pragma unroll
                            for (int cg = 0; cg < 16; ++cg)
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[i][cg / 4][(cg % 4) * 4 + e] *= inv[cg / (HLD / 8)];
                        } else if (hx.gate) {
                            // v + gate[row, head] * value_embeds[idx[row]] (ve_apply_fwd)
                            const int64_t H = hx.cpart / HLD;
                            const float* ve = hx.table + hx.idx[row] * hx.cpart + pcol;
                            float g[NH];
#pragma unroll
                            for (int h = 0; h < NH; ++h) g[h] = hx.gate[row * H + pcol / HLD + h];
#pragma unroll
                            for (int cg = 0; cg < 16; ++cg) {
                                const float4 e4 = *reinterpret_cast<const float4*>(ve + cg * 8 + 4 * hh);
                                const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                                for (int e = 0; e < 4; ++e)
                                    acc[i][cg / 4][(cg % 4) * 4 + e] += g[cg / (HLD / 8)] * ev[e];
                            }
                        }
                    } else if constexpr (EPI == EPI_DOUT_D) {
                        // D[row, head] = sum over the head's columns of bf16(dO) * O
                        const float* orow = hx.o + row * ldc + col0;
                        float ds[NH];
#pragma unroll
                        for (int h = 0; h < NH; ++h) ds[h] = 0.f;
#pragma unroll
                        for (int cg = 0; cg < 16; ++cg) {
                            const float4 o4 = *reinterpret_cast<const float4*>(orow + cg * 8 + 4 * hh);
                            const float ov[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                ds[cg / (HLD / 8)] += (float)(bf16)acc[i][cg / 4][(cg % 4) * 4 + e] * ov[e];
                        }
                        const int64_t H = N / HLD;
#pragma unroll
                        for (int h = 0; h < NH; ++h) {
                            const float t = ds[h] + __shfl_xor(ds[h], 32, kWave);
                            if (hh == 0) hx.d[row * H + col0 / HLD + h] = t;
                        }
                    }
                }
#pragma unroll
                for (int jp = 0; jp < WTN / 2; ++jp) {
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                        for (int g4 = 0; g4 < 4; ++g4) {
                            const int j = 2 * jp + jj;
                            float4 x = make_float4(acc[i][j][g4 * 4], acc[i][j][g4 * 4 + 1], acc[i][j][g4 * 4 + 2],
                                                   acc[i][j][g4 * 4 + 3]);
                            if constexpr (EPI == EPI_RELU2)
                                x = make_float4(x.x > 0.f ? x.x * x.x : 0.f, x.y > 0.f ? x.y * x.y : 0.f,
                                                x.z > 0.f ? x.z * x.z : 0.f, x.w > 0.f ? x.w * x.w : 0.f);
                            else if constexpr (EPI == EPI_SOFTCAP)
                                x = softcap4(x, cap);
                            bf16x4 v;
                            v[0] = (bf16)x.x;
                            v[1] = (bf16)x.y;
                            v[2] = (bf16)x.z;
                            v[3] = (bf16)x.w;
                            const int c = jj * 8 + g4 * 2 + hh;
                            const int slot = (((c >> 1) ^ (m & 7)) << 1) + ((c & 1) ^ ((m >> 3) & 1));
                            *reinterpret_cast<bf16x4*>(bstrip + m * 128 + slot * 8) = v;
                        }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const int r = p * 8 + rr;
                        u32x4 q = *reinterpret_cast<const u32x4*>(bstrip + r * 128 + ((c16 ^ (r & 7)) << 4));
                        if (p & 1) q = __builtin_shufflevector(q, q, 2, 3, 0, 1);  // r / 8 odd
                        u32x4* const qd = reinterpret_cast<u32x4*>(lbase + (int64_t)(i * 32 + p * 8) * ldo + jp * 64);
                        // q, k, v are plain stores: the attention kernels read each k / v
                        // row many times, so keeping them in the caches pays; other
                        // outputs stream past L2 (nontemporal)
                        if constexpr (EPI == EPI_QKV) *qd = q;
                        else __builtin_nontemporal_store(q, qd);
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
#pragma unroll
                for (int j = 0; j < WTN; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
            }
            continue;
        }
        if constexpr (!HL) {
        constexpr bool PRE = EPI == EPI_ACCUM || EPI == EPI_ADD || EPI == EPI_RELU2_BWD;
        // The operand the epilogue combines with (C, the residual or the
        // pre-activation) is loaded one half strip ahead, into a two-slot
        // register ring, so its latency hides behind the previous strip.
        float4 pre[2][PRE ? 4 : 1];
        auto load_pre = [&](int s, float4 (&dst)[PRE ? 4 : 1]) {
            if constexpr (PRE) {
                const int64_t rb = cbase + (int64_t)(s * 16) * ldc;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int64_t o = rb + (int64_t)(t * 4) * ldc + clo;
                    if constexpr (EPI == EPI_ACCUM) dst[t] = ld4(C + o);
                    else if constexpr (EPI == EPI_ADD) dst[t] = ld4(static_cast<const float*>(aux) + o);
                    else dst[t] = ld4(static_cast<const TC*>(aux) + o);
                }
            }
        };
        load_pre(0, pre[0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int s = i * 2 + h;
                const int64_t rb = cbase + (int64_t)(s * 16) * ldc;
                if (s + 1 < 8) load_pre(s + 1, pre[(s + 1) & 1]);
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int vv = 0; vv < 8; ++vv) {
                        const int v = h * 8 + vv;
                        const int r = acc_row(v, lane) - 16 * h;
                        strip[r * 64 + ((j * 32 + r32) ^ (((r >> 2) & 1) << 5))] = acc[i][j][v];
                    }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int r = t * 4 + lrow;
                    const float4 x = *reinterpret_cast<const float4*>(strip + r * 64 + (lcol ^ (((r >> 2) & 1) << 5)));
                    const int64_t o = rb + (int64_t)(t * 4) * ldc + clo;
                    if constexpr (EPI == EPI_PARTIAL) {
                        const int64_t row = row0 + i * 32 + h * 16 + r;
                        st4nt(partial + ((int64_t)z * M + row) * N + col0 + lcol, x);
                    } else if constexpr (EPI == EPI_STORE) {
                        st4nt(C + o, x);
                    } else if constexpr (EPI == EPI_ACCUM || EPI == EPI_ADD) {
                        st4nt(C + o, add4(pre[s & 1][PRE ? t : 0], x));
                    } else if constexpr (EPI == EPI_RELU2) {
                        st4nt(C + o, make_float4(x.x > 0.f ? x.x * x.x : 0.f, x.y > 0.f ? x.y * x.y : 0.f,
                                               x.z > 0.f ? x.z * x.z : 0.f, x.w > 0.f ? x.w * x.w : 0.f));
                    } else if constexpr (EPI == EPI_SOFTCAP) {
                        st4nt(C + o, softcap4(x, cap));
                    } else if constexpr (EPI == EPI_RELU2_BWD) {
                        const float4 a = pre[s & 1][PRE ? t : 0];
                        st4nt(C + o, make_float4(relu2_grad(a.x, x.x), relu2_grad(a.y, x.y), relu2_grad(a.z, x.z),
                                               relu2_grad(a.w, x.w)));
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
        }
        }  // !HL
    }
}

// ---- row-complete persistent GEMM (512 output columns per row) ----
// The forward's residual products whose output rows feed an RMSNorm (c_proj
// and mlp_proj at C = 512): one 512-thread workgroup per CU walks 128-row
// items, each the whole 128 x 512 output block, so the epilogue holds complete
// rows and runs the row pass of resid_norm (ar_fused.hip) itself:
//   x = r + acc (the residual add), or for the next layer's input
//   x = sa[l] (r + acc) + sb[l] x0 (scaled_add_fwd, ops.mojo:579-594);
//   x (fp32), rms = sqrt(mean(x^2) + 1e-5) (ops.mojo:61-104), xn = bf16(x / rms),
//   and on value-embedding layers xg = (x / rms)[:, :32] (fp32) and
//   gate[h] = 2 sigmoid(sum_c w[h, c] xg[c]) (ve_gate_fwd, ops.mojo:516-541).
// Same data movement as gemm_pk (direct-to-LDS copies, two stages, the stream
// of k-tiles running across items): A tile 128 x 64, B tile 512 x 64 (80 KB
// per stage).  8 waves of 64 x 128 (2 x 4) with transposed accumulators (lane:
// one row, four consecutive columns per group), so a row's sum of squares is a
// lane sum, one exchange with lane ^ 32 and a four-wave sum through LDS (the
// stage the item's last k-tile used) in a fixed order.
constexpr int kRcBM = 128, kRcN = 512;
constexpr int kRcOpA = kRcBM * kPkBK * 2, kRcOpB = kRcN * kPkBK * 2, kRcStage = kRcOpA + kRcOpB;
constexpr int kRcLds = 2 * kRcStage;  // 160 KB

struct RcArgs {
    const float* r;       // residual, fp32 [M, 512] (may alias x_out)
    float* x_out;         // fp32 [M, 512]
    float* rms_out;       // [M]
    bf16* xn_out;         // bf16 [M, 512]
    const float* x0;      // scaled form: x0 [M, 512]
    const float* sa;      // scaled form: sa[layer], sb[layer]
    const float* sb;
    int64_t layer;
    float* xg_out;        // value-embedding gate (gate_out null: none): xg [M, 32]
    float* gate_out;      // gate [M, nkv]
    const float* gate_w;  // [nkv, 32]
    int nkv;
};

template <bool SCALED>
__global__ __launch_bounds__(kPkThreads) void gemm_rc(const bf16* A, const bf16* B, int64_t M, int64_t K, int64_t lda,
                                                     int64_t ldb, RcArgs ra) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int wm = wave >> 2, wn = wave & 3;
    const int items = (int)(M / kRcBM);
    const int grid = (int)gridDim.x, b = (int)blockIdx.x;
    const int nk = (int)(K / kPkBK);
    const int nmine = (items - b + grid - 1) / grid;
    const int G = nmine * nk;

    // copies: slot j * 512 + wave * 64 + lane of a tile (A: j < 2, B: j < 8),
    // K-major layout (unit c of row r at r * 8 + (c ^ ((r >> 1) & 7)))
    unsigned aoffs[2], boffs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int slot = j * kPkThreads + wave * 64 + lane;
        const int r = slot >> 3, c = (slot & 7) ^ ((r >> 1) & 7);
        if (j < 2) aoffs[j] = (unsigned)(r * lda + c * 8) * 2u;
        boffs[j] = (unsigned)(r * ldb + c * 8) * 2u;
    }
    const unsigned lds0 = lds_addr(smem_raw) + wave * 1024;
    int di = 0, dkt = 0;
    const char* pa = reinterpret_cast<const char*>(A);
    const char* pb = reinterpret_cast<const char*>(B);
    auto issue = [&](int g) {
        if (dkt == 0) {
            pa = reinterpret_cast<const char*>(A) + 2 * (int64_t)(di * grid + b) * kRcBM * lda;
            pb = reinterpret_cast<const char*>(B);
        }
        const unsigned st = lds0 + (g & 1) * kRcStage;
#pragma unroll
        for (int j = 0; j < 2; ++j) dma16s(pa, aoffs[j], st + j * 8192);
#pragma unroll
        for (int j = 0; j < 8; ++j) dma16s(pb, boffs[j], st + kRcOpA + j * 8192);
        pa += 2 * kPkBK;
        pb += 2 * kPkBK;
        if (++dkt == nk) {
            dkt = 0;
            ++di;
        }
    };

    const int r32 = lane & 31, hi = lane >> 5;
    int aoff[4], boff[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int rA = wm * 64 + r32, rB = wn * 128 + r32;
        aoff[ks] = (rA * 8 + ((2 * ks + hi) ^ ((rA >> 1) & 7))) * 16;
        boff[ks] = (rB * 8 + ((2 * ks + hi) ^ ((rB >> 1) & 7))) * 16;
    }
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    float sa = 0.f, sb = 0.f;
    if constexpr (SCALED) {
        sa = ra.sa[ra.layer];
        sb = ra.sb[ra.layer];
    }

    if (G > 0) issue(0);
    int ckt = 0, ci = 0;
    for (int g = 0; g < G; ++g) {
        vm_wait<0>();
        __builtin_amdgcn_s_barrier();
        if (g + 1 < G) issue(g + 1);
        const unsigned char* sa_ = smem_raw + (g & 1) * kRcStage;
        const unsigned char* sb_ = sa_ + kRcOpA;
        auto frags = [&](int ks, bf16x8 (&fa)[2], bf16x8 (&fb)[4]) {
#pragma unroll
            for (int i = 0; i < 2; ++i) fa[i] = *reinterpret_cast<const bf16x8*>(sa_ + aoff[ks] + i * 4096);
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const bf16x8*>(sb_ + boff[ks] + j * 4096);
        };
        bf16x8 fa[2][2], fb[2][4];
        frags(0, fa[0], fb[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks < 3) frags(ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);  // next k-step's reads ahead of these MFMAs (as in gemm_pk)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks & 1][j], fa[ks & 1][i], acc[i][j], 0, 0,
                                                                         0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (++ckt != nk) continue;
        ckt = 0;
        const int it = ci++;

        // Epilogue.  Lane (m, hh): row row0 + 32 i + m, columns 128 wn +
        // 8 cg + 4 hh + 0..3 (cg = 4 j + g4) = acc[i][j][4 g4 + 0..3].
        __syncthreads();  // every wave is done with stage g & 1: it holds the row sums
        float* const red = reinterpret_cast<float*>(smem_raw + (g & 1) * kRcStage);  // [wm][i][wn][32]
        const int m = lane & 31, hh = lane >> 5;
        const int64_t row0 = ((int64_t)it * grid + b) * kRcBM + wm * 64;  // local item it is item it * grid + b
        const int col0 = wn * 128 + 4 * hh;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t row = row0 + i * 32 + m;
            const float* rrow = ra.r + row * kRcN + col0;
            const float* xrow = SCALED ? ra.x0 + row * kRcN + col0 : nullptr;
            float p = 0.f;
#pragma unroll
            for (int cg = 0; cg < 16; ++cg) {
                const float4 r4 = *reinterpret_cast<const float4*>(rrow + cg * 8);
                const float rv[4] = {r4.x, r4.y, r4.z, r4.w};
                float xv[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (SCALED) {
                    const float4 x4 = *reinterpret_cast<const float4*>(xrow + cg * 8);
                    xv[0] = x4.x;
                    xv[1] = x4.y;
                    xv[2] = x4.z;
                    xv[3] = x4.w;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = rv[e] + acc[i][cg / 4][(cg % 4) * 4 + e];
                    if constexpr (SCALED) v = sa * v + sb * xv[e];
                    acc[i][cg / 4][(cg % 4) * 4 + e] = v;
                    p += v * v;
                }
            }
            p += __shfl_xor(p, 32, kWave);
            if (hh == 0) red[((wm * 2 + i) * 4 + wn) * 32 + m] = p;
        }
        __syncthreads();
        // Outputs through a wave-private strip (32 rows x 64 columns, fp32) in
        // the same stage, read back row-contiguous (lane: row 4 t + lane / 16,
        // columns 4 (lane % 16)), so that x and xn go out as whole row segments.
        constexpr int SLD = 68;
        float* const strip = reinterpret_cast<float*>(smem_raw + (g & 1) * kRcStage + 2048) + wave * 32 * SLD;
        auto row_rms = [&](int i, int rl) {
            const float* rp = red + (wm * 2 + i) * 4 * 32 + rl;
            const float ss = ((rp[0] + rp[32]) + rp[64]) + rp[96];
            return sqrtf(ss / (float)kRcN + 1e-5f);
        };
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t rowb = row0 + i * 32;
            if (wn == 0 && lane < 32) ra.rms_out[rowb + lane] = row_rms(i, lane);
#pragma unroll
            for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
                for (int cg = 0; cg < 8; ++cg) {
                    const int j = (pass * 8 + cg) / 4, v0 = ((pass * 8 + cg) % 4) * 4;
                    *reinterpret_cast<float4*>(strip + m * SLD + cg * 8 + 4 * hh) =
                        make_float4(acc[i][j][v0], acc[i][j][v0 + 1], acc[i][j][v0 + 2], acc[i][j][v0 + 3]);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int rl = t * 4 + (lane >> 4), c4 = (lane & 15) * 4;
                    const float4 x4 = *reinterpret_cast<const float4*>(strip + rl * SLD + c4);
                    const float rms = row_rms(i, rl);
                    const int64_t o = (rowb + rl) * kRcN + wn * 128 + pass * 64 + c4;
                    st4nt(ra.x_out + o, x4);
                    st4nt(ra.xn_out + o, make_float4(x4.x / rms, x4.y / rms, x4.z / rms, x4.w / rms));
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            if (ra.gate_out && wn == 0) {
                // channels 0..31: groups cg 0..3 of the wn = 0 waves (this lane:
                // 8 cg + 4 hh + 0..3), the rest in lane ^ 32; the normalised
                // values in fp32
                const int64_t row = rowb + m;
                const float rms = row_rms(i, m);
                float nv[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) nv[v] = acc[i][0][v] / rms;
                float* xg = ra.xg_out + row * 32 + 4 * hh;
#pragma unroll
                for (int cg = 0; cg < 4; ++cg)
                    *reinterpret_cast<float4*>(xg + cg * 8) =
                        make_float4(nv[cg * 4], nv[cg * 4 + 1], nv[cg * 4 + 2], nv[cg * 4 + 3]);
                for (int h = 0; h < ra.nkv; ++h) {
                    const float* w = ra.gate_w + h * 32 + 4 * hh;
                    float q = 0.f;
#pragma unroll
                    for (int cg = 0; cg < 4; ++cg)
#pragma unroll
                        for (int e = 0; e < 4; ++e) q += w[cg * 8 + e] * nv[cg * 4 + e];
                    q += __shfl_xor(q, 32, kWave);
                    if (hh == 0) ra.gate_out[row * ra.nkv + h] = 2.0f * (1.0f / (1.0f + __expf(-q)));
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
        }
    }
}

// Vector form of splitk_reduce_k (N % 4 == 0, ldc % 4 == 0, 16-byte aligned
// partial / C): four columns per thread, the split partials' loads issued
// eight at a time ahead of their in-order adds (same order as the scalar form).
template <typename TC>
__global__ __launch_bounds__(256) void splitk_reduce4_k(TC* C, const float* partial, int64_t M, int64_t N,
                                                        int64_t ldc, int64_t splits, int accumulate) {
    const int64_t mn = M * N, n4 = mn / 4;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n4; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = j * 4, r = i / N, c = i % N;
        float4 s = accumulate ? ld4(C + r * ldc + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        int64_t z = 0;
        for (; z + 8 <= splits; z += 8) {
            float4 p[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) p[u] = *reinterpret_cast<const float4*>(partial + (z + u) * mn + i);
#pragma unroll
            for (int u = 0; u < 8; ++u) s = add4(s, p[u]);
        }
        for (; z < splits; ++z) s = add4(s, *reinterpret_cast<const float4*>(partial + z * mn + i));
        st4(C + r * ldc + c, s);
    }
}

template <typename TC>
static void splitk_reduce(hipStream_t st, TC* C, const float* partial, int64_t M, int64_t N, int64_t ldc,
                          int64_t splits, bool accumulate, int64_t batch, int64_t sC) {
    const bool vec = batch == 1 && N % 4 == 0 && ldc % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(partial)) & 15) == 0;
    if (vec)
        splitk_reduce4_k<TC><<<flat_grid(M * N / 4, 256), 256, 0, st>>>(C, partial, M, N, ldc, splits,
                                                                        accumulate ? 1 : 0);
    else
        splitk_reduce_k<TC><<<flat_grid(M * N * batch, 256 * 4), 256, 0, st>>>(C, partial, M, N, ldc, splits,
                                                                               accumulate ? 1 : 0, batch, sC);
}

template <bool BF16, typename TL>
constexpr size_t lds_bytes() {
    using MM = Mfma<BF16>;
    // K-major tiles are the larger layout (padded rows); TR tiles fit inside.
    const size_t stages = (size_t)2 * (TL::BM + TL::BN) * MM::LDK * sizeof(typename MM::LT);
    const size_t strips = (size_t)(TL::THREADS / 64) * 32 * (TL::WN + 8) * sizeof(float);
    return stages > strips ? stages : strips;
}

}  // namespace

namespace ar {

template <bool BF16>
static int64_t choose_splits(int64_t tiles, int64_t K, int64_t splits_req, int64_t& kps, int64_t target = 512) {
    constexpr int BKt = Mfma<BF16>::BK;
    int64_t splits = splits_req;
    if (splits < 1) {
        // Aim for `target` workgroups when the reduction is long.
        splits = 1;
        while (tiles * splits < target && K / (splits * 2) >= 4 * BKt) splits *= 2;
    }
    kps = ((K + splits - 1) / splits + BKt - 1) / BKt * BKt;
    if (kps < BKt) kps = BKt;
    splits = (K + kps - 1) / kps;
    return splits < 1 ? 1 : splits;
}

// Launches one GEMM in GEMM space: C[mo, no] (+)= sum_r A(mo, r) B(no, r).
// epi: EPI_STORE / EPI_ACCUM select by `accumulate` when epi < 0.
template <typename TA, typename TB, typename TC, bool AK, bool BKM, bool BF16, typename TL>
static int32_t gemm_launch_t(hipStream_t st, TC* C, const TA* A, const TB* B, int64_t M, int64_t N, int64_t K,
                             int64_t lda, int64_t ldb, int64_t ldc, bool accumulate, int64_t splits_req,
                             float* partial, const char* nm, int64_t batch, int64_t sA, int64_t sB, int64_t sC,
                             int epi, const void* aux, void* aux_out, float cap, float beta) {
    const int64_t tiles = ((M + TL::BM - 1) / TL::BM) * ((N + TL::BN - 1) / TL::BN);
    int64_t kps = 0;
    // one 256x256 workgroup per CU, two 128x128 ones
    const int64_t target = TL::BM == 256 ? 256 : 512;
    const int64_t splits = epi >= 0 ? 1 : choose_splits<BF16>(tiles * batch, K, splits_req, kps, target);
    if (epi >= 0) choose_splits<BF16>(tiles * batch, K, 1, kps);
    const size_t lds = lds_bytes<BF16, TL>();
    const unsigned grid = (unsigned)(tiles * splits * batch);
#define AR_GK(E)                                                                                              \
    gemm_k<TA, TB, TC, AK, BKM, BF16, E, TL><<<grid, TL::THREADS, lds, st>>>(C, A, B, M, N, K, lda, ldb, ldc, kps, \
                                                                            partial, batch, sA, sB, sC, aux,    \
                                                                            aux_out, cap, beta)
    if (epi >= 0) {
        switch (epi) {
            case EPI_ADD: AR_GK(EPI_ADD); break;
            case EPI_RELU2: AR_GK(EPI_RELU2); break;
            case EPI_SOFTCAP: AR_GK(EPI_SOFTCAP); break;
            case EPI_RELU2_BWD: AR_GK(EPI_RELU2_BWD); break;
            case EPI_AXPBY: AR_GK(EPI_AXPBY); break;
            default: return set_error(AR_EINVAL, "%s: bad epilogue %d", nm, epi);
        }
        return check_launch(nm);
    }
    if (splits == 1) {
        if (accumulate) AR_GK(EPI_ACCUM);
        else AR_GK(EPI_STORE);
        return check_launch(nm);
    }
    if (!partial) return set_error(AR_EINVAL, "%s: split-K scratch missing", nm);
    AR_GK(EPI_PARTIAL);
#undef AR_GK
    splitk_reduce<TC>(st, C, partial, M, N, ldc, splits, accumulate, batch, sC);
    return check_launch(nm);
}

// ---- persistent bf16-operand GEMM (gemm_pk) ----
// GEMM-space shapes it takes: whole 256 x 256 tiles, 64-deep k-tiles, 16-byte
// aligned operands whose rows start on 16-byte boundaries.
static bool pk_shape(int64_t gm, int64_t gn, int64_t gk) {
    return gm > 0 && gn > 0 && gk > 0 && gm % 256 == 0 && gn % 256 == 0 && gk % kPkBK == 0;
}
static bool pk_ok(int64_t gm, int64_t gn, int64_t gk, int64_t lda, int64_t ldb, int64_t ldc, const void* A,
                  const void* B, const void* C) {
    // per-lane DMA / epilogue offsets and item indices are 32-bit
    const bool fits = lda < (1 << 22) && ldb < (1 << 22) && ldc < (1 << 22) && (gm / 256) * (gn / 256) * gk / kPkBK < (1ll << 30);
    return fits && pk_shape(gm, gn, gk) && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0 &&
           ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) & 15) == 0;
}
static int pk_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}
// Split count of the persistent kernel: the largest power of two (each split
// a whole number of k-tiles, at least 4 of them) whose work items still fit
// one round of the persistent workgroups, one per CU.  One more doubling
// would spill items into a second round, which costs the same k-steps on the
// busiest workgroup plus one more partial epilogue and twice the partials.
static int64_t pk_splits(int64_t tiles, int64_t gk) {
    const int64_t wgs = pk_cus();
    int64_t s = 1;
    while (tiles * 2 * s <= wgs && gk % (2 * s * kPkBK) == 0 && gk / (2 * s) >= 4 * kPkBK) s *= 2;
    return s;
}

// C (+)= A . B^T in GEMM space with gemm_pk (operands checked by pk_ok).
// epi < 0: STORE / ACCUM by `accumulate`, split over the reduction when
// splits > 1 (fp32 partials in `partial`, then an in-order reduce).
template <bool AK, bool BKM, typename TC>
static int32_t pk_launch(hipStream_t st, TC* C, const bf16* A, const bf16* B, int64_t gm, int64_t gn, int64_t gk,
                         int64_t lda, int64_t ldb, int64_t ldc, bool accumulate, int64_t splits, float* partial,
                         int epi, const void* aux, void* aux_out, float cap, const char* nm) {
    if (splits < 1) splits = 1;
    if (gk % (splits * kPkBK) != 0) return set_error(AR_EINVAL, "%s: split %lld does not divide K", nm, (long long)splits);
    const int64_t kps = gk / splits, items = (gm / 256) * (gn / 256) * splits;
    const int cus = pk_cus();
    const unsigned grid = (unsigned)(items < cus ? items : cus);
#define AR_PK(E)                                                                                                      do {                                                                                                                  static bool attr_set = false;                                                                                     if (!attr_set) {                                                                                                      if (hipFuncSetAttribute((const void*)gemm_pk<AK, BKM, TC, E>,                                                                              hipFuncAttributeMaxDynamicSharedMemorySize, kPkLds) != hipSuccess)                            return set_error(AR_EHIP, "%s: cannot set the LDS size", nm);                                                 attr_set = true;                                                                                              }                                                                                                                 gemm_pk<AK, BKM, TC, E><<<grid, kPkThreads, kPkLds, st>>>(C, A, B, gm, gn, lda, ldb, ldc, kps, splits,                                                                       partial, aux, aux_out, cap, PkHead{});                         } while (0)
    if (epi >= 0) {
        if (splits != 1) return set_error(AR_EINVAL, "%s: fused epilogues take no reduction split", nm);
        if constexpr (AK) {  // fused epilogues exist for the NT and NN layouts only
            switch (epi) {
                case EPI_ADD: AR_PK(EPI_ADD); break;
                case EPI_RELU2: AR_PK(EPI_RELU2); break;
                case EPI_SOFTCAP: AR_PK(EPI_SOFTCAP); break;
                case EPI_RELU2_BWD: AR_PK(EPI_RELU2_BWD); break;
                default: return set_error(AR_EINVAL, "%s: bad epilogue %d", nm, epi);
            }
            return check_launch(nm);
        } else {
            return set_error(AR_EINVAL, "%s: no fused epilogue for this layout", nm);
        }
    }
    if (splits == 1) {
        if (accumulate) AR_PK(EPI_ACCUM);
        else AR_PK(EPI_STORE);
        return check_launch(nm);
    }
    if (!partial) return set_error(AR_EINVAL, "%s: split-K scratch missing", nm);
    AR_PK(EPI_PARTIAL);
#undef AR_PK
    splitk_reduce<TC>(st, C, partial, gm, gn, ldc, splits, accumulate, 1, 0);
    return check_launch(nm);
}

// NT product on the head-aligned persistent kernel with a head epilogue
// (EPI_QKV / EPI_DOUT_D); hd selects the instance.
template <int EPI>
static int32_t pk_head_launch(hipStream_t st, bf16* C, const bf16* A, const bf16* B, int64_t gm, int64_t gn, int64_t gk,
                              int64_t ldc, const PkHead& hx, int64_t hd, const char* nm) {
    const int64_t items = (gm / 256) * (gn / 256);
    const int cus = pk_cus();
    const unsigned grid = (unsigned)(items < cus ? items : cus);
#define AR_PKH(HD)                                                                                                   \
    do {                                                                                                             \
        static bool attr_set = false;                                                                                \
        if (!attr_set) {                                                                                             \
            if (hipFuncSetAttribute((const void*)gemm_pk<true, true, bf16, EPI, HD>,                                 \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kPkLds) != hipSuccess)               \
                return set_error(AR_EHIP, "%s: cannot set the LDS size", nm);                                        \
            attr_set = true;                                                                                         \
        }                                                                                                            \
        gemm_pk<true, true, bf16, EPI, HD><<<grid, kPkThreads, kPkLds, st>>>(C, A, B, gm, gn, gk, gk, ldc, gk, 1,     \
                                                                             nullptr, nullptr, nullptr, 0.f, hx);    \
    } while (0)
    if (hd == 128) AR_PKH(128);
    else if (hd == 64) AR_PKH(64);
    else return set_error(AR_EUNSUPPORTED, "%s: head_dim %lld", nm, (long long)hd);
#undef AR_PKH
    return check_launch(nm);
}

bool gemm_rc_fusable(int64_t M, int64_t C, int64_t K) {
    return C == kRcN && M > 0 && M % kRcBM == 0 && K > 0 && K % kPkBK == 0 && K < (1 << 20) &&
           M / kRcBM < (1 << 30) / (K / kPkBK);
}

int32_t gemm_rc_norm(hipStream_t st, const bf16* A, const bf16* W, int64_t M, int64_t K, const float* r, float* x_out,
                     float* rms_out, bf16* xn_out, const float* x0, const float* sa, const float* sb, int64_t layer,
                     float* xg_out, float* gate_out, const float* gate_w, int64_t nkv) {
    if (!gemm_rc_fusable(M, kRcN, K) || ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(W) |
                                          reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(x_out) |
                                          reinterpret_cast<uintptr_t>(xn_out)) & 15) != 0 ||
        (gate_out && (nkv <= 0 || nkv > 64 || !xg_out || !gate_w)))
        return set_error(AR_EINVAL, "gemm_rc_norm: unsupported shape / alignment");
    RcArgs ra{r, x_out, rms_out, xn_out, x0, sa, sb, layer, xg_out, gate_out, gate_w, (int)nkv};
    const int64_t items = M / kRcBM;
    const int cus = pk_cus();
    const unsigned grid = (unsigned)(items < cus ? items : cus);
#define AR_RC(SC)                                                                                                    \
    do {                                                                                                             \
        static bool attr_set = false;                                                                                \
        if (!attr_set) {                                                                                             \
            if (hipFuncSetAttribute((const void*)gemm_rc<SC>, hipFuncAttributeMaxDynamicSharedMemorySize, kRcLds) != \
                hipSuccess)                                                                                          \
                return set_error(AR_EHIP, "gemm_rc_norm: cannot set the LDS size");                                  \
            attr_set = true;                                                                                         \
        }                                                                                                            \
        gemm_rc<SC><<<grid, kPkThreads, kRcLds, st>>>(A, W, M, K, K, K, ra);                                         \
    } while (0)
    if (x0) AR_RC(true);
    else AR_RC(false);
#undef AR_RC
    return check_launch("gemm_rc_norm");
}

bool gemm_head_fusable(int64_t M, int64_t C, int64_t hd) {
    return (hd == 64 || hd == 128) && C % 256 == 0 && pk_shape(M, 3 * C, C) && pk_shape(M, C, C) &&
           3 * C < (1 << 22);
}

int32_t gemm_qkv_fused(hipStream_t st, bf16* q, bf16* k, bf16* v, const bf16* xn, const bf16* w, int64_t M, int64_t C,
                       int64_t hd, const float* cos_t, const float* sin_t, int64_t period, const float* gate,
                       const float* table, const int64_t* idx) {
    if (!((hd == 64 || hd == 128) && C % 256 == 0 && period > 0 && pk_ok(M, 3 * C, C, C, C, C, xn, w, q) &&
          ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) == 0))
        return AR_EUNSUPPORTED;
    PkHead hx{};
    hx.q = q;
    hx.k = k;
    hx.v = v;
    hx.cos_t = cos_t;
    hx.sin_t = sin_t;
    hx.period = period;
    hx.gate = gate;
    hx.table = table;
    hx.idx = idx;
    hx.cpart = C;
    return pk_head_launch<EPI_QKV>(st, q, xn, w, M, 3 * C, C, 3 * C, hx, hd, "linear_fwd (q|k|v, fused post)");
}

int32_t gemm_dout_d_fused(hipStream_t st, bf16* dout, float* d, const bf16* gy, const bf16* wt, const float* o,
                          int64_t M, int64_t C, int64_t hd) {
    if (!((hd == 64 || hd == 128) && pk_ok(M, C, C, C, C, C, gy, wt, dout) &&
          (reinterpret_cast<uintptr_t>(o) & 15) == 0))
        return AR_EUNSUPPORTED;
    PkHead hx{};
    hx.o = o;
    hx.d = d;
    return pk_head_launch<EPI_DOUT_D>(st, dout, gy, wt, M, C, C, C, hx, hd, "linear_bwd_dx (c_proj, fused D)");
}

// Large tiles when the problem has enough of them to fill the chip, or when
// a long reduction (split over K) gives each of a few large tiles enough work.
inline bool use_large(int64_t M, int64_t N, int64_t K, int64_t batch) {
    const int64_t t = ((M + 255) / 256) * ((N + 255) / 256) * batch;
    return t >= 256 || (K >= 16384 && t >= 4);
}

template <typename TA, typename TB, typename TC, bool AK, bool BKM, bool BF16>
static int32_t gemm_launch(hipStream_t st, TC* C, const TA* A, const TB* B, int64_t M, int64_t N, int64_t K,
                           int64_t lda, int64_t ldb, int64_t ldc, bool accumulate, int64_t splits_req,
                           float* partial, const char* nm, int64_t batch = 1, int64_t sA = 0, int64_t sB = 0,
                           int64_t sC = 0, int epi = -1, const void* aux = nullptr, void* aux_out = nullptr,
                           float cap = 0.f, float beta = 0.f) {
    if (use_large(M, N, K, batch))
        return gemm_launch_t<TA, TB, TC, AK, BKM, BF16, TileL>(st, C, A, B, M, N, K, lda, ldb, ldc, accumulate,
                                                               splits_req, partial, nm, batch, sA, sB, sC, epi, aux,
                                                               aux_out, cap, beta);
    return gemm_launch_t<TA, TB, TC, AK, BKM, BF16, TileS>(st, C, A, B, M, N, K, lda, ldb, ldc, accumulate,
                                                           splits_req, partial, nm, batch, sA, sB, sC, epi, aux,
                                                           aux_out, cap, beta);
}

// GEMM-space sizes of a reference-layout call.
static void gemm_space(int layout, int64_t M, int64_t N, int64_t K, int64_t& gm, int64_t& gn, int64_t& gk) {
    if (layout == 0) { gm = M; gn = N; gk = K; }
    else if (layout == 1) { gm = M; gn = K; gk = N; }
    else { gm = N; gn = K; gk = M; }
}

// Split count of gemm_k's automatic choice for a TN call.
static int64_t gemm_k_splits(bool bf16, int64_t gm, int64_t gn, int64_t gk) {
    int64_t kps;
    const bool large = use_large(gm, gn, gk, 1);
    const int64_t tiles = large ? ((gm + 255) / 256) * ((gn + 255) / 256) : ((gm + 127) / 128) * ((gn + 127) / 128);
    const int64_t target = large ? 256 : 512;
    return bf16 ? choose_splits<true>(tiles, gk, 0, kps, target) : choose_splits<false>(tiles, gk, 0, kps, target);
}

// Split count of a TN call: the persistent kernel's for the shapes it runs
// (bf16 operands in memory, whole tiles), otherwise gemm_k's; scratch sized
// with it serves either kernel.
int64_t gemm_auto_splits(int layout, bool bf16, bool bf16_operands, int64_t M, int64_t N, int64_t K) {
    if (layout != 2) return 1;
    int64_t gm, gn, gk;
    gemm_space(layout, M, N, K, gm, gn, gk);
    // its split count also serves gemm_k, which takes the count as given if
    // it runs instead (a misaligned operand)
    if (bf16 && bf16_operands && pk_shape(gm, gn, gk)) return pk_splits((gm / 256) * (gn / 256), gk);
    return gemm_k_splits(bf16, gm, gn, gk);
}

int64_t gemm_partial_elems(int layout, int64_t M, int64_t N, int64_t K, int64_t splits) {
    int64_t gm, gn, gk;
    gemm_space(layout, M, N, K, gm, gn, gk);
    return splits > 1 ? splits * gm * gn : 0;
}

// Batched, GEMM-space form used by Muon: C_b[mo,no] = sum_r A_b(mo,r) B_b(no,r)
// with A/B K-major (ak/bk) or MN-major, operand b at base + b * stride.  No
// reduction split: the batch supplies the parallelism.
// The same with bf16 operands in memory (copies of fp32 matrices, rounded as
// the fp32-operand form rounds them on load, so the products are identical),
// and an optional bf16 copy Cb of the fp32 result (same strides as C).
int32_t gemm_batched_bf16(hipStream_t st, bool ak, bool bk, float* C, bf16* Cb, const bf16* A, const bf16* B,
                          int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                          int64_t sA, int64_t sB, int64_t sC, const float* aux, float alpha, float beta) {
    const int epi = aux ? EPI_AXPBY : -1;
#define AR_GB(AKv, BKv)                                                                                          \
    gemm_launch<bf16, bf16, float, AKv, BKv, true>(st, C, A, B, M, N, K, lda, ldb, ldc, false, 1, nullptr,         \
                                                   "gemm_batched_bf16", batch, sA, sB, sC, epi, aux, Cb, alpha, beta)
    if (ak && bk) return AR_GB(true, true);
    if (ak && !bk) return AR_GB(true, false);
    if (!ak && !bk) return AR_GB(false, false);
    return AR_GB(false, true);
#undef AR_GB
}

int32_t gemm_batched_f32(hipStream_t st, bool bf, bool ak, bool bk, float* C, const float* A, const float* B,
                         int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                         int64_t sA, int64_t sB, int64_t sC, const float* aux, float alpha, float beta) {
    const int epi = aux ? EPI_AXPBY : -1;
#define AR_GB(AKv, BKv)                                                                                        \
    (bf ? gemm_launch<float, float, float, AKv, BKv, true>(st, C, A, B, M, N, K, lda, ldb, ldc, false, 1, nullptr, \
                                                           "gemm_batched", batch, sA, sB, sC, epi, aux, nullptr, \
                                                           alpha, beta)                                       \
        : gemm_launch<float, float, float, AKv, BKv, false>(st, C, A, B, M, N, K, lda, ldb, ldc, false, 1, nullptr, \
                                                            "gemm_batched", batch, sA, sB, sC, epi, aux, nullptr, \
                                                            alpha, beta))
    if (ak && bk) return AR_GB(true, true);
    if (ak && !bk) return AR_GB(true, false);
    if (!ak && !bk) return AR_GB(false, false);
    return AR_GB(false, true);
#undef AR_GB
}

// Reference-layout GEMM with per-operand storage types (bf16 compute).
template <typename TX, typename TW, typename TC>
static int32_t gemm_typed(hipStream_t st, int layout, TC* C, const TX* X, const TW* W, int64_t M, int64_t N,
                          int64_t K, bool accumulate, int64_t splits, float* partial) {
    if constexpr (std::is_same<TX, bf16>::value && std::is_same<TW, bf16>::value) {
        // bf16 operands in memory: the persistent direct-to-LDS kernel when the shape allows
        if (layout == 0 && pk_ok(M, N, K, K, K, N, X, W, C))
            return pk_launch<true, true, TC>(st, C, X, W, M, N, K, K, K, N, accumulate, 1, nullptr, -1, nullptr,
                                             nullptr, 0.f, "linear_fwd");
        if (layout == 1 && pk_ok(M, K, N, N, K, K, X, W, C))
            return pk_launch<true, false, TC>(st, C, X, W, M, K, N, N, K, K, accumulate, 1, nullptr, -1, nullptr,
                                              nullptr, 0.f, "linear_bwd_dx");
        if (layout == 2 && pk_ok(N, K, M, N, K, K, X, W, C)) {
            const int64_t s = splits >= 1 ? splits : pk_splits((N / 256) * (K / 256), M);
            if (M % (s * kPkBK) == 0)
                return pk_launch<false, false, TC>(st, C, X, W, N, K, M, N, K, K, accumulate, s, partial, -1, nullptr,
                                                   nullptr, 0.f, "linear_bwd_dw");
        }
    }
    if (layout == 0)
        return gemm_launch<TX, TW, TC, true, true, true>(st, C, X, W, M, N, K, K, K, N, accumulate, 1, nullptr,
                                                         "linear_fwd");
    if (layout == 1)
        return gemm_launch<TX, TW, TC, true, false, true>(st, C, X, W, M, K, N, N, K, K, accumulate, 1, nullptr,
                                                          "linear_bwd_dx");
    if (splits < 1)
        splits = gemm_auto_splits(2, true, std::is_same<TX, bf16>::value && std::is_same<TW, bf16>::value, M, N, K);
    return gemm_launch<TX, TW, TC, false, false, true>(st, C, X, W, N, K, M, N, K, K, accumulate, splits, partial,
                                                       "linear_bwd_dw");
}

int32_t gemm_bf16io(hipStream_t st, int layout, void* C, int c_bf16, const void* X, int x_bf16, const void* W,
                    int w_bf16, int64_t M, int64_t N, int64_t K, bool accumulate, int64_t splits, float* partial) {
#define AR_GT(TX, TW, TC) \
    gemm_typed<TX, TW, TC>(st, layout, (TC*)C, (const TX*)X, (const TW*)W, M, N, K, accumulate, splits, partial)
    if (x_bf16 && w_bf16 && c_bf16) return AR_GT(bf16, bf16, bf16);
    if (x_bf16 && w_bf16 && !c_bf16) return AR_GT(bf16, bf16, float);
    if (x_bf16 && !w_bf16 && !c_bf16) return AR_GT(bf16, float, float);
    if (!x_bf16 && w_bf16 && !c_bf16) return AR_GT(float, bf16, float);
    if (!x_bf16 && w_bf16 && c_bf16) return AR_GT(float, bf16, bf16);
    if (!x_bf16 && !w_bf16 && c_bf16) return AR_GT(float, float, bf16);
    return AR_GT(float, float, float);
#undef AR_GT
}

// NT (layout 0) / NN (layout 1) GEMM with a fused epilogue (bf16 compute).
// epi: 3 ADD (aux = fp32 R), 4 RELU2 (aux_out = act), 5 SOFTCAP (cap),
// 6 RELU2_BWD (aux = pre-activation).  TX/TW/TC per the flags.
int32_t gemm_epilogue(hipStream_t st, int layout, int epi, void* C, int c_bf16, const void* X, int x_bf16,
                      const void* W, int w_bf16, int64_t M, int64_t N, int64_t K, const void* aux, void* aux_out,
                      float cap) {
    if (x_bf16 && w_bf16) {
        // bf16 operands in memory: the persistent direct-to-LDS kernel when the shape allows
        const bf16 *Xb = (const bf16*)X, *Wb = (const bf16*)W;
        if (layout == 0 && pk_ok(M, N, K, K, K, N, X, W, C))
            return c_bf16 ? pk_launch<true, true, bf16>(st, (bf16*)C, Xb, Wb, M, N, K, K, K, N, false, 1, nullptr, epi,
                                                        aux, aux_out, cap, "gemm_epilogue")
                          : pk_launch<true, true, float>(st, (float*)C, Xb, Wb, M, N, K, K, K, N, false, 1, nullptr,
                                                         epi, aux, aux_out, cap, "gemm_epilogue");
        if (layout == 1 && pk_ok(M, K, N, N, K, K, X, W, C))
            return c_bf16 ? pk_launch<true, false, bf16>(st, (bf16*)C, Xb, Wb, M, K, N, N, K, K, false, 1, nullptr, epi,
                                                         aux, aux_out, cap, "gemm_epilogue")
                          : pk_launch<true, false, float>(st, (float*)C, Xb, Wb, M, K, N, N, K, K, false, 1, nullptr,
                                                          epi, aux, aux_out, cap, "gemm_epilogue");
    }
#define AR_GE(TX, TW, TC)                                                                                          \
    (layout == 0 ? gemm_launch<TX, TW, TC, true, true, true>(st, (TC*)C, (const TX*)X, (const TW*)W, M, N, K, K, K, N, \
                                                             false, 1, nullptr, "gemm_epilogue", 1, 0, 0, 0, epi, aux, \
                                                             aux_out, cap)                                         \
                 : gemm_launch<TX, TW, TC, true, false, true>(st, (TC*)C, (const TX*)X, (const TW*)W, M, K, N, N, K,  \
                                                              K, false, 1, nullptr, "gemm_epilogue", 1, 0, 0, 0, epi, \
                                                              aux, aux_out, cap))
    if (x_bf16 && w_bf16 && c_bf16) return AR_GE(bf16, bf16, bf16);
    if (x_bf16 && w_bf16 && !c_bf16) return AR_GE(bf16, bf16, float);
    if (!x_bf16 && w_bf16 && c_bf16) return AR_GE(float, bf16, bf16);
    if (!x_bf16 && w_bf16 && !c_bf16) return AR_GE(float, bf16, float);
    return set_error(AR_EINVAL, "gemm_epilogue: unsupported operand types");
#undef AR_GE
}

int32_t gemm_f32_add(hipStream_t st, bool bf, float* C, const float* X, const float* W, const float* R, int64_t M,
                     int64_t N, int64_t K) {
    if (bf)
        return gemm_launch<float, float, float, true, true, true>(st, C, X, W, M, N, K, K, K, N, false, 1, nullptr,
                                                                  "linear_fwd_add", 1, 0, 0, 0, EPI_ADD, R, nullptr,
                                                                  0.f);
    return gemm_launch<float, float, float, true, true, false>(st, C, X, W, M, N, K, K, K, N, false, 1, nullptr,
                                                               "linear_fwd_add", 1, 0, 0, 0, EPI_ADD, R, nullptr, 0.f);
}

int32_t gemm_f32(hipStream_t st, int layout, bool bf, float* C, const float* X, const float* W, int64_t M, int64_t N,
                 int64_t K, bool accumulate, int64_t splits, float* partial) {
    if (layout == 0) {
        if (bf)
            return gemm_launch<float, float, float, true, true, true>(st, C, X, W, M, N, K, K, K, N, accumulate, 1,
                                                                      nullptr, "linear_fwd");
        return gemm_launch<float, float, float, true, true, false>(st, C, X, W, M, N, K, K, K, N, accumulate, 1,
                                                                   nullptr, "linear_fwd");
    }
    if (layout == 1) {
        // GEMM (mo=M, no=K, r=N): A = dY [M][N] K-major, B(no=k, r=n) = W[n][k] MN-major.
        if (bf)
            return gemm_launch<float, float, float, true, false, true>(st, C, X, W, M, K, N, N, K, K, accumulate, 1,
                                                                       nullptr, "linear_bwd_dx");
        return gemm_launch<float, float, float, true, false, false>(st, C, X, W, M, K, N, N, K, K, accumulate, 1,
                                                                    nullptr, "linear_bwd_dx");
    }
    // TN: GEMM (mo=N, no=K, r=M): A(mo=n, r=m) = dY[m][n] MN-major, B(no=k, r=m) = X[m][k] MN-major.
    if (splits < 1) splits = gemm_auto_splits(2, bf, false, M, N, K);
    if (bf)
        return gemm_launch<float, float, float, false, false, true>(st, C, X, W, N, K, M, N, K, K, accumulate,
                                                                    splits, partial, "linear_bwd_dw");
    return gemm_launch<float, float, float, false, false, false>(st, C, X, W, N, K, M, N, K, K, accumulate, splits,
                                                                 partial, "linear_bwd_dw");
}

}  // namespace ar

// =====================================================================
// C ABI
// =====================================================================

static int32_t check_gemm_args(const void* C, const void* A, const void* B, int64_t M, int64_t N, int64_t K,
                               const char* nm) {
    if (!C || !A || !B) return set_error(AR_EINVAL, "%s: null pointer", nm);
    if (M < 0 || N < 0 || K < 0) return set_error(AR_EINVAL, "%s: negative dimension", nm);
    if ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) & 3)
        return set_error(AR_EINVAL, "%s: operands must be 4-byte aligned floats", nm);
    return AR_OK;
}

static inline bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
    const char *pa = (const char*)a, *pb = (const char*)b;
    return pa < pb + bbytes && pb < pa + abytes;
}

// The matrix-core kernels take dimensions in multiples of 8 and 16-byte
// aligned operands.  Other calls run the same kernels on zero-padded copies
// in the workspace (the padding adds zero products only) and copy the valid
// region back: the tail path of the reference's bounds-checked tiles
// (ops.mojo:150-168).
static bool gemm_direct(const void* C, const void* A, const void* B, int64_t M, int64_t N, int64_t K) {
    return ((M | N | K) & 7) == 0 &&
           ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) & 15) == 0;
}
static inline int64_t r8(int64_t x) { return (x + 7) & ~int64_t(7); }
static inline size_t al256(size_t b) { return (b + 255) & ~size_t(255); }

namespace {
// dst[r][c] (row stride ldd) = src[r][c] (row stride lds) inside rows x
// cols, 0 elsewhere in the drows x dcols destination.
__global__ void copy2d_k(float* dst, int64_t ldd, const float* src, int64_t lds, int64_t rows, int64_t cols,
                         int64_t drows, int64_t dcols) {
    const int64_t n = drows * dcols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / dcols, c = i - r * dcols;
        dst[r * ldd + c] = (r < rows && c < cols) ? src[r * lds + c] : 0.f;
    }
}
}  // namespace

static int32_t copy2d(hipStream_t st, float* dst, int64_t ldd, const float* src, int64_t lds, int64_t rows,
                      int64_t cols, int64_t drows, int64_t dcols) {
    if (drows * dcols == 0) return AR_OK;
    copy2d_k<<<flat_grid(drows * dcols, 256), 256, 0, st>>>(dst, ldd, src, lds, rows, cols, drows, dcols);
    return check_launch("gemm pad copy");
}

// layout 0: C[M,N] = X[M,K] W[N,K]^T; 1: C[M,K] = X[M,N] W[N,K]; 2: C[N,K] += X[M,N]^T W[M,K].
// Operand shapes (rows, cols) per layout, in that order: X, W, C.
static void gemm_operand_shapes(int layout, int64_t M, int64_t N, int64_t K, int64_t sh[3][2]) {
    const int64_t x[3][2] = {{M, K}, {M, N}, {M, N}};
    const int64_t w[3][2] = {{N, K}, {N, K}, {M, K}};
    const int64_t c[3][2] = {{M, N}, {M, K}, {N, K}};
    for (int i = 0; i < 2; ++i) {
        sh[0][i] = x[layout][i];
        sh[1][i] = w[layout][i];
        sh[2][i] = c[layout][i];
    }
}

static size_t gemm_pad_bytes(int layout, bool bf, int64_t M, int64_t N, int64_t K) {
    int64_t sh[3][2];
    gemm_operand_shapes(layout, r8(M), r8(N), r8(K), sh);
    size_t b = 0;
    for (int i = 0; i < 3; ++i) b += al256((size_t)sh[i][0] * sh[i][1] * sizeof(float));
    if (layout == 2) {
        const int64_t s = ar::gemm_auto_splits(2, bf, false, r8(M), r8(N), r8(K));
        if (s > 1) b += al256((size_t)ar::gemm_partial_elems(2, r8(M), r8(N), r8(K), s) * sizeof(float));
    }
    return b;
}

// Workspace bytes of one linear_* call (0 when it needs none).
static size_t gemm_ws_bytes(int layout, bool bf, const void* C, const void* X, const void* W, int64_t M, int64_t N,
                            int64_t K) {
    if (!gemm_direct(C, X, W, M, N, K)) return gemm_pad_bytes(layout, bf, M, N, K);
    size_t b = 0;
    if (layout == 1 && overlaps(C, M * K * 4, X, M * N * 4)) b += al256((size_t)M * N * sizeof(float));
    if (layout == 2) {
        const int64_t s = ar::gemm_auto_splits(2, bf, false, M, N, K);
        if (s > 1) b += al256((size_t)ar::gemm_partial_elems(2, M, N, K, s) * sizeof(float));
    }
    return b;
}

static int32_t gemm_padded(hipStream_t st, int layout, bool bf, float* C, const float* X, const float* W, int64_t M,
                           int64_t N, int64_t K, char* ws) {
    int64_t sh[3][2], ph[3][2];
    gemm_operand_shapes(layout, M, N, K, sh);
    gemm_operand_shapes(layout, r8(M), r8(N), r8(K), ph);
    float* xp = (float*)ws;
    float* wp = (float*)(ws + al256((size_t)ph[0][0] * ph[0][1] * 4));
    float* cp = (float*)((char*)wp + al256((size_t)ph[1][0] * ph[1][1] * 4));
    float* part = (float*)((char*)cp + al256((size_t)ph[2][0] * ph[2][1] * 4));
    // the copies read all of X before C is written: alias-safe (linear_bwd_dx in place)
    int32_t r = copy2d(st, xp, ph[0][1], X, sh[0][1], sh[0][0], sh[0][1], ph[0][0], ph[0][1]);
    if (!r) r = copy2d(st, wp, ph[1][1], W, sh[1][1], sh[1][0], sh[1][1], ph[1][0], ph[1][1]);
    if (!r && layout == 2) r = copy2d(st, cp, ph[2][1], C, sh[2][1], sh[2][0], sh[2][1], ph[2][0], ph[2][1]);
    if (r) return r;
    const int64_t splits = layout == 2 ? ar::gemm_auto_splits(2, bf, false, r8(M), r8(N), r8(K)) : 1;
    r = ar::gemm_f32(st, layout, bf, cp, xp, wp, r8(M), r8(N), r8(K), layout == 2, splits, part);
    if (r) return r;
    return copy2d(st, C, sh[2][1], cp, ph[2][1], sh[2][0], sh[2][1], sh[2][0], sh[2][1]);
}

// Where a linear_* call takes its scratch from: the workspace bound to its
// stream, or (fixed != nullptr) a caller-supplied region of fixed_bytes.
struct ScratchSrc {
    char* fixed;
    size_t fixed_bytes;
};

static int32_t linear_call(ar_stream_t s, int layout, bool bf, float* C, const float* X, const float* W, int64_t M,
                           int64_t N, int64_t K, const char* nm, ScratchSrc src_ws = ScratchSrc{nullptr, 0}) {
    int32_t st = check_gemm_args(C, X, W, M, N, K, nm);
    if (st) return st;
    int64_t sh[3][2];
    gemm_operand_shapes(layout, M, N, K, sh);
    const size_t cb = (size_t)sh[2][0] * sh[2][1] * 4;
    if (sh[2][0] * sh[2][1] == 0) return AR_OK;
    if (overlaps(C, cb, W, (size_t)sh[1][0] * sh[1][1] * 4) ||
        (layout != 1 && overlaps(C, cb, X, (size_t)sh[0][0] * sh[0][1] * 4)))
        return set_error(AR_EINVAL, "%s: output overlaps an input", nm);
    const int64_t red = layout == 0 ? K : (layout == 1 ? N : M);  // reduction length
    if (red == 0) return layout == 2 ? AR_OK : ar_zero_buffer(s, C, sh[2][0] * sh[2][1]);
    const size_t need = gemm_ws_bytes(layout, bf, C, X, W, M, N, K);
    char* ws = nullptr;
    if (need && src_ws.fixed) {
        if (need > src_ws.fixed_bytes)
            return set_error(AR_EINVAL, "%s: this shape needs %zu bytes of scratch, above the fixed %zu", nm, need,
                             src_ws.fixed_bytes);
        ws = src_ws.fixed;
    } else if (need) {
        ws = (char*)ar::workspace(S(s), need, &st);
        if (!ws) return st;
    }
    if (!gemm_direct(C, X, W, M, N, K)) return gemm_padded(S(s), layout, bf, C, X, W, M, N, K, ws);
    const float* src = X;
    if (layout == 1 && overlaps(C, cb, X, (size_t)M * N * 4)) {
        // model.mojo:906 calls this in place; read all of dY first (copy).
        if (hipMemcpyAsync(ws, X, (size_t)M * N * sizeof(float), hipMemcpyDeviceToDevice, S(s)) != hipSuccess)
            return set_error(AR_EHIP, "linear_bwd_dx: alias copy failed");
        src = (const float*)ws;
    }
    int64_t splits = 1;
    float* partial = nullptr;
    if (layout == 2) {
        splits = ar::gemm_auto_splits(2, bf, false, M, N, K);
        if (splits > 1) partial = (float*)ws;
    }
    return ar::gemm_f32(S(s), layout, bf, C, src, W, M, N, K, layout == 2, splits, partial);
}

static int32_t linear_fwd_impl(ar_stream_t s, float* out, const float* in, const float* w, int64_t M, int64_t N,
                               int64_t K, bool bf) {
    return linear_call(s, 0, bf, out, in, w, M, N, K, "linear_fwd");
}
static int32_t linear_bwd_dx_impl(ar_stream_t s, float* dx, const float* dy, const float* w, int64_t M, int64_t N,
                                  int64_t K, bool bf) {
    return linear_call(s, 1, bf, dx, dy, w, M, N, K, "linear_bwd_dx");
}
static int32_t linear_bwd_dw_impl(ar_stream_t s, float* dw, const float* dy, const float* x, int64_t M, int64_t N,
                                  int64_t K, bool bf) {
    return linear_call(s, 2, bf, dw, dy, x, M, N, K, "linear_bwd_dw");
}

extern "C" int32_t ar_linear_fwd(ar_stream_t stream, float* output, const float* input, const float* weight,
                                 int64_t M, int64_t N, int64_t K) {
    return linear_fwd_impl(stream, output, input, weight, M, N, K, false);
}
extern "C" int32_t ar_linear_fwd_bf16(ar_stream_t stream, float* output, const float* input, const float* weight,
                                      int64_t M, int64_t N, int64_t K) {
    return linear_fwd_impl(stream, output, input, weight, M, N, K, true);
}
extern "C" int32_t ar_linear_bwd_dx(ar_stream_t stream, float* grad_input, const float* grad_output,
                                    const float* weight, int64_t M, int64_t N, int64_t K) {
    return linear_bwd_dx_impl(stream, grad_input, grad_output, weight, M, N, K, false);
}
extern "C" int32_t ar_linear_bwd_dx_bf16(ar_stream_t stream, float* grad_input, const float* grad_output,
                                         const float* weight, int64_t M, int64_t N, int64_t K) {
    return linear_bwd_dx_impl(stream, grad_input, grad_output, weight, M, N, K, true);
}
extern "C" int32_t ar_linear_bwd_dw(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                    const float* input, int64_t M, int64_t N, int64_t K) {
    return linear_bwd_dw_impl(stream, grad_weight, grad_output, input, M, N, K, false);
}
extern "C" int32_t ar_linear_bwd_dw_bf16(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                         const float* input, int64_t M, int64_t N, int64_t K) {
    return linear_bwd_dw_impl(stream, grad_weight, grad_output, input, M, N, K, true);
}

// ---- linear_bwd_dw_bf16 with no workspace: scratch in a fixed device array ----
// For callers that cannot allocate device memory or bind a workspace (code
// under stream capture, serving loops, harnesses that forbid it).  The split-K
// partials (and, for shapes off the 8-multiple / 16-byte-aligned grid, the
// zero-padded operand copies) go to `scratch`, one copy per device, held for
// the life of the process.  Every call on a device shares that device's array:
// calls that overlap in time on one device (two streams, two threads) race.
// Nothing in it needs to start at zero: the partials and the padded copies
// are written in full before they are read.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// Device address of this device's `scratch` (the host-side name is only a
// handle for the symbol lookup), looked up once per device.
static char* noalloc_scratch(int32_t* status) {
    constexpr int kMaxDev = 64;
    static std::mutex mu;
    static char* addr[kMaxDev] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
        *status = set_error(AR_EHIP, "linear_bwd_dw_bf16_noalloc: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            *status = set_error(AR_EHIP, "linear_bwd_dw_bf16_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = static_cast<char*>(p);
    }
    *status = AR_OK;
    return addr[dev];
}

extern "C" int32_t ar_linear_bwd_dw_bf16_noalloc(ar_stream_t stream, float* grad_weight, const float* grad_output,
                                                 const float* input, int64_t M, int64_t N, int64_t K) {
    // the arguments first: a bad call is AR_EINVAL before any device query
    int32_t st = check_gemm_args(grad_weight, grad_output, input, M, N, K, "linear_bwd_dw_bf16_noalloc");
    if (st) return st;
    char* p = noalloc_scratch(&st);
    if (!p) return st;
    return linear_call(stream, 2, true, grad_weight, grad_output, input, M, N, K, "linear_bwd_dw_bf16_noalloc",
                       ScratchSrc{p, kNoAllocScratchBytes});
}

// Reference-layout GEMM with bf16 or fp32 storage per operand; bf16 matrix
// cores, fp32 accumulation.  No counterpart in the reference (fp32 only): the
// storage-typed form the bf16 training step uses.
extern "C" int32_t ar_gemm_mixed(ar_stream_t stream, int32_t layout, void* C, int32_t c_bf16, const void* X,
                                 int32_t x_bf16, const void* W, int32_t w_bf16, int64_t M, int64_t N, int64_t K,
                                 int32_t accumulate) {
    int32_t st = check_gemm_args(C, X, W, M, N, K, "gemm_mixed");
    if (st) return st;
    if (!gemm_direct(C, X, W, M, N, K))
        return set_error(AR_EINVAL, "gemm_mixed: M, N, K must be multiples of 8 and operands 16-byte aligned");
    if (layout < 0 || layout > 2) return set_error(AR_EINVAL, "gemm_mixed: layout must be 0 (NT), 1 (NN) or 2 (TN)");
    if (M == 0 || N == 0 || K == 0) return AR_OK;
    const int64_t splits = layout == 2 ? ar::gemm_auto_splits(2, true, x_bf16 && w_bf16, M, N, K) : 1;
    float* partial = nullptr;
    if (splits > 1) {
        partial = (float*)ar::workspace(S(stream), (size_t)ar::gemm_partial_elems(2, M, N, K, splits) * sizeof(float), &st);
        if (!partial) return st;
    }
    return ar::gemm_bf16io(S(stream), layout, C, c_bf16, X, x_bf16, W, w_bf16, M, N, K, accumulate != 0, splits,
                           partial);
}
