// ar_common.hpp -- shared helpers for the gfx950 (CDNA4) kernel library.
//
// Conventions for every kernel source in this directory:
//   * wave64 everywhere; reductions use DPP/ds_swizzle-backed __shfl_xor.
//   * fp32 arithmetic in element kernels; bf16 only as a storage / MFMA
//     operand type, always with fp32 accumulation.
//   * entry points return AR_OK or a negative ar_status and never throw.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ar_ops.h"

namespace ar {

using bf16 = __bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---- error plumbing and workspaces (ar_runtime.hip) ----
int32_t set_error(int32_t code, const char* fmt, ...);
int32_t check_launch(const char* what);
inline hipStream_t S(ar_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// The scratch of the workspace the caller bound to stream st on the current
// device (ar_workspace_bind), if it holds at least `bytes`; otherwise null and
// *status = AR_ENOMEM with a message naming the bytes needed.  Never allocates.
void* workspace(hipStream_t st, size_t bytes, int32_t* status);

// ---- device helpers ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024).  `red` must hold
// blockDim.x/64 floats.  Every thread receives the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave, nw = blockDim.x / kWave;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave, nw = blockDim.x / kWave;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
    return t;
}

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<bf16>(bf16 v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }

// Direct global -> LDS loads (global_load_lds_dword{,x4}): lane i writes LDS
// bytes [lds + size * i, +size), lds wave-uniform.  Issued from inline asm
// so that the compiler does not treat later LDS reads as possibly aliasing
// the in-flight copy (it would wait for every outstanding prefetch before
// them); callers order the copies with an explicit s_waitcnt vmcnt and a
// barrier.  Compiler-tracked global loads issued after one of these are
// waited for with counts that ignore it, which waits for it too (loads
// complete in order): keep such loads ahead of the copies they should not
// wait for.  m0 is clobbered: the kernels that use these keep nothing of
// their own in m0 (their ISA has no other m0 reference), so clang's warning
// that a reserved register in a clobber list may not be preserved is
// silenced here.  tests/test_isa_m0.py compiles the kernels that use these
// helpers and fails if any other instruction reads or writes m0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
__device__ __forceinline__ void dma16(const void* g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g)
                 : "memory", "m0");
}
// The same with a wave-uniform base address (an SGPR pair) plus a per-lane
// 32-bit byte offset: no per-lane 64-bit address arithmetic per copy.
__device__ __forceinline__ void dma16s(const void* base, unsigned voff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(base)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g)
                 : "memory", "m0");
}

#pragma clang diagnostic pop

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Grid for a flat element-wise kernel: grid-stride loops, capped so a launch
// never exceeds what 256 CUs can keep resident many times over.
inline unsigned flat_grid(int64_t n, int per_block_items) {
    int64_t g = cdiv(n, per_block_items);
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (unsigned)g;
}

}  // namespace ar

#define AR_CHECK_ARG(cond, ...)                                   \
    do {                                                          \
        if (!(cond)) return ar::set_error(AR_EINVAL, __VA_ARGS__); \
    } while (0)

#define AR_LAUNCH_CHECK(what) ar::check_launch(what)
