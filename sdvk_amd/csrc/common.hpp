// common.hpp -- shared types, status plumbing and small device helpers for the
// gfx950 kernels behind include/mi_sdvk.h.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "mi_sdvk.h"

namespace mi {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------- host status --

// Records a thread-local reason and returns `code` (used as `return fail(...)`).
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps the launch's hipGetLastError() to MI_ERR_HIP (with its text) or MI_OK.
int check_launch(const char* what);

// Plan overrides set through mi_tuning_set (status.hip): process-wide, read
// with one atomic load per call, never from the environment. Defaults mean
// "the built-in rules decide". They pick tiles, split counts and workgroup
// sizes only: no override changes an operator's arithmetic beyond the
// summation order of a different plan.
constexpr int kGemmBuilds = 7;  // tile builds of gemm_q8.hip (kNumCfg)
struct Tuning {
    std::atomic<int> gemm_cfg{-1};          // tile build, or -1
    std::atomic<int> gemm_splits{1};        // K splits with gemm_cfg (workspace entries)
    std::atomic<int> nn_general{0};         // 1: the NN GEMM's untiled kernel for every shape
    std::atomic<int> nn_splits{0};          // NN GEMM K splits, or 0
    std::atomic<int> attn_nw{0};            // fp16 attention waves per workgroup (2, 4), or 0
    std::atomic<int> attn_split_rest{-1};   // key split: rest blocks (0 = never split), or -1
    std::atomic<int> attn_split_pieces{2};  // key split: pieces per rest block
    std::atomic<int> attn_direct_store{0};  // 1: attention outputs stored from the MFMA layout
    std::atomic<int> attn_simd_waves{0};    // fp16 attention build: 2 or 3 waves per SIMD, or 0
};
Tuning& tuning();

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// [a, a+na) and [b, b+nb) overlap (byte ranges); empty ranges never overlap.
inline bool overlaps(const void* a, uint64_t na, const void* b, uint64_t nb) {
    if (!a || !b || na == 0 || nb == 0) return false;
    uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}

inline unsigned ceil_div(uint64_t a, uint64_t b) { return static_cast<unsigned>((a + b - 1) / b); }

// Sums the partial planes of a K-split GEMM in split order into C (gemm_q8.hip).
// P holds batch * splits planes of [M, N] floats (row stride N): batch item z,
// split s at P + (z * splits + s) * M * N. op 0: C = sum + bias (bias may be
// NULL); op 1: C += sum; op 2: C += sum + bias. The order of the additions is
// fixed, so results repeat bit for bit.
void launch_splitk_reduce(const float* P, uint32_t splits, float* C, const float* bias, uint32_t M, uint32_t N,
                          uint32_t ldc, uint64_t sC, uint32_t batch, int op, hipStream_t s);

// ----------------------------------------------------------- device helpers --

// fp16 bit pattern -> fp32, exact for every pattern (subnormals scaled by
// 2^-24 explicitly so the result does not depend on the denormal mode).
__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        float v = static_cast<float>(m) * 5.9604644775390625e-8f;  // m * 2^-24
        return __uint_as_float(__float_as_uint(v) | sign);
    }
    uint32_t bits = (e == 0x1fu) ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    return __uint_as_float(bits);
}

// erf GELU, Abramowitz & Stegun 7.1.26 (the published rational approximation
// the reference shader uses): erf(z) ~ 1 - (a1 t + ... + a5 t^5) exp(-z^2),
// t = 1 / (1 + p z), z >= 0, odd extension.
// Contraction is off: every multiply and add rounds on its own, so the GELU
// computes the same bits in every kernel it is inlined into (the GEGLU GEMM
// epilogue and the separate GEGLU kernel agree exactly). The reciprocal and
// the exponential are the hardware's (v_rcp_f32, 1 ulp; v_exp_f32 on
// -z^2 log2(e)): the shader's division and exp carry GLSL's relaxed precision
// too (unary_fwd.comp:32-34), and the error they add here (~1e-7 of the
// output, where exp(-z^2) matters) is far inside the approximation's own.
__device__ __forceinline__ float gelu_erf(float v) {
#pragma clang fp contract(off)
    const float xs = v * 0.70710678118654752440f;
    const float ax = fabsf(xs);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * ax);
    const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
    const float e = 1.0f - poly * __builtin_amdgcn_exp2f(-ax * ax * 1.44269504088896341f);
    const float erf = xs >= 0.0f ? e : -e;
    return 0.5f * v * (1.0f + erf);
}

// Scheduling groups for one K step (instruction-class masks of
// __builtin_amdgcn_sched_group_barrier: 0x008 MFMA, 0x002 VALU, 0x100 LDS read,
// 0x200 LDS write). The step's first fragment reads go first; then every MFMA
// is followed by a share of the next fragment reads and of the store phase
// (conversions, dequantisation, LDS writes of the other stage), so that work
// issues in the MFMA shadow instead of between MFMA bursts.
template <int NMFMA, int NREAD0, int NREAD, int NVALU, int NWRITE>
__device__ __forceinline__ void interleave_step() {
    __builtin_amdgcn_sched_group_barrier(0x100, NREAD0, 0);
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (NREAD + NMFMA - 1) / NMFMA, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, (NVALU + NMFMA - 1) / NMFMA, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, (NWRITE + NMFMA - 1) / NMFMA, 0);
    }
}

// Remaps a linear workgroup id so that consecutive logical tiles land on the
// same XCD. The dispatcher hands workgroup b to XCD b % 8; tiles that share an
// operand should share that XCD's L2.
// Lane index within the wave from the exec-mask bit counts (v_mbcnt), not from
// threadIdx.x: a kernel that needs the lane again after a long loop computes it
// there instead of keeping threadIdx-derived values live across the loop.
__device__ __forceinline__ int lane_id() {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
}

__device__ __forceinline__ unsigned xcd_swizzle(unsigned b, unsigned nb) {
    constexpr unsigned kXcd = 8;
    unsigned xcd = b % kXcd, local = b / kXcd;
    unsigned per = nb / kXcd, rem = nb % kXcd;
    return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

}  // namespace mi
