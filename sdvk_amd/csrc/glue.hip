// glue.hip -- the SDXL transformer block's elementwise / row kernels for gfx950:
// LayerNorm, GEGLU and the in-place residual add.
//
// Reference behaviour:
//   * LayerNorm: src/Modules/Diffusion/sdvkgen.cpp:1094-1103 and
//     shaders/layernorm_fwd.comp:15-38 -- per row of d, mean first, then the
//     mean of squared deviations (two passes, no E[x^2] - mean^2), eps inside
//     the square root, optional affine gamma / beta;
//   * GEGLU: sdvkgen.cpp:1709-1720 -- h = [rows, 2F] (one linear), y = h[:, :F]
//     * gelu(h[:, F:]) with the erf GELU of unary_fwd.comp:28-36
//     (Abramowitz & Stegun 7.1.26, |error| <= 1.5e-7);
//   * residual add: add2 {t, t, a} in place (sdvkgen.cpp:1746,1751,1762).
//
// All three are HBM-bound: each element is read and written once. LayerNorm
// keeps a wave's row in registers (one wave per row, float4 lanes) so the
// two passes cost no extra traffic; GEGLU and add stream float4 with a
// grid-stride loop.
#include "common.hpp"

#include <algorithm>

namespace mi {
namespace {

constexpr int kLnCache = 16;  // float4 per lane cached in registers: rows up to 64 * 4 * 16 = 4096

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// The wave's sum in every lane, mostly by DPP: quad swaps, then the half-row
// and row mirrors (lane i of 8 / 16 reads lane 7 - i / 15 - i) leave each row
// of 16 with its sum; two cross-row exchanges finish. Four of the six steps
// stay in the VALU instead of six LDS permutes of the xor butterfly.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0xb1>(v);   // quad_perm [1, 0, 3, 2]
    v = dpp_add<0x4e>(v);   // quad_perm [2, 3, 0, 1]
    v = dpp_add<0x141>(v);  // row_half_mirror
    v = dpp_add<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Stores four fp32 results as TO: fp32 as they are, fp16 rounded once (RNE)
// each -- the value a GEMM staging an fp32 tensor would round them to. The
// empty register constraint makes the fp32 values opaque, so the rounding to fp16 cannot fuse
// into the instruction that produced them (a mixed-precision fma rounds the
// exact result once, which can differ from rounding the fp32 result).
template <typename TO>
__device__ __forceinline__ void store4(TO* p, floatx4 v) {
    if constexpr (sizeof(TO) == 4) {
        *reinterpret_cast<floatx4*>(p) = v;
    } else {
        asm volatile("" : "+v"(v));
        *reinterpret_cast<half4*>(p) = half4{static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]),
                                             static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
    }
}

// One wave per row; 4 rows per 256-thread workgroup. d % 4 == 0, 16-byte aligned rows
// (8-byte for fp16 output). NC float4 per lane (d <= 256 NC). Every load of the
// row -- x, and gamma / beta -- issues at the start as buffer loads whose range
// is the row (chunks past d read as zeros: no branch, no access), so a wave
// waits out one memory round trip; gamma / beta loaded after the reductions,
// chunk by chunk, had cost a round trip per chunk.
template <typename TO, int NC>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, TO* __restrict__ y,
                                                            uint32_t rows, uint32_t d, float eps) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const uint32_t n4 = d / 4;
    const int nbytes = static_cast<int>(d * 4);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + static_cast<uint64_t>(row) * d), 0, nbytes, 0x00020000);
    TO* yr = y + static_cast<uint64_t>(row) * d;
    floatx4 c[NC], g[NC], b[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i)
        c[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rx, (lane + 64 * i) * 16, 0, 0));
    if (gamma) {
        const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(gamma), 0, nbytes,
                                                                            0x00020000);
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(beta), 0, nbytes,
                                                                            0x00020000);
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            g[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rg, (lane + 64 * i) * 16, 0, 0));
            b[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rb, (lane + 64 * i) * 16, 0, 0));
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) s += (c[i][0] + c[i][1]) + (c[i][2] + c[i][3]);
    const float mean = wave_sum_dpp(s) / static_cast<float>(d);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const uint32_t j = lane + 64 * i;
        if (j < n4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float dv = c[i][e] - mean;
                ss += dv * dv;
            }
        }
    }
    const float var = wave_sum_dpp(ss) / static_cast<float>(d);
    const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const uint32_t j = lane + 64 * i;
        if (j < n4) {
            floatx4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (c[i][e] - mean) * inv;
            if (gamma) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = v[e] * g[i][e] + b[i][e];
            }
            store4(yr + 4 * j, v);
        }
    }
}

// General rows (any d, any alignment): one wave per row, three passes over memory.
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, float* __restrict__ y,
                                                        uint32_t rows, uint32_t d, float eps) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + static_cast<uint64_t>(row) * d;
    float* yr = y + static_cast<uint64_t>(row) * d;
    float s = 0.0f;
    for (uint32_t j = lane; j < d; j += 64) s += xr[j];
    const float mean = wave_sum(s) / static_cast<float>(d);
    float ss = 0.0f;
    for (uint32_t j = lane; j < d; j += 64) {
        const float dv = xr[j] - mean;
        ss += dv * dv;
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(d) + eps);
    for (uint32_t j = lane; j < d; j += 64) {
        float v = (xr[j] - mean) * inv;
        if (gamma) v = v * gamma[j] + beta[j];
        yr[j] = v;
    }
}

// y[r, j] = h[r, j] * gelu(h[r, F + j]); F % 4 == 0 and 16-byte aligned rows
// (8-byte for fp16 y). Thread (x, y) of the grid takes float4 column
// blockIdx.x * 256 + tid of rows blockIdx.y, blockIdx.y + gridDim.y, ... (no
// index division per element).
template <typename TO>
__global__ __launch_bounds__(256) void geglu_vec_kernel(const float* __restrict__ h, TO* __restrict__ y, uint32_t rows,
                                                        uint32_t F) {
    const uint32_t f4 = F / 4;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= f4) return;
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const floatx4* hr = reinterpret_cast<const floatx4*>(h + static_cast<uint64_t>(r) * 2 * F);
        const floatx4 a = hr[j], b = hr[f4 + j];
        floatx4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = a[e] * gelu_erf(b[e]);
        store4(y + static_cast<uint64_t>(r) * F + 4 * j, o);
    }
}

__global__ __launch_bounds__(256) void geglu_kernel(const float* __restrict__ h, float* __restrict__ y, uint32_t rows,
                                                    uint32_t F) {
    const uint64_t total = static_cast<uint64_t>(rows) * F;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint64_t r = i / F, j = i % F;
        y[i] = h[r * 2 * F + j] * gelu_erf(h[r * 2 * F + F + j]);
    }
}

__global__ __launch_bounds__(256) void add_vec_kernel(floatx4* __restrict__ x, const floatx4* __restrict__ a, uint64_t n4) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n4; i += static_cast<uint64_t>(gridDim.x) * 256) {
        floatx4 v = x[i];
        const floatx4 w = a[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += w[e];
        x[i] = v;
    }
}

__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ x, const float* __restrict__ a, uint64_t n) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += static_cast<uint64_t>(gridDim.x) * 256) x[i] += a[i];
}

// Grid for a grid-stride elementwise kernel: enough workgroups to cover the
// work, capped at 8 per CU.
unsigned stride_grid(uint64_t items) {
    const uint64_t g = (items + 255) / 256;
    return static_cast<unsigned>(g < 2048 ? (g ? g : 1) : 2048);
}

// The vector LayerNorm with the fewest float4 per lane that hold a row of d.
template <typename TO>
void launch_layernorm_vec(const float* x, const float* gamma, const float* beta, TO* y, uint32_t rows, uint32_t d,
                          float eps, hipStream_t s) {
    const unsigned grid = ceil_div(rows, 4);
    const uint32_t nc = ceil_div(d / 4, 64u);
    if (nc <= 2) layernorm_vec_kernel<TO, 2><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, d, eps);
    else if (nc <= 3) layernorm_vec_kernel<TO, 3><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, d, eps);
    else if (nc <= 5) layernorm_vec_kernel<TO, 5><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, d, eps);
    else if (nc <= 8) layernorm_vec_kernel<TO, 8><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, d, eps);
    else layernorm_vec_kernel<TO, kLnCache><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, d, eps);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_layernorm(const float* x, const float* gamma, const float* beta, float* y, uint32_t rows, uint32_t d,
                            float eps, void* stream) {
    const char* fn = "mi_layernorm";
    if (!x || !y) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if ((gamma == nullptr) != (beta == nullptr)) return fail(MI_ERR_INVALID_ARG, "%s: gamma and beta go together", fn);
    if (rows == 0) return MI_OK;
    if (d == 0) return fail(MI_ERR_INVALID_ARG, "%s: d == 0", fn);
    const uint64_t bytes = static_cast<uint64_t>(rows) * d * 4;
    if (x != y && overlaps(x, bytes, y, bytes)) return fail(MI_ERR_ALIASING, "%s: y partially overlaps x", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = d % 4 == 0 && d <= 64u * 4 * kLnCache && aligned(x, 16) && aligned(y, 16) &&
                     (!gamma || (aligned(gamma, 16) && aligned(beta, 16)));
    if (vec) launch_layernorm_vec<float>(x, gamma, beta, y, rows, d, eps, s);
    else layernorm_kernel<<<ceil_div(rows, 4), 256, 0, s>>>(x, gamma, beta, y, rows, d, eps);
    return check_launch(fn);
}

extern "C" int mi_geglu(const float* h, float* y, uint32_t rows, uint32_t F, void* stream) {
    const char* fn = "mi_geglu";
    if (!h || !y) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (rows == 0 || F == 0) return MI_OK;
    if (overlaps(h, static_cast<uint64_t>(rows) * 2 * F * 4, y, static_cast<uint64_t>(rows) * F * 4))
        return fail(MI_ERR_ALIASING, "%s: y overlaps h", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (F % 4 == 0 && aligned(h, 16) && aligned(y, 16)) {
        // ~2048 workgroups in all: the rows are strided over grid.y
        const unsigned gx = ceil_div(F / 4, 256);
        const unsigned gy = static_cast<unsigned>(std::min<uint64_t>(rows, std::max<uint64_t>(1, 2048 / gx)));
        geglu_vec_kernel<float><<<dim3(gx, gy), 256, 0, s>>>(h, y, rows, F);
    }
    else
        geglu_kernel<<<stride_grid(static_cast<uint64_t>(rows) * F), 256, 0, s>>>(h, y, rows, F);
    return check_launch(fn);
}

extern "C" int mi_layernorm_f16(const float* x, const float* gamma, const float* beta, void* y, uint32_t rows,
                                uint32_t d, float eps, void* stream) {
    const char* fn = "mi_layernorm_f16";
    if (!x || !y) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if ((gamma == nullptr) != (beta == nullptr)) return fail(MI_ERR_INVALID_ARG, "%s: gamma and beta go together", fn);
    if (rows == 0) return MI_OK;
    if (d == 0 || d % 4 || d > 64u * 4 * kLnCache)
        return fail(MI_ERR_UNSUPPORTED, "%s: d=%u (a multiple of 4, at most %u)", fn, d, 64u * 4 * kLnCache);
    if (!aligned(x, 16) || !aligned(y, 8) || (gamma && (!aligned(gamma, 16) || !aligned(beta, 16))))
        return fail(MI_ERR_ALIGNMENT, "%s: x, gamma, beta 16-byte and y 8-byte aligned", fn);
    if (overlaps(x, static_cast<uint64_t>(rows) * d * 4, y, static_cast<uint64_t>(rows) * d * 2))
        return fail(MI_ERR_ALIASING, "%s: y overlaps x", fn);
    launch_layernorm_vec<_Float16>(x, gamma, beta, static_cast<_Float16*>(y), rows, d, eps,
                                   static_cast<hipStream_t>(stream));
    return check_launch(fn);
}

extern "C" int mi_geglu_f16(const float* h, void* y, uint32_t rows, uint32_t F, void* stream) {
    const char* fn = "mi_geglu_f16";
    if (!h || !y) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (rows == 0 || F == 0) return MI_OK;
    if (F % 4) return fail(MI_ERR_UNSUPPORTED, "%s: F=%u is not a multiple of 4", fn, F);
    if (!aligned(h, 16) || !aligned(y, 8)) return fail(MI_ERR_ALIGNMENT, "%s: h 16-byte and y 8-byte aligned", fn);
    if (overlaps(h, static_cast<uint64_t>(rows) * 2 * F * 4, y, static_cast<uint64_t>(rows) * F * 2))
        return fail(MI_ERR_ALIASING, "%s: y overlaps h", fn);
    const unsigned gx = ceil_div(F / 4, 256);
    const unsigned gy = static_cast<unsigned>(std::min<uint64_t>(rows, std::max<uint64_t>(1, 2048 / gx)));
    geglu_vec_kernel<_Float16><<<dim3(gx, gy), 256, 0, static_cast<hipStream_t>(stream)>>>(
        h, static_cast<_Float16*>(y), rows, F);
    return check_launch(fn);
}

extern "C" int mi_add_inplace(float* x, const float* a, uint64_t n, void* stream) {
    const char* fn = "mi_add_inplace";
    if (!x || !a) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (n == 0) return MI_OK;
    if (x != a && overlaps(x, n * 4, a, n * 4)) return fail(MI_ERR_ALIASING, "%s: a partially overlaps x", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n % 4 == 0 && aligned(x, 16) && aligned(a, 16))
        add_vec_kernel<<<stride_grid(n / 4), 256, 0, s>>>(reinterpret_cast<floatx4*>(x),
                                                           reinterpret_cast<const floatx4*>(a), n / 4);
    else
        add_kernel<<<stride_grid(n), 256, 0, s>>>(x, a, n);
    return check_launch(fn);
}
