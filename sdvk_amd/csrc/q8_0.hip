// q8_0.hip -- GGUF Q8_0 block decode on the GPU.
//
//   mi_q8_0_dequant      34-byte blocks -> fp32 (bit-exact, Gguf.cpp:514-523) / fp16
//   mi_q8_split_dequant  split payload + fp32 scales -> fp32 / fp16 (gemm_nt_q8_v.comp:37-43)
//   mi_q8_0_to_split     34-byte blocks -> split layout (Gguf.cpp:559-583 readQ8Into)
//
// All three are HBM-bound streams: one thread per 8 elements (a quarter block)
// for the block formats, one per packed payload word for the split format.
#include "common.hpp"

namespace mi {
namespace {

// The 8 q bytes at byte offset `o` (2-byte aligned) of a block stream, read as
// 16-bit halves (the stream has no stronger alignment: blocks are 34 bytes).
__device__ __forceinline__ void load_q8(const uint8_t* base, uint64_t o, uint32_t& lo, uint32_t& hi) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(base + o);
    lo = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 16);
    hi = static_cast<uint32_t>(p[2]) | (static_cast<uint32_t>(p[3]) << 16);
}

__device__ __forceinline__ float sbyte(uint32_t w, int i) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * i)) & 0xffu));
}

template <typename TO>
__global__ __launch_bounds__(256) void q8_0_dequant_kernel(const uint8_t* __restrict__ blocks,
                                                           TO* __restrict__ out, uint64_t groups) {
    uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    uint64_t blk = g >> 2;
    uint32_t j = static_cast<uint32_t>(g & 3u);
    const uint8_t* b = blocks + blk * 34u;
    float d = fp16_bits_to_f32(*reinterpret_cast<const uint16_t*>(b));
    uint32_t lo, hi;
    load_q8(b, 2u + 8u * j, lo, hi);
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = d * sbyte(lo, i);
        v[4 + i] = d * sbyte(hi, i);
    }
    if constexpr (sizeof(TO) == 4) {
        floatx4* o = reinterpret_cast<floatx4*>(out + g * 8u);
        o[0] = floatx4{v[0], v[1], v[2], v[3]};
        o[1] = floatx4{v[4], v[5], v[6], v[7]};
    } else {
        half8 h;
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(v[i]);
        *reinterpret_cast<half8*>(out + g * 8u) = h;
    }
}

template <typename TO>
__global__ __launch_bounds__(256) void q8_split_dequant_kernel(const uint32_t* __restrict__ payload,
                                                               const float* __restrict__ scales,
                                                               TO* __restrict__ out, uint64_t words) {
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= words) return;
    uint32_t w = payload[i];
    float s = scales[i >> 3];  // 4 elements per word, 32 per scale
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = sbyte(w, k) * s;
    if constexpr (sizeof(TO) == 4) {
        *reinterpret_cast<floatx4*>(out + i * 4u) = floatx4{v[0], v[1], v[2], v[3]};
    } else {
        half4 h;
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = static_cast<_Float16>(v[k]);
        *reinterpret_cast<half4*>(out + i * 4u) = h;
    }
}

__global__ __launch_bounds__(256) void q8_0_to_split_kernel(const uint8_t* __restrict__ blocks,
                                                            uint32_t* __restrict__ payload,
                                                            float* __restrict__ scales, uint64_t groups) {
    uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    uint64_t blk = g >> 2;
    uint32_t j = static_cast<uint32_t>(g & 3u);
    const uint8_t* b = blocks + blk * 34u;
    uint32_t lo, hi;
    load_q8(b, 2u + 8u * j, lo, hi);
    payload[g * 2u] = lo;
    payload[g * 2u + 1u] = hi;
    if (j == 0) scales[blk] = fp16_bits_to_f32(*reinterpret_cast<const uint16_t*>(b));
}

constexpr uint64_t kMaxElems = uint64_t(1) << 40;

// Quantizer (sdvkgen.cpp:533-544, the reference's requantization rule): per
// block of 32, amax = max |w|, d = fp16(amax / 127), q = clamp(trunc(w * 127 /
// amax +- 0.5), -127, 127); an all-zero block gives d = 0, q = 0. One thread
// per block. Contraction stays off so that w * inv + 0.5 rounds twice, as in
// the reference's scalar code.
__global__ __launch_bounds__(256) void q8_0_quantize_kernel(const float* __restrict__ w, uint8_t* __restrict__ blocks,
                                                            uint64_t nblocks) {
#pragma clang fp contract(off)
    const uint64_t b = blockIdx.x * 256ull + threadIdx.x;
    if (b >= nblocks) return;
    const float* x = w + b * 32;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        v[i] = x[i];
        amax = fmaxf(amax, fabsf(v[i]));
    }
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    const _Float16 d = static_cast<_Float16>(amax > 0.0f ? amax / 127.0f : 0.0f);
    uint16_t* out = reinterpret_cast<uint16_t*>(blocks + b * 34);
    out[0] = __builtin_bit_cast(uint16_t, d);
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        int q[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float t = v[i + e] * inv;
            int r = static_cast<int>(t + (t >= 0.0f ? 0.5f : -0.5f));
            q[e] = r < -127 ? -127 : (r > 127 ? 127 : r);
        }
        out[1 + i / 2] = static_cast<uint16_t>((q[0] & 0xff) | ((q[1] & 0xff) << 8));
    }
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_q8_0_dequant(const void* blocks, void* out, int out_dtype, uint64_t n, void* stream) {
    if (n == 0) return MI_OK;
    if (!blocks || !out) return fail(MI_ERR_INVALID_ARG, "mi_q8_0_dequant: null pointer");
    if (out_dtype != MI_F32 && out_dtype != MI_F16)
        return fail(MI_ERR_INVALID_ARG, "mi_q8_0_dequant: out_dtype %d", out_dtype);
    if (n % 32 || n > kMaxElems) return fail(MI_ERR_UNSUPPORTED, "mi_q8_0_dequant: n=%llu is not a multiple of 32",
                                             (unsigned long long)n);
    if (!aligned(blocks, 2) || !aligned(out, 16)) return fail(MI_ERR_ALIGNMENT, "mi_q8_0_dequant: alignment");
    uint64_t esz = out_dtype == MI_F32 ? 4 : 2;
    if (overlaps(blocks, n / 32 * 34, out, n * esz)) return fail(MI_ERR_ALIASING, "mi_q8_0_dequant: out overlaps blocks");
    uint64_t groups = n / 8;
    dim3 grid(ceil_div(groups, 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (out_dtype == MI_F32)
        q8_0_dequant_kernel<float><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(blocks), static_cast<float*>(out), groups);
    else
        q8_0_dequant_kernel<_Float16><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(blocks), static_cast<_Float16*>(out), groups);
    return check_launch("mi_q8_0_dequant");
}

extern "C" int mi_q8_split_dequant(const uint32_t* payload, const float* scales, void* out, int out_dtype,
                                   uint64_t n, void* stream) {
    if (n == 0) return MI_OK;
    if (!payload || !scales || !out) return fail(MI_ERR_INVALID_ARG, "mi_q8_split_dequant: null pointer");
    if (out_dtype != MI_F32 && out_dtype != MI_F16)
        return fail(MI_ERR_INVALID_ARG, "mi_q8_split_dequant: out_dtype %d", out_dtype);
    if (n % 4 || n > kMaxElems) return fail(MI_ERR_UNSUPPORTED, "mi_q8_split_dequant: n=%llu is not a multiple of 4",
                                            (unsigned long long)n);
    if (!aligned(payload, 4) || !aligned(scales, 4) || !aligned(out, 16))
        return fail(MI_ERR_ALIGNMENT, "mi_q8_split_dequant: alignment");
    uint64_t esz = out_dtype == MI_F32 ? 4 : 2;
    if (overlaps(payload, n, out, n * esz) || overlaps(scales, (n + 31) / 32 * 4, out, n * esz))
        return fail(MI_ERR_ALIASING, "mi_q8_split_dequant: out overlaps an input");
    uint64_t words = n / 4;
    dim3 grid(ceil_div(words, 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (out_dtype == MI_F32)
        q8_split_dequant_kernel<float><<<grid, 256, 0, s>>>(payload, scales, static_cast<float*>(out), words);
    else
        q8_split_dequant_kernel<_Float16><<<grid, 256, 0, s>>>(payload, scales, static_cast<_Float16*>(out), words);
    return check_launch("mi_q8_split_dequant");
}

extern "C" int mi_q8_0_to_split(const void* blocks, uint32_t* payload, float* scales, uint64_t n, void* stream) {
    if (n == 0) return MI_OK;
    if (!blocks || !payload || !scales) return fail(MI_ERR_INVALID_ARG, "mi_q8_0_to_split: null pointer");
    if (n % 32 || n > kMaxElems) return fail(MI_ERR_UNSUPPORTED, "mi_q8_0_to_split: n=%llu is not a multiple of 32",
                                             (unsigned long long)n);
    if (!aligned(blocks, 2) || !aligned(payload, 4) || !aligned(scales, 4))
        return fail(MI_ERR_ALIGNMENT, "mi_q8_0_to_split: alignment");
    if (overlaps(blocks, n / 32 * 34, payload, n) || overlaps(blocks, n / 32 * 34, scales, n / 32 * 4) ||
        overlaps(payload, n, scales, n / 32 * 4))
        return fail(MI_ERR_ALIASING, "mi_q8_0_to_split: buffers overlap");
    uint64_t groups = n / 8;
    q8_0_to_split_kernel<<<dim3(ceil_div(groups, 256)), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint8_t*>(blocks), payload, scales, groups);
    return check_launch("mi_q8_0_to_split");
}

extern "C" int mi_q8_0_quantize(const float* w, void* blocks, uint64_t n, void* stream) {
    if (n == 0) return MI_OK;
    if (!w || !blocks) return fail(MI_ERR_INVALID_ARG, "mi_q8_0_quantize: null pointer");
    if (n % 32 || n > kMaxElems)
        return fail(MI_ERR_UNSUPPORTED, "mi_q8_0_quantize: n=%llu is not a multiple of 32", (unsigned long long)n);
    if (!aligned(w, 4) || !aligned(blocks, 2)) return fail(MI_ERR_ALIGNMENT, "mi_q8_0_quantize: alignment");
    if (overlaps(w, n * 4, blocks, n / 32 * 34)) return fail(MI_ERR_ALIASING, "mi_q8_0_quantize: blocks overlap w");
    const uint64_t nb = n / 32;
    q8_0_quantize_kernel<<<dim3(ceil_div(nb, 256)), 256, 0, static_cast<hipStream_t>(stream)>>>(
        w, static_cast<uint8_t*>(blocks), nb);
    return check_launch("mi_q8_0_quantize");
}
