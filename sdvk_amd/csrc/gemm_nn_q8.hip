// gemm_nn_q8.hip -- Q8 NN GEMM for gfx950: C[M,N] (=|+=) deq(A[M,K]) . B[K,N]
//
// The weights-left product of sdvk's convolution paths: out[cout, P] =
// W[cout, cin * k * k] . col[cin * k * k, P] after im2col (3x3 convs, the
// stride-2 downsamplers and 1x1 convs; sdvkgen.cpp:944-948,1133-1180).
// Reference behaviour: src/Modules/GPU/shaders/gemm_nn_q8_v.comp: A is the split
// Q8 layout (int8 payload, fp32 scale per 32 FLAT elements: value at flat
// index fl = z*sA + m*lda + k is int8(payload[fl]) * scales[fl >> 5], :23-28,
// 54-64), B fp32 row-major, mode 0 stores / mode 1 accumulates, batch on z
// offsets A, B and C, zero leading dimensions default to K, N, N (:38-40).
//
// This is the first MFMA version (not yet tuned): a workgroup computes a
// 64 x 64 tile of C with four waves of one 32 x 32 v_mfma_f32_32x32x16_f16
// tile each, 32 k per step. W is dequantised to fp16 per 4-element group with
// that group's flat scale (exactly the shader's staging unit), B is rounded to
// fp16 and stored transposed ([n][k]) so both MFMA operands are 8 consecutive
// k per lane. Small LDS (10 KB) and registers let eight workgroups share a CU,
// which hides the unpipelined load -> store -> barrier -> MFMA sequence.
// Every global access goes through a buffer resource whose range is exactly
// the operand's extent: a read outside it returns zeros and a write outside
// it is dropped.
#include "common.hpp"

namespace mi {
namespace {

struct NnArgs {
    const uint8_t* Aq;
    const float* S;
    const float* B;
    float* C;
    uint32_t M, N, K, mode, lda, ldb, ldc;
    uint32_t sA, sB, sC;                      // batch strides (elements), < 2^31 by validation
    uint32_t a_bytes, s_bytes, b_bytes, c_bytes;  // whole-buffer extents
};

constexpr int kTM = 64, kTN = 64, kTK = 32;
constexpr int kLd = kTK + 8;  // LDS row stride in halves (16-byte pad)

__global__ __launch_bounds__(256) void gemm_nn_q8_kernel(NnArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 As[kTM * kLd];  // [m][k]
    __shared__ __attribute__((aligned(16))) _Float16 Bs[kTN * kLd];  // [n][k]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t m0 = blockIdx.y * kTM, n0 = blockIdx.x * kTN, z = blockIdx.z;

    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.Aq), 0, static_cast<int>(a.a_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.S), 0, static_cast<int>(a.s_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rB =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.B), 0, static_cast<int>(a.b_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rC = __builtin_amdgcn_make_buffer_rsrc(a.C, 0, static_cast<int>(a.c_bytes), 0x00020000);

    // staging units: W row wr, k offset wc (two 4-element groups); B k-row br, n offset bc (two float4)
    const uint32_t wr = tid >> 2, wc = (tid & 3) * 8;
    const uint32_t br = tid >> 3, bc = (tid & 7) * 8;
    const uint32_t wm_row = m0 + wr;
    const uint32_t a_row = z * a.sA + wm_row * a.lda;  // flat index of W row wm_row, k = 0
    const uint32_t bn = n0 + bc;

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    for (uint32_t k0 = 0; k0 < a.K; k0 += kTK) {
        // W: two 4-element groups of row wm_row, each with its own flat scale
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t k = k0 + wc + 4 * j;
            half4 h = {0, 0, 0, 0};
            if (wm_row < a.M && k < a.K) {
                const uint32_t fl = a_row + k;
                const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rA, fl, 0, 0);
                const float s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rS, (fl >> 5) * 4, 0, 0));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    h[e] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((w >> (8 * e)) & 0xffu)) * s);
            }
            *reinterpret_cast<half4*>(&As[wr * kLd + wc + 4 * j]) = h;
        }
        // B: two float4 of k-row k0 + br, stored transposed
        {
            const uint32_t k = k0 + br;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t n = bn + 4 * j;
                floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (k < a.K && n < a.N)
                    v = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        rB, (z * a.sB + k * a.ldb + n) * 4, 0, 0));
#pragma unroll
                for (int e = 0; e < 4; ++e) Bs[(bc + 4 * j + e) * kLd + br] = static_cast<_Float16>(v[e]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kTK / 16; ++s) {
            const half8 af = *reinterpret_cast<const half8*>(&As[(wm * 32 + l32) * kLd + 16 * s + 8 * g]);
            const half8 bf = *reinterpret_cast<const half8*>(&Bs[(wn * 32 + l32) * kLd + 16 * s + 8 * g]);
            // D[i][j] = sum_k af(row i)[k] * bf(col j)[k]: i = m, j = n
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
        }
        __syncthreads();
    }

    // lane holds column n = l32 and rows 8 (r / 4) + 4 g + r % 4 of the wave's
    // tile: for each r, 32 lanes write 32 consecutive floats of one row
    const uint32_t n = n0 + wn * 32 + l32;
    if (n >= a.N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t m = m0 + wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m >= a.M) continue;
        const uint32_t off = (z * a.sC + m * a.ldc + n) * 4;
        float v = acc[r];
        if (a.mode != 0) v += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rC, off, 0, 0));
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rC, off, 0, 0);
    }
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_gemm_nn_q8_split(const uint32_t* payload, const float* scales, const float* B, float* C, uint32_t M,
                                   uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb, uint32_t ldc,
                                   uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC, void* stream) {
    const char* fn = "mi_gemm_nn_q8_split";
    if (M == 0 || N == 0) return MI_OK;
    if (!payload || !scales || !B || !C) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (mode > 1) return fail(MI_ERR_INVALID_ARG, "%s: mode %u (0 = store, 1 = accumulate)", fn, mode);
    if (batch == 0) return fail(MI_ERR_INVALID_ARG, "%s: batch 0", fn);
    if (batch > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: batch %u > 65535", fn, batch);
    // the shader stages 4 values at a time and zero-fills a partial group
    // (gemm_nn_q8_v.comp:58,79); such shapes are rejected, not emulated
    if (K % 4 || N % 4) return fail(MI_ERR_UNSUPPORTED, "%s: K=%u and N=%u must be multiples of 4", fn, K, N);
    if (lda == 0) lda = K;
    if (ldb == 0) ldb = N;
    if (ldc == 0) ldc = N;
    if (lda < K || ldb < N || ldc < N)
        return fail(MI_ERR_INVALID_ARG, "%s: lda %u < K %u, ldb %u < N %u or ldc %u < N", fn, lda, K, ldb, N, ldc);
    if (!aligned(payload, 4) || lda % 4 || sA % 4)
        return fail(MI_ERR_ALIGNMENT, "%s: payload must be 4-byte aligned, lda and sA multiples of 4", fn);
    if (!aligned(scales, 4) || !aligned(C, 4)) return fail(MI_ERR_ALIGNMENT, "%s: scales / C alignment", fn);
    if (!aligned(B, 16) || ldb % 4 || sB % 4)
        return fail(MI_ERR_ALIGNMENT, "%s: B must be 16-byte aligned, ldb and sB multiples of 4", fn);
    const uint64_t a_el = static_cast<uint64_t>(batch - 1) * sA + static_cast<uint64_t>(M - 1) * lda + K;
    const uint64_t b_el = static_cast<uint64_t>(batch - 1) * sB + static_cast<uint64_t>(K ? K - 1 : 0) * ldb + N;
    const uint64_t c_el = static_cast<uint64_t>(batch - 1) * sC + static_cast<uint64_t>(M - 1) * ldc + N;
    const uint64_t s_el = (a_el + 31) / 32;
    const uint64_t lim = uint64_t(1) << 31;
    if (a_el >= lim || b_el * 4 >= lim || c_el * 4 >= lim || sA >= lim || sB >= lim || sC >= lim)
        return fail(MI_ERR_UNSUPPORTED, "%s: an operand spans 2 GiB or more", fn);
    if (overlaps(C, c_el * 4, payload, a_el) || overlaps(C, c_el * 4, scales, s_el * 4) ||
        overlaps(C, c_el * 4, B, b_el * 4))
        return fail(MI_ERR_ALIASING, "%s: C overlaps an input", fn);
    if (ceil_div(M, kTM) > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: M=%u too large", fn, M);
    // K == 0 runs the kernel too: no k step, the epilogue stores (mode 0) or adds (mode 1) the empty sum
    NnArgs a{};
    a.Aq = reinterpret_cast<const uint8_t*>(payload);
    a.S = scales;
    a.B = B;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.mode = mode;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.sA = static_cast<uint32_t>(sA);
    a.sB = static_cast<uint32_t>(sB);
    a.sC = static_cast<uint32_t>(sC);
    a.a_bytes = static_cast<uint32_t>(a_el);
    a.s_bytes = static_cast<uint32_t>(s_el * 4);
    a.b_bytes = static_cast<uint32_t>(b_el * 4);
    a.c_bytes = static_cast<uint32_t>(c_el * 4);
    const dim3 grid(ceil_div(N, kTN), ceil_div(M, kTM), batch);
    gemm_nn_q8_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
    return check_launch(fn);
}
