// gemm_q8.hip -- Q8_0 NT GEMM for gfx950:  C[M,N] (=|+=) A[M,K] . deq(W[N,K])^T (+bias)
//
// Reference behaviour: src/Modules/GPU/shaders/gemm_nt_q8_v.comp (mode / bias /
// lda / ldc / batch semantics :37-54,115-127) and gemm_nt_q8.comp; host routing
// sdvkgen.cpp:917-936. The algorithm here is our own:
//
//   * one workgroup computes a BM x BN tile of C; the K loop advances one Q8_0
//     block column (32 k) per step, so every step sees exactly one scale per
//     weight row;
//   * A (fp32) is streamed with coalesced 16-byte loads, rounded to fp16 and
//     written to LDS; the weight block is streamed (34-byte GGUF blocks or the
//     reference's split int8 + fp32-scale planes), dequantised to fp16
//     (w = d * q, rounded once) and written to LDS;
//   * waves multiply LDS fragments with v_mfma_f32_32x32x16_f16 (fp32
//     accumulation); the next step's global loads are in flight while the
//     current step's MFMAs run (register prefetch + two LDS stages, one
//     barrier per step);
//   * workgroup ids are remapped so the tiles of one A row-panel run on one
//     XCD and share its L2.
#include "common.hpp"

namespace mi {
namespace {

constexpr int kLdk = 40;  // LDS row stride in halves: 32 k + 8 pad (80 B, conflict-free 16-B reads)

struct GemmArgs {
    const float* A;
    const uint8_t* W;       // 34-byte blocks, or the split int8 payload
    const float* scales;    // split layout only
    const float* bias;
    float* C;
    uint32_t M, N, K, mode, lda, ldc;
    uint64_t sA, sC;
    uint32_t tiles_n;       // ceil(N / BN)
    uint32_t ksteps;        // ceil(K / 32)
};

// ---- weight loaders: 8 consecutive k of one weight row per thread ---------------

enum WKind { kBlocks34 = 0, kSplit = 1 };

struct WRaw {
    uint32_t lo, hi;  // 8 int8 weights, little-endian
    float s0, s1;     // scale of weights 0-3 and 4-7
};

// 34-byte blocks: row n, block kb starts at byte (n*K/32 + kb)*34; the 8 q bytes
// for group j sit at +2+8j, which is 2-byte aligned: read the covering aligned
// dwords and funnel-shift.
__device__ __forceinline__ WRaw load_w_blocks(const GemmArgs& a, uint32_t n, uint32_t kb, uint32_t j) {
    WRaw r;
    uint64_t blk = (static_cast<uint64_t>(n) * (a.K >> 5) + kb) * 34u;
    float d = fp16_bits_to_f32(*reinterpret_cast<const uint16_t*>(a.W + blk));
    uint64_t addr = blk + 2u + 8u * j;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(a.W + (addr & ~uint64_t(3)));
    uint32_t w0 = p[0], w1 = p[1];
    if (addr & 2u) {
        uint32_t w2 = p[2];
        r.lo = __builtin_amdgcn_alignbit(w1, w0, 16);
        r.hi = __builtin_amdgcn_alignbit(w2, w1, 16);
    } else {
        r.lo = w0;
        r.hi = w1;
    }
    r.s0 = d;
    r.s1 = d;
    return r;
}

// Split layout: flat element f = n*K + k, int8 at byte f, scale at f >> 5.
// K % 4 == 0, so each 4-group shares a scale; weights at k >= K are zero.
__device__ __forceinline__ WRaw load_w_split(const GemmArgs& a, uint32_t n, uint32_t kb, uint32_t j) {
    WRaw r{0u, 0u, 0.0f, 0.0f};
    uint32_t k = kb * 32u + 8u * j;
    if (k >= a.K) return r;
    uint64_t f = static_cast<uint64_t>(n) * a.K + k;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(a.W);
    r.lo = p[f >> 2];
    r.s0 = a.scales[f >> 5];
    if (k + 4u < a.K) {
        r.hi = p[(f >> 2) + 1u];
        r.s1 = a.scales[(f + 4u) >> 5];
    }
    return r;
}

__device__ __forceinline__ half8 dequant8(const WRaw& r) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((r.lo >> (8 * i)) & 0xffu)) * r.s0);
        h[4 + i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((r.hi >> (8 * i)) & 0xffu)) * r.s1);
    }
    return h;
}

// ---- the kernel ---------------------------------------------------------------------

template <int BM, int BN, int WM, int WN, int WK>
__global__ __launch_bounds__(WM * WN * 64) void gemm_q8_kernel(GemmArgs a) {
    constexpr int NT = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;     // wave tile
    constexpr int FM = TM / 32, FN = TN / 32;     // 32x32 MFMA tiles per wave
    constexpr int A_IT = BM * 8 / NT;             // float4 loads per thread per step
    constexpr int W_UNITS = BN * 4;               // (row, 8-k group) units per step
    constexpr int W_IT = (W_UNITS + NT - 1) / NT;
    static_assert(BM * 8 % NT == 0, "A staging must divide evenly");
    static_assert(FM >= 1 && FN >= 1, "wave tile below 32x32");

    __shared__ _Float16 As[2][BM * kLdk];
    __shared__ _Float16 Ws[2][BN * kLdk];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int wm = wave % WM, wn = wave / WM;

    const unsigned tile = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t m0 = (tile / a.tiles_n) * BM;
    const uint32_t n0 = (tile % a.tiles_n) * BN;
    const float* A = a.A + static_cast<uint64_t>(blockIdx.z) * a.sA;
    float* C = a.C + static_cast<uint64_t>(blockIdx.z) * a.sC;

    floatx4 areg[A_IT];
    WRaw wreg[W_IT];

    auto load_step = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < A_IT; ++i) {
            int f = tid + i * NT;
            uint32_t row = m0 + (f >> 3);
            uint32_t k = kb * 32u + (f & 7) * 4u;
            floatx4 v = {0.f, 0.f, 0.f, 0.f};
            if (row < a.M && k < a.K) v = *reinterpret_cast<const floatx4*>(A + static_cast<uint64_t>(row) * a.lda + k);
            areg[i] = v;
        }
#pragma unroll
        for (int i = 0; i < W_IT; ++i) {
            int u = tid + i * NT;
            uint32_t n = n0 + (u >> 2);
            WRaw r{0u, 0u, 0.0f, 0.0f};
            if (u < W_UNITS && n < a.N) {
                if constexpr (WK == kBlocks34) r = load_w_blocks(a, n, kb, u & 3);
                else r = load_w_split(a, n, kb, u & 3);
            }
            wreg[i] = r;
        }
    };
    auto store_step = [&](int st) {
#pragma unroll
        for (int i = 0; i < A_IT; ++i) {
            int f = tid + i * NT;
            half4 h;
            h[0] = static_cast<_Float16>(areg[i][0]);
            h[1] = static_cast<_Float16>(areg[i][1]);
            h[2] = static_cast<_Float16>(areg[i][2]);
            h[3] = static_cast<_Float16>(areg[i][3]);
            *reinterpret_cast<half4*>(&As[st][(f >> 3) * kLdk + (f & 7) * 4]) = h;
        }
#pragma unroll
        for (int i = 0; i < W_IT; ++i) {
            int u = tid + i * NT;
            if (u < W_UNITS) *reinterpret_cast<half8*>(&Ws[st][(u >> 2) * kLdk + (u & 3) * 8]) = dequant8(wreg[i]);
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (a.ksteps > 0) {
        load_step(0);
        store_step(0);
    }
    __syncthreads();

    for (uint32_t kb = 0; kb < a.ksteps; ++kb) {
        const int st = kb & 1;
        const bool more = kb + 1 < a.ksteps;
        if (more) load_step(kb + 1);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            half8 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const half8*>(&As[st][(wm * TM + 32 * i + l32) * kLdk + 16 * s + 8 * g]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&Ws[st][(wn * TN + 32 * j + l32) * kLdk + 16 * s + 8 * g]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) store_step(st ^ 1);
        __syncthreads();
    }

    // Epilogue. Lane holds column l32 of each 32x32 tile and rows 8(r/4) + 4g + r%4.
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const uint32_t n = n0 + wn * TN + 32 * j + l32;
        if (n >= a.N) continue;
        const float bv = (a.mode == 0 && a.bias) ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * TM + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (m >= a.M) continue;
                float* c = C + static_cast<uint64_t>(m) * a.ldc + n;
                if (a.mode == 0) *c = acc[i][j][r] + bv;
                else *c += acc[i][j][r];
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int WK>
void launch(const GemmArgs& a0, uint32_t batch, hipStream_t s) {
    GemmArgs a = a0;
    a.tiles_n = ceil_div(a.N, BN);
    unsigned tiles = ceil_div(a.M, BM) * a.tiles_n;
    gemm_q8_kernel<BM, BN, WM, WN, WK><<<dim3(tiles, 1, batch), WM * WN * 64, 0, s>>>(a);
}

// Tile configuration by problem size. Large M: 256x128 tiles (8 waves, 64x64
// each); small M (cross-attention K/V projections, M = 2 x 77): 64x64 tiles.
template <int WK>
void dispatch(const GemmArgs& a, uint32_t batch, hipStream_t s) {
    if (a.M >= 1024) launch<256, 128, 4, 2, WK>(a, batch, s);
    else launch<64, 64, 2, 2, WK>(a, batch, s);
}

int validate(const char* fn, const float* A, const void* W, const float* C, uint32_t M, uint32_t N, uint32_t K,
             uint32_t mode, uint32_t& lda, uint32_t& ldc, uint32_t batch, uint64_t sA, uint64_t sC) {
    if (!A || !W || !C) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (mode > 1) return fail(MI_ERR_INVALID_ARG, "%s: mode %u (0 = store, 1 = accumulate)", fn, mode);
    if (batch == 0) return fail(MI_ERR_INVALID_ARG, "%s: batch 0", fn);
    if (batch > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: batch %u > 65535", fn, batch);
    if (lda == 0) lda = K;
    if (ldc == 0) ldc = N;
    if (lda < K || ldc < N) return fail(MI_ERR_INVALID_ARG, "%s: lda %u < K %u or ldc %u < N %u", fn, lda, K, ldc, N);
    if (!aligned(A, 16) || lda % 4 || sA % 4) return fail(MI_ERR_ALIGNMENT, "%s: A must be 16-byte aligned, lda and sA multiples of 4", fn);
    if (!aligned(C, 4)) return fail(MI_ERR_ALIGNMENT, "%s: C must be 4-byte aligned", fn);
    if (static_cast<uint64_t>(M) * N > (uint64_t(1) << 40)) return fail(MI_ERR_UNSUPPORTED, "%s: M*N too large", fn);
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_gemm_nt_q8_0(const float* A, const void* W, const float* bias, float* C, uint32_t M, uint32_t N,
                               uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA,
                               uint64_t sC, void* stream) {
    const char* fn = "mi_gemm_nt_q8_0";
    if (M == 0 || N == 0) return MI_OK;
    if (K % 32) return fail(MI_ERR_UNSUPPORTED, "%s: K=%u is not a multiple of 32 (Q8_0 block)", fn, K);
    int st = validate(fn, A, W, C, M, N, K, mode, lda, ldc, batch, sA, sC);
    if (st) return st;
    if (!aligned(W, 16)) return fail(MI_ERR_ALIGNMENT, "%s: W must be 16-byte aligned", fn);
    uint64_t cbytes = (static_cast<uint64_t>(batch - 1) * sC + static_cast<uint64_t>(M - 1) * ldc + N) * 4;
    uint64_t abytes = (static_cast<uint64_t>(batch - 1) * sA + static_cast<uint64_t>(M - 1) * lda + K) * 4;
    uint64_t wbytes = static_cast<uint64_t>(N) * (K / 32) * 34;
    if (overlaps(C, cbytes, A, abytes) || overlaps(C, cbytes, W, wbytes) || overlaps(C, cbytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: C overlaps an input", fn);
    GemmArgs a{A, static_cast<const uint8_t*>(W), nullptr, bias, C, M, N, K, mode, lda, ldc, sA, sC, 0, K / 32};
    dispatch<kBlocks34>(a, batch, static_cast<hipStream_t>(stream));
    return check_launch(fn);
}

extern "C" int mi_gemm_nt_q8_split(const float* A, const uint32_t* payload, const float* scales, const float* bias,
                                   float* C, uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda,
                                   uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sC, void* stream) {
    const char* fn = "mi_gemm_nt_q8_split";
    if (M == 0 || N == 0) return MI_OK;
    if (K % 4) return fail(MI_ERR_UNSUPPORTED, "%s: K=%u is not a multiple of 4", fn, K);
    int st = validate(fn, A, payload, C, M, N, K, mode, lda, ldc, batch, sA, sC);
    if (st) return st;
    if (!scales) return fail(MI_ERR_INVALID_ARG, "%s: null scales", fn);
    if (!aligned(payload, 4) || !aligned(scales, 4)) return fail(MI_ERR_ALIGNMENT, "%s: payload/scales alignment", fn);
    uint64_t cbytes = (static_cast<uint64_t>(batch - 1) * sC + static_cast<uint64_t>(M - 1) * ldc + N) * 4;
    uint64_t abytes = (static_cast<uint64_t>(batch - 1) * sA + static_cast<uint64_t>(M - 1) * lda + K) * 4;
    uint64_t nk = static_cast<uint64_t>(N) * K;
    if (overlaps(C, cbytes, A, abytes) || overlaps(C, cbytes, payload, nk) ||
        overlaps(C, cbytes, scales, (nk + 31) / 32 * 4) || overlaps(C, cbytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: C overlaps an input", fn);
    GemmArgs a{A, reinterpret_cast<const uint8_t*>(payload), scales, bias, C, M, N, K, mode, lda, ldc, sA, sC, 0,
               (K + 31) / 32};
    dispatch<kSplit>(a, batch, static_cast<hipStream_t>(stream));
    return check_launch(fn);
}
