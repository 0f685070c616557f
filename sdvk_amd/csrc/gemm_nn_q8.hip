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
// Two kernels:
//
//   * gemm_nn_q8_tiled_kernel (weights 16-byte aligned with lda, sA multiples
//     of 16, K a multiple of 64: every SDXL conv): 128 x 256 tiles, eight
//     waves of 64 x 64 v_mfma_f32_32x32x16_f16 tiles, 64 k per step, two LDS
//     stages and two register sets in flight (the loads of step j + 2 are
//     issued before step j's MFMAs; step j + 1's dequantisation and B
//     conversion run between them). W is dequantised once per workgroup: 16
//     bytes of one row per thread, which lie inside one 32-element scale block
//     (16-aligned flat index), as fp16(float(q) * s) computed exactly as
//     fma(float(q + 128), s, -128 s). B is read as row-coalesced 16-byte pieces
//     of four k rows and transposed in registers (a 4 x 4 block of k by n per
//     thread) so LDS holds [n][k] and both MFMA operands are 8 consecutive k
//     per lane. With a caller workspace (mi_gemm_nn_q8_split_ws), grids that
//     would leave CUs idle split K: each split stores its partial tile into the
//     workspace and a reduce kernel adds them in split order (fixed, so a call
//     repeats bit for bit).
//   * gemm_nn_q8_kernel (every other shape): 64 x 64 tiles, four waves of one
//     32 x 32 tile, 32 k per step, no software pipelining; W is dequantised per
//     4-element group with that group's flat scale (exactly the shader's
//     staging unit), B is rounded to fp16 and stored transposed ([n][k]).
//
// Every global read goes through a buffer resource whose range is exactly the
// operand's extent with the whole offset in the lane offset: a read outside it
// returns zeros. The general kernel's writes go through such a resource too.
#include "common.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

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
    uint32_t splits, steps_per_split;         // tiled kernel: K splits (blockIdx.z = batch * splits + split)
    uint64_t plane;                           // K splits: floats per partial plane (C = workspace, ldc = N)
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

// ---- tiled kernel --------------------------------------------------------------

constexpr int kBM2 = 128, kBN2 = 256, kBK2 = 64;
constexpr int kLd2 = kBK2 + 8;   // LDS row stride in halves (16-byte pad: conflict-free reads and writes)
constexpr int kNT2 = 512;        // eight waves: 2 (m) x 4 (n), 64 x 64 each
constexpr uint32_t kCUs = 256;

template <bool SPLITK>
__global__ __launch_bounds__(kNT2) void gemm_nn_q8_tiled_kernel(NnArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (kBM2 + kBN2) * kLd2];
    auto Ws = reinterpret_cast<_Float16 (*)[kBM2 * kLd2]>(smem);              // [m][k]
    auto Bs = reinterpret_cast<_Float16 (*)[kBN2 * kLd2]>(smem + 2 * kBM2 * kLd2);  // [n][k]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t n0 = blockIdx.x * kBN2, m0 = blockIdx.y * kBM2;
    // B in LDS: row n holds its 64 k as 16 units of 4 halves, unit u at slot
    // u ^ 2 ((n / 16) % 4). The 8-byte writes of the store phase (32 lanes:
    // 16 quads of n x 2 k blocks) then cover all 64 banks once, and the 16-byte
    // fragment reads (16 consecutive rows, one even unit pair) stay
    // conflict-free and 16-byte aligned.
    auto b_slot = [](uint32_t n, uint32_t u) { return n * kLd2 + 4 * (u ^ (2 * ((n >> 4) & 3))); };
    const uint32_t z = blockIdx.z / a.splits, split = blockIdx.z % a.splits;
    const uint32_t ksteps = a.K / kBK2;
    const uint32_t s_begin = SPLITK ? split * a.steps_per_split : 0;
    const uint32_t s_end = SPLITK ? min(ksteps, s_begin + a.steps_per_split) : ksteps;

    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.Aq), 0, static_cast<int>(a.a_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.S), 0, static_cast<int>(a.s_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rB =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.B), 0, static_cast<int>(a.b_bytes), 0x00020000);

    // W: thread -> row wr, 16 k at wq; flat index of the step's first byte
    // (rows past M read other rows or zeros: they feed outputs never stored)
    const uint32_t wr = tid >> 2, wq = (tid & 3) * 16;
    const uint32_t w_fl = z * a.sA + (m0 + wr) * a.lda + wq;
    // B: thread -> k block kb (4 rows), n quad bq; pass p adds 32 rows. Lane l
    // of wave w takes quad 16 (w / 2) + l % 16 of k block 4 (w % 2) + l / 16, so
    // one load instruction reads 4 whole 256-byte row pieces instead of 8 rows
    // x 128 bytes (a CU's load path costs an instruction by the rows it
    // touches: 18 against 34 cycles per 1 KB in the probe).
    const uint32_t kb = 4 * (wave & 1) + (lane >> 4), bq = 16 * (wave >> 1) + (lane & 15);
    const uint32_t b_el = z * a.sB + (4 * kb) * a.ldb + n0 + 4 * bq;

    uint32_t wraw[2][4];
    float wsc[2];
    floatx4 braw[2][2][4];
    auto load = [&](uint32_t ks_in, auto RS) {
        constexpr int rs = decltype(RS)::value;
        const uint32_t ks = __builtin_amdgcn_readfirstlane(ks_in);
        const uint32_t fl = w_fl + ks * kBK2;
        const auto w = __builtin_amdgcn_raw_buffer_load_b128(rA, fl, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) wraw[rs][e] = w[e];
        wsc[rs] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rS, (fl >> 5) * 4, 0, 0));
        const uint32_t b0 = b_el + ks * kBK2 * a.ldb;
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                braw[rs][p][i] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(rB, (b0 + (32 * p + i) * a.ldb) * 4, 0, 0));
    };
    auto store = [&](auto RS, auto ST) {
        constexpr int rs = decltype(RS)::value;
        constexpr int st = decltype(ST)::value;
        // fp16(float(q) * s) = fp16(fma(float(q + 128), s, -128 s)): one fp32 rounding of the exact product
        const float s = wsc[rs], ms = -128.0f * s;
        half8 h[2];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t u = wraw[rs][e] ^ 0x80808080u;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb)
                h[e >> 1][4 * (e & 1) + bb] =
                    static_cast<_Float16>(__builtin_fmaf(static_cast<float>((u >> (8 * bb)) & 0xffu), s, ms));
        }
        *reinterpret_cast<half8*>(&Ws[st][wr * kLd2 + wq]) = h[0];
        *reinterpret_cast<half8*>(&Ws[st][wr * kLd2 + wq + 8]) = h[1];
        // B: the 4 x 4 block (k rows i, n columns e) goes to LDS rows n as 4 consecutive k
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                *reinterpret_cast<half4*>(&Bs[st][b_slot(4 * bq + e, 8 * p + kb)]) =
                    half4{static_cast<_Float16>(braw[rs][p][0][e]), static_cast<_Float16>(braw[rs][p][1][e]),
                          static_cast<_Float16>(braw[rs][p][2][e]), static_cast<_Float16>(braw[rs][p][3][e])};
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    auto compute = [&](auto ST) {
        constexpr int st = decltype(ST)::value;
#pragma unroll
        for (int s = 0; s < kBK2 / 16; ++s) {
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const half8*>(&Ws[st][(wm * 64 + 32 * i + l32) * kLd2 + 16 * s + 8 * g]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&Bs[st][b_slot(wn * 64 + 32 * j + l32, 4 * s + 2 * g)]);
            // D[i][j] = sum_k af(row i)[k] bf(col j)[k]: i = m, j = n
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    constexpr int kMfma = 2 * 2 * (kBK2 / 16), kRead0 = 4, kReads = 4 * (kBK2 / 16);
    constexpr int kValu = 4 + 16 * 2 + 8 + 16, kWrites = 2 + 8;

    // Step j computes from LDS stage j & 1 while the loads of step j + 2 (into
    // register set j & 1) are in flight and set (j + 1) & 1 is stored; loads
    // past the last step re-read it (unused), so the loop has no load branches.
    const uint32_t n_steps = s_end - s_begin, last = s_end - 1;
    if (n_steps > 0) {
        load(s_begin, S0{});
        store(S0{}, S0{});
        load(min(s_begin + 1, last), S1{});
    }
    __syncthreads();
    uint32_t j = 0;
    for (; j + 2 <= n_steps; j += 2) {
        load(min(s_begin + j + 2, last), S0{});
        __builtin_amdgcn_sched_barrier(0);
        compute(S0{});
        store(S1{}, S1{});
        interleave_step<kMfma, kRead0, kReads - kRead0, kValu, kWrites>();
        __syncthreads();
        load(min(s_begin + j + 3, last), S1{});
        __builtin_amdgcn_sched_barrier(0);
        compute(S1{});
        store(S0{}, S0{});
        interleave_step<kMfma, kRead0, kReads - kRead0, kValu, kWrites>();
        __syncthreads();
    }
    if (j < n_steps) compute(S0{});

    // lane holds column n = l32 and rows 8 (r / 4) + 4 g + r % 4 of each
    // 32 x 32 tile: for each r, 32 lanes cover 32 consecutive floats of a row
    // split K: the split's partial plane of the workspace (row stride ldc = N)
    float* C = a.C + (SPLITK ? (static_cast<uint64_t>(z) * a.splits + split) * a.plane : static_cast<uint64_t>(z) * a.sC);
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
        const uint32_t n = n0 + wn * 64 + 32 * jt + l32;
        if (n >= a.N) continue;
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * 64 + 32 * it + 8 * (r >> 2) + 4 * g + (r & 3);
                if (m >= a.M) continue;
                float* c = C + static_cast<uint64_t>(m) * a.ldc + n;
                if constexpr (SPLITK) *c = acc[it][jt][r];
                else *c = a.mode != 0 ? *c + acc[it][jt][r] : acc[it][jt][r];
            }
    }
}

}  // namespace
}  // namespace mi

using namespace mi;

namespace mi {
namespace {

bool nn_tiled(const uint32_t* payload, uint32_t K, uint32_t lda, uint64_t sA) {
    // mi_tuning_set("nn_kernel", "general"): the untiled kernel for every shape (tests)
    return K > 0 && K % kBK2 == 0 && aligned(payload, 16) && lda % 16 == 0 && sA % 16 == 0 &&
           tuning().nn_general.load(std::memory_order_relaxed) == 0;
}

// K splits of the tiled kernel: one 8-wave workgroup per CU; the most splits
// whose workgroups all run at once (tiles x splits <= CUs), keeping at least
// four 64-wide steps per split. Measured on MI355X against the doubling rule
// (split until the grid covers the CUs): 320x4096x2880 48 tiles x 5 splits
// 33.2 us against x 8 48.6 us; 640x4096x5760 80 x 3 73.9 against x 4 103.7;
// 1280x1024x11520 40 x 6 73.8 against x 8 111.6 (a second partial round of
// workgroups costs a whole round).
uint32_t nn_splits(uint32_t M, uint32_t N, uint32_t K, uint32_t batch) {
    const uint64_t tiles = static_cast<uint64_t>(ceil_div(N, kBN2)) * ceil_div(M, kBM2) * batch;
    const uint32_t ksteps = K / kBK2;
    uint32_t splits = 1;
    const int forced = tuning().nn_splits.load(std::memory_order_relaxed);  // mi_tuning_set("nn_splits")
    if (forced > 0) {
        splits = static_cast<uint32_t>(forced);
        splits = std::min<uint32_t>({splits, std::max(1u, ksteps), 65535u / std::max(1u, batch)});
    } else if (tiles < kCUs) {
        splits = static_cast<uint32_t>(std::min<uint64_t>({kCUs / tiles, ksteps / 4, 65535u / std::max(1u, batch)}));
        splits = std::max(1u, splits);
    }
    if (splits > 1) splits = ceil_div(ksteps, ceil_div(ksteps, splits));
    return splits;
}

int gemm_nn(const char* fn, const uint32_t* payload, const float* scales, const float* B, float* C, uint32_t M,
            uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t batch,
            uint64_t sA, uint64_t sB, uint64_t sC, void* ws, uint64_t ws_bytes, hipStream_t st) {
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
    a.splits = 1;
    if (ws && ws_bytes) {
        if (!aligned(ws, 16)) return fail(MI_ERR_ALIGNMENT, "%s: workspace must be 16-byte aligned", fn);
        if (overlaps(ws, ws_bytes, payload, a_el) || overlaps(ws, ws_bytes, scales, s_el * 4) ||
            overlaps(ws, ws_bytes, B, b_el * 4) || overlaps(ws, ws_bytes, C, c_el * 4))
            return fail(MI_ERR_ALIASING, "%s: workspace overlaps an operand", fn);
    }
    const bool tiled = nn_tiled(payload, K, lda, sA);
    if (!tiled) {
        const dim3 grid(ceil_div(N, kTN), ceil_div(M, kTM), batch);
        gemm_nn_q8_kernel<<<grid, 256, 0, st>>>(a);
        return check_launch(fn);
    }
    const uint32_t ksteps = K / kBK2;
    uint32_t splits = ws ? nn_splits(M, N, K, batch) : 1;
    const uint64_t plane = static_cast<uint64_t>(M) * N;
    if (splits > 1 && static_cast<uint64_t>(batch) * splits * plane * 4 > ws_bytes) splits = 1;
    if (splits > 1) {
        // partial planes into the workspace, then their sum in split order
        NnArgs p = a;
        p.steps_per_split = ceil_div(ksteps, splits);
        p.splits = splits;
        p.C = static_cast<float*>(ws);
        p.ldc = N;
        p.plane = plane;
        p.mode = 0;
        gemm_nn_q8_tiled_kernel<true><<<dim3(ceil_div(N, kBN2), ceil_div(M, kBM2), batch * splits), kNT2, 0, st>>>(p);
        launch_splitk_reduce(static_cast<const float*>(ws), splits, C, nullptr, M, N, ldc, sC, batch, mode == 0 ? 0 : 1,
                             st);
    } else {
        a.steps_per_split = ksteps;
        gemm_nn_q8_tiled_kernel<false><<<dim3(ceil_div(N, kBN2), ceil_div(M, kBM2), batch), kNT2, 0, st>>>(a);
    }
    return check_launch(fn);
}

}  // namespace
}  // namespace mi

extern "C" int mi_gemm_nn_q8_split(const uint32_t* payload, const float* scales, const float* B, float* C, uint32_t M,
                                   uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb, uint32_t ldc,
                                   uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC, void* stream) {
    return mi::gemm_nn("mi_gemm_nn_q8_split", payload, scales, B, C, M, N, K, mode, lda, ldb, ldc, batch, sA, sB, sC,
                       nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int mi_gemm_nn_q8_split_ws(const uint32_t* payload, const float* scales, const float* B, float* C,
                                      uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb,
                                      uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC,
                                      void* workspace, uint64_t workspace_bytes, void* stream) {
    return mi::gemm_nn("mi_gemm_nn_q8_split_ws", payload, scales, B, C, M, N, K, mode, lda, ldb, ldc, batch, sA, sB,
                       sC, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" uint64_t mi_gemm_nn_q8_workspace_bytes(uint32_t M, uint32_t N, uint32_t K, uint32_t batch) {
    // the tiled kernel's split plan (shapes the untiled kernel serves use none of it)
    if (M == 0 || N == 0 || batch == 0 || K == 0 || K % mi::kBK2) return 0;
    const uint32_t splits = mi::nn_splits(M, N, K, batch);
    return splits > 1 ? static_cast<uint64_t>(batch) * splits * M * N * 4 : 0;
}
