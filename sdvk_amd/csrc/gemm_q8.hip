// gemm_q8.hip -- Q8_0 NT GEMM for gfx950:  C[M,N] (=|+=) A[M,K] . deq(W[N,K])^T (+bias)
//
// Reference behaviour: src/Modules/GPU/shaders/gemm_nt_q8_v.comp (mode / bias /
// lda / ldc / batch semantics :37-54,115-127) and gemm_nt_q8.comp; host routing
// sdvkgen.cpp:917-936. The algorithm here is our own:
//
//   * a workgroup computes a BM x BN tile of C; each K step covers KB Q8_0
//     block columns (32 k each), so every weight row sees whole blocks;
//   * A (fp32) is streamed with coalesced 16-byte loads, rounded to fp16 and
//     written to LDS; the weight blocks are streamed (34-byte GGUF blocks or
//     the reference's split int8 + fp32-scale planes), dequantised once per
//     workgroup to fp16 (w = d * q, rounded once) and written to LDS;
//   * waves multiply LDS fragments with v_mfma_f32_32x32x16_f16 (fp32
//     accumulation). The next step's global loads are in flight while the
//     current step's MFMAs run (register prefetch + two LDS stages, one
//     barrier per step);
//   * workgroup ids are remapped so that each XCD runs a compact block of
//     tiles (a grouped tile order cut into one contiguous chunk per XCD) and
//     its workgroups share A and W panels in that XCD's L2;
//   * grids too small to fill 256 CUs may split K when the caller passes a
//     workspace (the *_ws entries): each split stores its partial tile into
//     the workspace and a reduce kernel adds the partials in split order, then
//     applies bias / accumulate. Every plan sums in a fixed order, so a call
//     repeats bit for bit; entries without a workspace never split K.
#include <algorithm>
#include <type_traits>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace mi {
namespace {

struct GemmArgs {
    const float* A;
    const uint8_t* W;       // 34-byte blocks, or the split int8 payload
    const float* scales;    // split layout only
    const float* bias;
    float* C;
    uint32_t M, N, K, mode, lda, ldc;
    uint64_t sA, sC;
    uint32_t tiles_n;       // ceil(N / BN)
    uint32_t ksteps;        // ceil(K / BK)
    uint32_t steps_per_split;
    uint32_t rowbytes;      // 34-byte layout: bytes per weight row
    uint32_t tiles_m;       // ceil(M / BM)
    uint32_t group_m;       // tile order: groups of group_m row panels, column-major inside a group
    uint32_t cvec;          // C rows 16-byte aligned (C % 16 == 0, ldc % 4 == 0, sC % 4 == 0)
    uint32_t bvec;          // bias 16-byte aligned
    uint32_t F;             // GEGLU epilogue: output columns (W has 2F rows: value rows, then gate rows)
    uint32_t out_half;      // GEGLU / plain mode-0 epilogue: output stored as fp16 (ldc in halves), the fp32 result rounded once
    uint64_t split_stride;  // K-split partials: elements between the planes of consecutive splits
};

// Epilogues. kEpiPlain: the reference's modes (0 stores acc + bias, 1 adds acc
// to C). kEpiResidual: C += acc + bias (a residual add fused into the GEMM).
// kEpiGeglu: W holds 2F rows (GEGLU's value rows, then its gate rows) and
// C[m, j] = (v + bias[j]) * gelu(g + bias[F + j]) for the value / gate
// products v, g of output column j: each 32-wide MFMA column tile holds 16
// value columns and the 16 gate columns that pair with them, so the
// epilogue combines them in registers and only F columns reach memory.
enum Epi { kEpiPlain = 0, kEpiGeglu = 1, kEpiResidual = 2 };

// W row of tile column c (0 <= c < BN) for an output tile starting at column
// o0: the first 16 columns of every 32 are value rows, the next 16 the gate
// rows of the same outputs; outputs past F read the last valid rows.
__device__ __forceinline__ uint32_t geglu_wrow(uint32_t o0, uint32_t c, uint32_t F) {
    const uint32_t o = min(o0 + 16u * (c >> 5) + (c & 15u), F - 1u);
    return (c & 16u) ? F + o : o;
}

GemmArgs make_args(const float* A, const uint8_t* W, const float* scales, const float* bias, float* C, uint32_t M,
                   uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc, uint64_t sA, uint64_t sC,
                   uint32_t rowbytes) {
    GemmArgs a{};
    a.A = A;
    a.W = W;
    a.scales = scales;
    a.bias = bias;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.mode = mode;
    a.lda = lda;
    a.ldc = ldc;
    a.sA = sA;
    a.sC = sC;
    a.rowbytes = rowbytes;
    const uint32_t ldc_e = ldc ? ldc : N;
    a.cvec = (reinterpret_cast<uintptr_t>(C) % 16 == 0 && ldc_e % 4 == 0 && sC % 4 == 0) ? 1u : 0u;
    a.bvec = reinterpret_cast<uintptr_t>(bias) % 16 == 0 ? 1u : 0u;
    return a;
}

enum WKind { kBlocks34 = 0, kSplit = 1 };

// fp16 bits of (1024 + u) for each byte u of x ^ 0x80808080: subtracting 1152
// leaves the signed byte value exactly (|q| <= 128 < 2^11).
__device__ __forceinline__ half8 dequant8_f16(uint32_t lo, uint32_t hi, _Float16 d) {
    const uint32_t xl = lo ^ 0x80808080u, xh = hi ^ 0x80808080u;
    const half2 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    const half2 dd = {d, d};
    half2 h0 = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, xl, 0x04010400u));
    half2 h1 = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, xl, 0x04030402u));
    half2 h2 = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, xh, 0x04010400u));
    half2 h3 = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, xh, 0x04030402u));
    h0 = (h0 - bias) * dd;  // one rounding of the exact product q * d
    h1 = (h1 - bias) * dd;
    h2 = (h2 - bias) * dd;
    h3 = (h3 - bias) * dd;
    return half8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// fp32 scales (split layout, arbitrary fp32): w = fp16(fp32(q) * s).
__device__ __forceinline__ half8 dequant8_f32(uint32_t lo, uint32_t hi, float s0, float s1) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((lo >> (8 * i)) & 0xffu)) * s0);
        h[4 + i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((hi >> (8 * i)) & 0xffu)) * s1);
    }
    return h;
}

// MFMAs and their fragment reads only (ping-pong compute halves).
template <int NMFMA, int NREAD0, int NREAD>
__device__ __forceinline__ void interleave_compute() {
    __builtin_amdgcn_sched_group_barrier(0x100, NREAD0, 0);
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (NREAD + NMFMA - 1) / NMFMA, 0);
    }
}

// One register set (PF = 1): the store phase consumes the loads issued at the
// start of the same step, so it may only begin after the first NHEAD MFMAs
// (which carry the fragment reads); the rest of the MFMAs each carry a share
// of the conversions, dequantisation and LDS writes. Left to itself the
// compiler hoists the conversions next to the loads and the wave waits out the
// whole memory latency with one MFMA issued.
template <int NMFMA, int NHEAD, int NREAD0, int NREAD, int NVALU, int NWRITE>
__device__ __forceinline__ void interleave_step_tail() {
    static_assert(NHEAD > 0 && NHEAD < NMFMA, "head and tail both hold MFMAs");
    constexpr int kTail = NMFMA - NHEAD;
    __builtin_amdgcn_sched_group_barrier(0x100, NREAD0, 0);
#pragma unroll
    for (int i = 0; i < NHEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (NREAD + NMFMA - 1) / NMFMA, 0);
    }
#pragma unroll
    for (int i = 0; i < kTail; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (NREAD + NMFMA - 1) / NMFMA, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, (NVALU + kTail - 1) / kTail, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, (NWRITE + kTail - 1) / kTail, 0);
    }
}

// ---- epilogue ---------------------------------------------------------------------
//
// Non-split: a wave's FM x FN accumulator tiles (32 x 32 each, transposed
// product: a lane holds row l32 and columns 8 q + 4 g + e) go to C one tile at
// a time through a wave-private 32 x kStageLd float region of LDS, read back
// as (row, 4 columns) units, so eight lanes write one 128-byte row segment per
// instruction. One runtime loop serves every tile, which keeps the epilogue a
// few hundred instructions (an unrolled per-tile epilogue with bias / mode /
// edge branches is tens of KB of code that every workgroup runs once, cold in
// the instruction cache).
// Split K: the plain product (a lane holds column l32 and rows
// 8 (r / 4) + 4 g + r % 4) is stored straight from the registers into the
// split's partial plane (row stride ldc = N), 32 consecutive floats per
// instruction; the reduce kernel adds the planes and applies bias / mode.
constexpr int kStageLd = 36;                       // floats per staged row (16-byte pad)
constexpr int kStageFloats = 32 * kStageLd;        // per wave

// GEGLU (EPI == kEpiGeglu): nw is the wave's first output column; tile b
// yields output columns nw + 16 (b % FN) + 0..15 from its value columns 0..15
// and gate columns 16..31.
template <int FM, int FN, bool SPLITK, int EPI = kEpiPlain>
__device__ __forceinline__ void store_tiles(const GemmArgs& a, float* C, float* stage, uint32_t mw, uint32_t nw,
                                            const floatx16 (&acc)[FM][FN], int lane) {
    static_assert(!(SPLITK && EPI == kEpiGeglu), "the GEGLU epilogue needs the whole K sum");
    const int l32 = lane & 31, g = lane >> 5;
    const bool vec = a.cvec != 0;
    const bool use_bias = !SPLITK && (EPI == kEpiResidual ? true : a.mode == 0) && a.bias != nullptr;
    const bool vec_bias = !use_bias || a.bvec != 0;
    if constexpr (SPLITK) {
        // no staging: one store instruction covers 32 consecutive floats of a row
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const uint32_t n = nw + 32 * fn + l32;
            if (n >= a.N) continue;
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = mw + 32 * fm + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m < a.M) C[static_cast<uint64_t>(m) * a.ldc + n] = acc[fm][fn][r];
                }
        }
        return;
    }
    // The bias values of the lane's columns, loaded once before the tile loop
    // (they depend on the tile's column block only): a load inside the loop
    // waits out a memory round trip -- and every store issued before it -- per
    // tile. GEGLU: value and gate biases of output columns nw + 16 fn + 4 (lane
    // % 4) + e; 16-byte path: columns nw + 32 fn + 4 (lane % 8) + e.
    float gbv[EPI == kEpiGeglu ? FN : 1][4], gbg[EPI == kEpiGeglu ? FN : 1][4];
    floatx4 bias4[EPI == kEpiGeglu ? 1 : FN];
    if constexpr (EPI == kEpiGeglu) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t j = min(nw + 16 * fn + (lane & 3) * 4 + e, a.F - 1);  // columns past F are never stored
                gbv[fn][e] = a.bias ? a.bias[j] : 0.0f;
                gbg[fn][e] = a.bias ? a.bias[a.F + j] : 0.0f;
            }
    } else {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const uint32_t n = nw + 32 * fn + (lane & 7) * 4;
            bias4[fn] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            if (use_bias && vec && vec_bias && n + 3 < a.N) bias4[fn] = *reinterpret_cast<const floatx4*>(a.bias + n);
        }
    }
    for (int b = 0; b < FM * FN; ++b) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
                if (b == fm * FN + fn) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<floatx4*>(&stage[l32 * kStageLd + 8 * q + 4 * g]) =
                            floatx4{acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1], acc[fm][fn][4 * q + 2],
                                    acc[fm][fn][4 * q + 3]};
                }
        // the staged tile is read back by other lanes of the wave: keep every
        // write of the wave ahead of every read (no instruction is emitted)
        __builtin_amdgcn_wave_barrier();
        if constexpr (EPI == kEpiGeglu) {
            // 32 rows x 4 groups of 4 output columns: value at column 4 c4, gate at 16 + 4 c4
            const uint32_t mb = mw + 32 * (b / FN), ob = nw + 16 * (b % FN);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int u = lane + 64 * i;
                const int row = u >> 2, col = (u & 3) * 4;
                const floatx4 v = *reinterpret_cast<const floatx4*>(&stage[row * kStageLd + col]);
                const floatx4 gt = *reinterpret_cast<const floatx4*>(&stage[row * kStageLd + 16 + col]);
                const uint32_t m = mb + row, n = ob + col;
                if (m >= a.M) continue;
                float* c = C + static_cast<uint64_t>(m) * a.ldc + n;
                floatx4 o;
                float bv[4], bg[4];
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    if (b % FN == fn) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            bv[e] = gbv[fn][e];
                            bg[e] = gbg[fn][e];
                        }
                    }
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (v[e] + bv[e]) * gelu_erf(gt[e] + bg[e]);
                if (a.out_half) {
                    // the fp32 value, then one RNE rounding to fp16 (the value an
                    // fp32 G would give the next GEMM's A staging); the empty register
                    // constraint keeps the rounding from fusing into the multiply
                    asm volatile("" : "+v"(o));
                    _Float16* ch = reinterpret_cast<_Float16*>(C) + static_cast<uint64_t>(m) * a.ldc + n;
                    const half4 h = {static_cast<_Float16>(o[0]), static_cast<_Float16>(o[1]),
                                     static_cast<_Float16>(o[2]), static_cast<_Float16>(o[3])};
                    if (vec && n + 3 < a.F) {
                        *reinterpret_cast<half4*>(ch) = h;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < a.F) ch[e] = h[e];
                    }
                } else if (vec && n + 3 < a.F) {
                    __builtin_nontemporal_store(o, reinterpret_cast<floatx4*>(c));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < a.F) c[e] = o[e];
                }
            }
            __builtin_amdgcn_wave_barrier();
            continue;
        }
        const uint32_t mb = mw + 32 * (b / FN), nb = nw + 32 * (b % FN);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = lane + 64 * i;
            const int row = u >> 3, col = (u & 7) * 4;
            const floatx4 v = *reinterpret_cast<const floatx4*>(&stage[row * kStageLd + col]);
            const uint32_t m = mb + row, n = nb + col;
            if (m >= a.M) continue;
            if (EPI == kEpiPlain && a.out_half) {
                // mode 0 with an fp16 output: acc + bias in fp32, then one RNE
                // rounding (the empty register constraint keeps the rounding from
                // fusing into the add)
                floatx4 o = v;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (use_bias) o[e] += a.bias[min(n + e, a.N - 1)];
                asm volatile("" : "+v"(o));
                const half4 h = {static_cast<_Float16>(o[0]), static_cast<_Float16>(o[1]),
                                 static_cast<_Float16>(o[2]), static_cast<_Float16>(o[3])};
                _Float16* ch = reinterpret_cast<_Float16*>(C) + static_cast<uint64_t>(m) * a.ldc + n;
                if (vec && n + 3 < a.N) {
                    *reinterpret_cast<half4*>(ch) = h;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < a.N) ch[e] = h[e];
                }
                continue;
            }
            float* c = C + static_cast<uint64_t>(m) * a.ldc + n;
            if (vec && vec_bias && n + 3 < a.N) {
                floatx4 bb = bias4[0];
#pragma unroll
                for (int fn = 1; fn < FN; ++fn)
                    if (b % FN == fn) bb = bias4[fn];
                if (EPI == kEpiResidual) {
                    // x + (acc + bias): the rounding of the separate GEMM + add
                    floatx4 o = v;
                    if (use_bias) o += bb;
                    *reinterpret_cast<floatx4*>(c) = *reinterpret_cast<const floatx4*>(c) + o;
                } else if (a.mode == 0) {
                    floatx4 o = v;
                    if (use_bias) o += bb;
                    // C is written once and not re-read here: streaming stores keep
                    // it from displacing the operand working set in L2
                    __builtin_nontemporal_store(o, reinterpret_cast<floatx4*>(c));
                } else {
                    *reinterpret_cast<floatx4*>(c) = *reinterpret_cast<const floatx4*>(c) + v;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (n + e >= a.N) continue;
                    if (EPI == kEpiResidual) c[e] += v[e] + (use_bias ? a.bias[n + e] : 0.0f);
                    else if (a.mode == 0) c[e] = v[e] + (use_bias ? a.bias[n + e] : 0.0f);
                    else c[e] += v[e];
                }
            }
        }
        // every read of this tile precedes the next tile's writes
        __builtin_amdgcn_wave_barrier();
    }
}

// AH: A holds fp16 values (fp16 activations from a producer that rounded them
// already); the staging then copies 16-byte units of 8 halves into LDS with no
// conversion. Otherwise A is fp32 and each 16-byte unit of 4 floats is rounded
// to fp16 (RNE) on its way to LDS: for A values that are fp16 numbers both
// paths stage the same bits.
// PP: the 8-wave two-register-set loop as two alternating wave groups (same
// MFMAs in the same k order per wave, so the same bits as the one-barrier loop).
template <int BM, int BN, int WM, int WN, int KB, int WK, bool SPLITK, bool KTAIL, int PF, int EPI = kEpiPlain,
          bool AH = false, bool PP = false>
__global__ __launch_bounds__(WM * WN * 64) void gemm_q8_kernel(GemmArgs a) {
    constexpr int NT = WM * WN * 64;
    constexpr int BK = 32 * KB;
    constexpr int LDK = BK + 8;                   // LDS row stride in halves (16-B pad)
    constexpr int TM = BM / WM, TN = BN / WN;     // wave tile
    constexpr int FM = TM / 32, FN = TN / 32;     // 32x32 MFMA tiles per wave
    constexpr int AE = AH ? 2 : 4;                // bytes per A element
    constexpr int AV = 16 / AE;                   // A elements per 16-byte unit
    constexpr int A_UNITS = BM * BK / AV;         // 16-byte A units per step
    constexpr int A_IT = A_UNITS / NT;
    constexpr int W_UNITS = BN * BK / 8;          // (row, 8-k group) per step
    constexpr int W_IT = W_UNITS / NT;
    // 34-byte blocks with two blocks per step: one whole block per lane (three
    // loads for 32 weights). Block wb of a step is weight row wb / KB, block
    // column wb % KB: the KB blocks of a row (its 68 contiguous bytes of the
    // step) sit on adjacent lanes, so one load instruction of a wave touches
    // 32 weight rows instead of 64. A load instruction's cost grows with the
    // rows it touches: one 192x256 step's W loads take 890 cycles of a CU's
    // load path this way against 1209 with a wave's lanes on 64 rows (a
    // load-only probe of the step on MI355X; 16 rows, the four blocks of two
    // steps, take 607 but gained nothing in the kernel).
    constexpr bool WBLK = WK == kBlocks34 && KB == 2 && !KTAIL;
    constexpr int W_BLOCKS = BN * KB;
    constexpr int WB_IT = (W_BLOCKS + NT - 1) / NT;
    // Twice as many threads as blocks in a 4-wave workgroup (the 64x64 and
    // 128x64 tiles): thread t dequantises half h = t / W_BLOCKS of block
    // t % W_BLOCKS (every thread loads its block's window), so the
    // dequantisation is spread over all four waves instead of two, which would
    // be half of the SIMDs. An 8-wave workgroup with as many threads (the
    // 256x128 tile, the 8-wave 128x128 tile) keeps whole blocks on its first
    // four waves, one per SIMD, and the other four issue their block loads out
    // of range (no memory access): 482 load-path cycles per step for the
    // 128x128 tile's weights in the probe, against 674 with every block loaded
    // twice.
    constexpr bool WHALF = WBLK && 2 * W_BLOCKS == NT && NT == 256;
    // Buffer-load fast path: two blocks per step keep each lane's byte
    // alignment fixed (68 = 0 mod 4), so the step advance is a scalar offset.
    constexpr bool FAST = KB == 2 && !KTAIL;
    static_assert(A_UNITS % NT == 0 && W_UNITS % NT == 0, "staging must divide evenly");
    static_assert(FM >= 1 && FN >= 1, "wave tile below 32x32");

    constexpr int kOperandHalves = 2 * (BM + BN) * LDK;
    constexpr int kStageHalves = 2 * NT / 64 * kStageFloats;
    __shared__ __attribute__((aligned(16))) _Float16 smem[kOperandHalves > kStageHalves ? kOperandHalves : kStageHalves];
    auto As = reinterpret_cast<_Float16 (*)[BM * LDK]>(smem);
    auto Ws = reinterpret_cast<_Float16 (*)[BN * LDK]>(smem + 2 * BM * LDK);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int wm = wave % WM, wn = wave / WM;
    // 8-wave builds: the epilogue takes the wave index from this SGPR copy and
    // the lane from v_mbcnt, so fewer threadIdx-derived VGPRs stay live across
    // the K loop (the 256x256 build, at its 256-register limit, spilled six of
    // them around the loop; three with this). The 4-wave builds keep the
    // prologue's values: with the same change the register allocator moved a
    // spill of the 4-wave 256x256 build into its K loop.
    constexpr bool kFreshLane = NT == 512;
    const int wave_s = kFreshLane ? __builtin_amdgcn_readfirstlane(wave) : wave;

    // Tile order: each XCD takes a contiguous chunk of a grouped order (groups
    // of group_m row panels, column-major inside a group), so the chunk is a
    // compact block of tiles and its workgroups share A and W panels in L2.
    const unsigned lin = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t gsz = a.group_m * a.tiles_n;
    const uint32_t grp = lin / gsz, rem = lin % gsz;
    const uint32_t rows_in = min(a.group_m, a.tiles_m - grp * a.group_m);
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((grp * a.group_m + rem % rows_in) * BM);
    // GEGLU: n0 is the tile's first output column (BN / 2 outputs per tile)
    const uint32_t n0 = __builtin_amdgcn_readfirstlane((rem / rows_in) * (EPI == kEpiGeglu ? BN / 2 : BN));
    const uint32_t s_begin = SPLITK ? blockIdx.y * a.steps_per_split : 0;
    const uint32_t s_end = SPLITK ? min(a.ksteps, s_begin + a.steps_per_split) : a.ksteps;

    // Per-thread byte offsets, fixed for the whole K loop. Rows past M / N read
    // the last valid row: they only feed outputs that are never stored.
    const char* Apanel = reinterpret_cast<const char*>(a.A) +
                         (static_cast<uint64_t>(blockIdx.z) * a.sA + static_cast<uint64_t>(m0) * a.lda) * AE;
    // the range covers exactly the panel's rows: a read past them returns zeros, never faults
    const uint32_t a_bytes = ((min(a.M - m0, static_cast<uint32_t>(BM)) - 1) * a.lda + a.K) * AE;
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(Apanel), 0, static_cast<int>(a_bytes), 0x00020000);
    // 34-byte layout: records up to W's 16-byte-aligned end (the documented
    // read extent); the range check zeroes whole dwords only past that.
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(a.W), 0, WK == kBlocks34 ? static_cast<int>((a.N * a.rowbytes + 15u) & ~15u) : -1,
        0x00020000);
    const __amdgpu_buffer_rsrc_t rS =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(WK == kSplit ? a.scales : a.A), 0, -1, 0x00020000);
    uint32_t a_off[A_IT];
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
        const int f = tid + i * NT;
        const uint32_t row = min(m0 + f / (BK / AV), a.M - 1) - m0;
        a_off[i] = (row * a.lda + (f % (BK / AV)) * AV) * AE;
    }
    uint32_t w_off[W_IT];   // blocks: byte of the unit's first q; split: flat element
    uint32_t w_aux[W_IT];   // blocks: byte of the block's scale; split: byte of the scale
    uint32_t w_k[W_IT];     // k of the unit's first weight within the step
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
        const int u = tid + i * NT;
        const uint32_t n = EPI == kEpiGeglu ? geglu_wrow(n0, u / (BK / 8), a.F) : min(n0 + u / (BK / 8), a.N - 1);
        w_k[i] = (u % (BK / 8)) * 8;
        if constexpr (WK == kBlocks34) {
            w_aux[i] = n * a.rowbytes + (w_k[i] / 32) * 34;
            w_off[i] = w_aux[i] + 2 + (w_k[i] % 32);
        } else {
            w_off[i] = n * a.K + w_k[i];
            w_aux[i] = (w_off[i] >> 5) * 4;
        }
    }

    // PF register sets of prefetched raw data. PF = 2: the loads for step k+2
    // are issued before step k's MFMAs (sets indexed by step parity, like the
    // LDS stages), so every global load has two steps of MFMA work to arrive
    // in; PF = 1 (large tiles, whose steps are long): the loads for step k+1.
    // The load phase is branch-free (raw words only; alignment shifts and
    // conversions happen at store time) so the waitcnt before each store
    // waits for its own set alone.
    floatx4 areg_[PF][A_IT];
    uint32_t w0_[PF][W_IT], w1_[PF][W_IT], w2_[PF][W_IT], wd_[PF][W_IT];
    float ws0_[PF][W_IT], ws1_[PF][W_IT];
    // 34-byte layout: lanes whose 8 q bytes start 2 mod 4 read one more dword
    // and funnel-shift by 16 bits; in the fast path the shift is fixed per lane.
    uint32_t w_sh[PF][W_IT];
#pragma unroll
    for (int i = 0; i < W_IT; ++i)
#pragma unroll
        for (int r = 0; r < PF; ++r) w_sh[r][i] = (w_off[i] & 2u) * 8u;
    // Whole-block staging: the 36-byte window at the block's 4-byte-aligned
    // start; the row stride is 0 mod 4 (K % 64 == 0) and a step advances 68
    // bytes, so a block's position inside its window (0 or 2 bytes) is fixed
    // for the lane. v_perm selectors pick d and the eight q dwords for either.
    // Threads past the step's W_BLOCKS blocks still issue the loads (out of
    // range: zeros, no memory access) and store nothing: a load under a branch
    // makes the compiler's wait counts assume it was skipped, so every later
    // wait would also retire the loads of the step just issued.
    uint32_t wb_off[WB_IT], wb_qsel[WB_IT], wb_dsel[WB_IT];
    uint32_t wbx_[PF][WB_IT][9];
#pragma unroll
    for (int i = 0; i < WB_IT; ++i) {
        const int wb = (tid + i * NT) % W_BLOCKS;
        const uint32_t n = EPI == kEpiGeglu ? geglu_wrow(n0, wb / KB, a.F) : min(n0 + wb / KB, a.N - 1);
        const uint32_t byte = n * a.rowbytes + (wb % KB) * 34;
        // past the step's blocks: out of range, so the load returns zeros and touches no memory
        wb_off[i] = (!WHALF && W_BLOCKS % NT != 0 && tid + i * NT >= W_BLOCKS) ? 0x80000000u : byte & ~3u;
        wb_qsel[i] = (byte & 2u) ? 0x07060504u : 0x05040302u;  // bytes 4..7 or 2..5 of (x[j+1]:x[j])
        wb_dsel[i] = (byte & 2u) ? 0x0c0c0302u : 0x0c0c0100u;  // bytes 2,3 or 0,1 of x[0]; 0x0c = zero
    }

    auto load_step = [&](uint32_t ks_in, auto RS) {
        constexpr int rs = decltype(RS)::value;
        // the step is wave-uniform; say so, or the buffer loads' scalar offsets
        // are built with a per-lane loop
        const uint32_t ks = __builtin_amdgcn_readfirstlane(ks_in);
#pragma unroll
        for (int i = 0; i < A_IT; ++i) {
            if constexpr (KTAIL) {
                const uint32_t k = ks * BK + ((tid + i * NT) % (BK / AV)) * AV;
                areg_[rs][i] = floatx4{0.f, 0.f, 0.f, 0.f};
                if (k < a.K) areg_[rs][i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rA, a_off[i], ks * BK * AE, 0));
            } else {
                areg_[rs][i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rA, a_off[i], ks * BK * AE, 0));
            }
        }
        if constexpr (WBLK) {
            const uint32_t soff = ks * (KB * 34);
#pragma unroll
            for (int i = 0; i < WB_IT; ++i) {
                const auto x0 = __builtin_amdgcn_raw_buffer_load_b128(rW, wb_off[i], soff, 0);
                const auto x1 = __builtin_amdgcn_raw_buffer_load_b128(rW, wb_off[i] + 16, soff, 0);
                wbx_[rs][i][8] = __builtin_amdgcn_raw_buffer_load_b32(rW, wb_off[i] + 32, soff, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wbx_[rs][i][e] = x0[e];
                    wbx_[rs][i][4 + e] = x1[e];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (WBLK ? 0 : W_IT); ++i) {
            if constexpr (WK == kBlocks34) {
                const uint32_t soff = ks * (KB * 34);
                const uint32_t addr = FAST ? w_off[i] : w_off[i] + soff;
                const uint32_t base = addr & ~3u;
                const uint32_t so = FAST ? soff : 0u;
                const auto w01 = __builtin_amdgcn_raw_buffer_load_b64(rW, base, so, 0);
                w0_[rs][i] = w01[0];
                w1_[rs][i] = w01[1];
                // third dword only matters when shifted; otherwise re-read the second
                w2_[rs][i] = __builtin_amdgcn_raw_buffer_load_b32(rW, base + ((addr & 2u) ? 8u : 4u), so, 0);
                wd_[rs][i] = __builtin_amdgcn_raw_buffer_load_b16(rW, FAST ? w_aux[i] : w_aux[i] + soff, so, 0);
                if constexpr (!FAST) w_sh[rs][i] = (addr & 2u) * 8u;  // shift of this set's step
            } else if constexpr (FAST) {
                const auto w01 = __builtin_amdgcn_raw_buffer_load_b64(rW, w_off[i], ks * BK, 0);
                w0_[rs][i] = w01[0];
                w1_[rs][i] = w01[1];
                ws0_[rs][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rS, w_aux[i], ks * KB * 4, 0));
                ws1_[rs][i] = ws0_[rs][i];
            } else {
                const uint32_t k = ks * BK + w_k[i];
                const uint64_t f = static_cast<uint64_t>(w_off[i]) + static_cast<uint64_t>(ks) * BK;
                const uint32_t* p = reinterpret_cast<const uint32_t*>(a.W);
                w0_[rs][i] = 0u;
                w1_[rs][i] = 0u;
                ws0_[rs][i] = 0.0f;
                ws1_[rs][i] = 0.0f;
                if (!KTAIL || k < a.K) {
                    w0_[rs][i] = p[f >> 2];
                    ws0_[rs][i] = a.scales[f >> 5];
                    if (!KTAIL || k + 4u < a.K) {
                        w1_[rs][i] = p[(f >> 2) + 1u];
                        ws1_[rs][i] = a.scales[(f + 4u) >> 5];
                    }
                }
            }
        }
    };
    auto store_step = [&](auto RS, auto ST) {
        constexpr int rs = decltype(RS)::value;  // register set
        constexpr int st = decltype(ST)::value;  // LDS stage
#pragma unroll
        for (int i = 0; i < A_IT; ++i) {
            const int f = tid + i * NT;
            if constexpr (AH) {
                *reinterpret_cast<half8*>(&As[st][(f / (BK / 8)) * LDK + (f % (BK / 8)) * 8]) =
                    __builtin_bit_cast(half8, areg_[rs][i]);
            } else {
                half4 h;
                h[0] = static_cast<_Float16>(areg_[rs][i][0]);
                h[1] = static_cast<_Float16>(areg_[rs][i][1]);
                h[2] = static_cast<_Float16>(areg_[rs][i][2]);
                h[3] = static_cast<_Float16>(areg_[rs][i][3]);
                *reinterpret_cast<half4*>(&As[st][(f / (BK / 4)) * LDK + (f % (BK / 4)) * 4]) = h;
            }
        }
        if constexpr (WHALF) {
            const uint32_t* x = wbx_[rs][0];
            const bool hi = tid >= W_BLOCKS;  // wave-uniform: W_BLOCKS is a multiple of 64
            uint32_t xs[5];
#pragma unroll
            for (int j = 0; j < 5; ++j) xs[j] = hi ? x[4 + j] : x[j];
            const _Float16 d = __builtin_bit_cast(
                _Float16, static_cast<uint16_t>(__builtin_amdgcn_perm(x[0], x[0], wb_dsel[0])));
            uint32_t q[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) q[j] = __builtin_amdgcn_perm(xs[j + 1], xs[j], wb_qsel[0]);
            const int wb = hi ? tid - W_BLOCKS : tid;
            _Float16* dst = &Ws[st][(wb / KB) * LDK + (wb % KB) * 32 + (hi ? 16 : 0)];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                *reinterpret_cast<half8*>(dst + 8 * j) = dequant8_f16(q[2 * j], q[2 * j + 1], d);
        } else if constexpr (WBLK) {
#pragma unroll
            for (int i = 0; i < WB_IT; ++i) {
                const int wb = tid + i * NT;
                if (W_BLOCKS % NT == 0 || wb < W_BLOCKS) {
                    const uint32_t* x = wbx_[rs][i];
                    const _Float16 d = __builtin_bit_cast(
                        _Float16, static_cast<uint16_t>(__builtin_amdgcn_perm(x[0], x[0], wb_dsel[i])));
                    uint32_t q[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_perm(x[j + 1], x[j], wb_qsel[i]);
                    _Float16* dst = &Ws[st][(wb / KB) * LDK + (wb % KB) * 32];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        *reinterpret_cast<half8*>(dst + 8 * j) = dequant8_f16(q[2 * j], q[2 * j + 1], d);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (WBLK ? 0 : W_IT); ++i) {
            const int u = tid + i * NT;
            half8 h;
            if constexpr (WK == kBlocks34) {
                const uint32_t lo = __builtin_amdgcn_alignbit(w1_[rs][i], w0_[rs][i], w_sh[rs][i]);
                const uint32_t hi = __builtin_amdgcn_alignbit(w2_[rs][i], w1_[rs][i], w_sh[rs][i]);
                h = dequant8_f16(lo, hi, __builtin_bit_cast(_Float16, static_cast<uint16_t>(wd_[rs][i])));
            } else {
                h = dequant8_f32(w0_[rs][i], w1_[rs][i], ws0_[rs][i], ws1_[rs][i]);
            }
            *reinterpret_cast<half8*>(&Ws[st][(u / (BK / 8)) * LDK + w_k[i]]) = h;
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto compute = [&](auto ST) {
        constexpr int st = decltype(ST)::value;
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            half8 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const half8*>(&As[st][(wm * TM + 32 * i + l32) * LDK + 16 * s + 8 * g]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&Ws[st][(wn * TN + 32 * j + l32) * LDK + 16 * s + 8 * g]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    // Stores: the transposed product (C^T), so a lane holds row
                    // m = l32 and four runs of four consecutive columns (16-byte
                    // stores). Split K: C, so a lane holds column l32 and the
                    // atomics of one instruction hit 32 consecutive floats.
                    if constexpr (SPLITK)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[j], af[i], acc[i][j], 0, 0, 0);
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;

    // Step j computes from LDS stage j&1. PF = 2: the loads of step j+2 (into
    // register set j&1) are in flight meanwhile, then set (j+1)&1, loaded one
    // step earlier, is stored. PF = 1: the loads of step j+1 are in flight and
    // stored after the MFMAs. Prefetches past the last step re-read it
    // (clamped, unused), so the load phase has no branches. Two steps per trip
    // keep every stage / set index a compile-time constant.
    constexpr int kMfma = FM * FN * (BK / 16);       // MFMAs per step
    constexpr int kRead0 = FM + FN;                  // fragment reads of the first k16 slice
    constexpr int kReads = (FM + FN) * (BK / 16);    // all fragment reads of a step
    constexpr int kWrites = A_IT + (WHALF ? 2 : WBLK ? 4 * WB_IT : W_IT);              // LDS writes of the store phase
    constexpr int kValu = (AH ? 0 : A_IT * 2) + (WHALF ? 36 : WBLK ? 60 * WB_IT : W_IT * 16);  // conversions + dequant (approx.)
    // Every workgroup sweeps K in the same order, so the workgroups that share
    // a panel read the same K slice at about the same time (L2 reuse).
    const uint32_t n_steps = s_end - s_begin;
    auto phys = [&](uint32_t j) { return s_begin + j; };
    const uint32_t last = n_steps - 1;
    if (n_steps > 0) {
        load_step(phys(0), S0{});
        store_step(S0{}, S0{});
        if constexpr (PF == 2) load_step(phys(min(1u, last)), S1{});
    }
    __syncthreads();
    uint32_t j = 0;
    if constexpr (PP) {
        static_assert(PF == 2 && NT == 512, "ping-pong: two register sets, two groups of four waves");
        // Ping-pong: waves 0-3 and 4-7 (one of each per SIMD) alternate inside
        // every step. While one group multiplies from stage s, the other issues
        // its loads of step + 2 and converts and writes its share of step + 1
        // into the other stage; two barriers per step, and a stage is written
        // only in halves in which no wave reads it. The sched_barriers keep each
        // instruction in its half (the MFMAs would otherwise sink past a
        // barrier into the next half).
        auto mem = [&](uint32_t ld, auto RL, auto RS) {
            __builtin_amdgcn_sched_barrier(0);
            load_step(phys(ld), RL);
            __builtin_amdgcn_sched_barrier(0);
            store_step(RS, RS);
            __builtin_amdgcn_sched_barrier(0);
        };
        auto comp = [&](auto ST) {
            __builtin_amdgcn_sched_barrier(0);
            compute(ST);
            interleave_compute<kMfma, kRead0, kReads - kRead0>();
            __builtin_amdgcn_sched_barrier(0);
        };
        if (n_steps < 2) {
            // one step: the tail below
        } else if (wave_s < 4) {
            // The first compute half is peeled so that the loop starts with the
            // half whose stores wait for the previous half's loads (a loop that
            // starts with MFMAs got a wait for the loads in flight at its top).
            // Barriers: 4 per two steps, as in the other group's loop; an odd
            // last step is computed in the last trip, with no barrier after it,
            // while the other group computes it in its tail.
            comp(S0{});
            __syncthreads();
            for (; j + 2 <= n_steps; j += 2) {
                mem(min(j + 2, last), S0{}, S1{});
                __syncthreads();
                comp(S1{});
                __syncthreads();
                mem(min(j + 3, last), S1{}, S0{});
                __syncthreads();
                if (j + 2 < n_steps) {
                    comp(S0{});
                    if (j + 4 <= n_steps) __syncthreads();
                }
            }
            j = n_steps;
        } else {
            for (; j + 2 <= n_steps; j += 2) {
                mem(min(j + 2, last), S0{}, S1{});
                __syncthreads();
                comp(S0{});
                __syncthreads();
                mem(min(j + 3, last), S1{}, S0{});
                __syncthreads();
                comp(S1{});
                __syncthreads();
            }
        }
    }
    for (; !PP && j + 2 <= n_steps; j += 2) {
        if constexpr (PF == 2) {
            load_step(phys(min(j + 2, last)), S0{});
            __builtin_amdgcn_sched_barrier(0);  // issue the prefetch before the MFMAs
            compute(S0{});
            store_step(S1{}, S1{});
            interleave_step<kMfma, kRead0, kReads - kRead0, kValu, kWrites>();
            __syncthreads();
            load_step(phys(min(j + 3, last)), S1{});
            __builtin_amdgcn_sched_barrier(0);
            compute(S1{});
            store_step(S0{}, S0{});
            interleave_step<kMfma, kRead0, kReads - kRead0, kValu, kWrites>();
            __syncthreads();
        } else {
            load_step(phys(j + 1), S0{});
            __builtin_amdgcn_sched_barrier(0);
            compute(S0{});
            store_step(S0{}, S1{});
            interleave_step_tail<kMfma, kMfma * 3 / 4, kRead0, kReads - kRead0, kValu, kWrites>();
            __syncthreads();
            load_step(phys(min(j + 2, last)), S0{});
            __builtin_amdgcn_sched_barrier(0);
            compute(S1{});
            store_step(S0{}, S0{});
            interleave_step_tail<kMfma, kMfma * 3 / 4, kRead0, kReads - kRead0, kValu, kWrites>();
            __syncthreads();
        }
    }
    if (j < n_steps) compute(S0{});

    float* C = a.C + static_cast<uint64_t>(blockIdx.z) * a.sC + (SPLITK ? blockIdx.y * a.split_stride : 0);
    __syncthreads();  // every wave is done with the operand tiles before LDS is reused
    const int wm_s = kFreshLane ? wave_s % WM : wm, wn_s = kFreshLane ? wave_s / WM : wn;
    store_tiles<FM, FN, SPLITK, EPI>(a, C, reinterpret_cast<float*>(smem) + wave_s * kStageFloats, m0 + wm_s * TM,
                                     EPI == kEpiGeglu ? n0 + wn_s * TN / 2 : n0 + wn_s * TN, acc,
                                     kFreshLane ? lane_id() : lane);
}

// K == 0: C[m, n] = bias[n] (or 0) in mode 0, C[m, n] += bias[n] in mode 2.
__global__ __launch_bounds__(256) void gemm_fill_kernel(float* C, const float* bias, uint32_t M, uint32_t N,
                                                        uint32_t ldc, uint64_t sC, uint32_t add) {
    const uint32_t n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const float v = bias ? bias[n] : 0.0f;
    float* c = C + static_cast<uint64_t>(blockIdx.z) * sC + n;
    for (uint32_t m = blockIdx.y; m < M; m += gridDim.y) {
        float* p = c + static_cast<uint64_t>(m) * ldc;
        *p = add ? *p + v : v;
    }
}

void launch_fill(float* C, const float* bias, uint32_t M, uint32_t N, uint32_t ldc, uint64_t sC, uint32_t batch,
                 bool add, hipStream_t s) {
    gemm_fill_kernel<<<dim3(ceil_div(N, 256), std::min<uint32_t>(M, 4096), batch), 256, 0, s>>>(C, bias, M, N, ldc,
                                                                                                sC, add ? 1u : 0u);
}

// The K splits' partial planes P[z][s] ([M, N], row stride N, `plane` floats
// apart; batch item z's planes start at z * splits * plane) are added in split
// order -- ((P0 + P1) + P2) + ... -- so the sum never depends on timing:
//   OP 0: C = sum + bias[n]   (mode 0; bias may be NULL)
//   OP 1: C = C + sum         (mode 1)
//   OP 2: C = C + (sum + bias[n])   (mode 2, the residual epilogue)
// VEC: 16-byte accesses over the flattened [M, N / 4] index (N % 4 == 0, C rows
// 16-byte aligned); a capped grid strides over the tile. SP > 0: exactly SP
// splits, every partial of a unit loaded before the first add (one memory
// round trip instead of one per split; the same adds in the same order).
template <int OP, bool VEC, int SP = 0>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* P, uint64_t plane, uint32_t splits, float* C,
                                                            const float* bias, uint32_t M, uint32_t N, uint32_t ldc,
                                                            uint64_t sC, uint32_t bvec) {
    const float* p = P + static_cast<uint64_t>(blockIdx.y) * splits * plane;
    float* c = C + static_cast<uint64_t>(blockIdx.y) * sC;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
    if constexpr (VEC) {
        const uint32_t N4 = N / 4;
        const uint64_t total = static_cast<uint64_t>(M) * N4;
        for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
            const uint32_t m = static_cast<uint32_t>(i / N4), n = static_cast<uint32_t>(i % N4) * 4;
            const float* q = p + static_cast<uint64_t>(m) * N + n;
            floatx4 v;
            if constexpr (SP > 0) {
                floatx4 part[SP];
#pragma unroll
                for (int sp = 0; sp < SP; ++sp) part[sp] = *reinterpret_cast<const floatx4*>(q + sp * plane);
                v = part[0];
#pragma unroll
                for (int sp = 1; sp < SP; ++sp) v += part[sp];
            } else {
                v = *reinterpret_cast<const floatx4*>(q);
                for (uint32_t sp = 1; sp < splits; ++sp) v += *reinterpret_cast<const floatx4*>(q + sp * plane);
            }
            floatx4 b = {0.0f, 0.0f, 0.0f, 0.0f};
            if (OP != 1 && bias)
                b = bvec ? *reinterpret_cast<const floatx4*>(bias + n)
                         : floatx4{bias[n], bias[n + 1], bias[n + 2], bias[n + 3]};
            floatx4* o = reinterpret_cast<floatx4*>(c + static_cast<uint64_t>(m) * ldc + n);
            if (OP == 0) *o = bias ? v + b : v;
            else if (OP == 1) *o = *o + v;
            else *o = *o + (bias ? v + b : v);
        }
    } else {
        const uint64_t total = static_cast<uint64_t>(M) * N;
        for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
            const uint32_t m = static_cast<uint32_t>(i / N), n = static_cast<uint32_t>(i % N);
            const float* q = p + i;
            float v = *q;
            for (uint32_t sp = 1; sp < splits; ++sp) v += q[sp * plane];
            const float b = (OP != 1 && bias) ? bias[n] : 0.0f;
            float* o = c + static_cast<uint64_t>(m) * ldc + n;
            if (OP == 0) *o = bias ? v + b : v;
            else if (OP == 1) *o = *o + v;
            else *o = *o + (bias ? v + b : v);
        }
    }
}

template <int OP>
void launch_reduce_op(const float* P, uint64_t plane, uint32_t splits, float* C, const float* bias, uint32_t M,
                      uint32_t N, uint32_t ldc, uint64_t sC, uint32_t batch, hipStream_t s) {
    const bool vec = reinterpret_cast<uintptr_t>(C) % 16 == 0 && N % 4 == 0 && ldc % 4 == 0 && sC % 4 == 0;
    const uint64_t units = static_cast<uint64_t>(M) * (vec ? N / 4 : N);
    const unsigned gx = static_cast<unsigned>(std::min<uint64_t>(std::max<uint64_t>(ceil_div(units, 256ull), 1), 1024));
    const uint32_t bvec = reinterpret_cast<uintptr_t>(bias) % 16 == 0 ? 1u : 0u;
    const dim3 grid(gx, batch);
    if (!vec) {
        splitk_reduce_kernel<OP, false><<<grid, 256, 0, s>>>(P, plane, splits, C, bias, M, N, ldc, sC, bvec);
        return;
    }
    switch (splits) {
        case 2: splitk_reduce_kernel<OP, true, 2><<<grid, 256, 0, s>>>(P, plane, splits, C, bias, M, N, ldc, sC, bvec); break;
        case 3: splitk_reduce_kernel<OP, true, 3><<<grid, 256, 0, s>>>(P, plane, splits, C, bias, M, N, ldc, sC, bvec); break;
        case 4: splitk_reduce_kernel<OP, true, 4><<<grid, 256, 0, s>>>(P, plane, splits, C, bias, M, N, ldc, sC, bvec); break;
        case 8: splitk_reduce_kernel<OP, true, 8><<<grid, 256, 0, s>>>(P, plane, splits, C, bias, M, N, ldc, sC, bvec); break;
        default: splitk_reduce_kernel<OP, true><<<grid, 256, 0, s>>>(P, plane, splits, C, bias, M, N, ldc, sC, bvec); break;
    }
}

}  // namespace

void launch_splitk_reduce(const float* P, uint32_t splits, float* C, const float* bias, uint32_t M, uint32_t N,
                          uint32_t ldc, uint64_t sC, uint32_t batch, int op, hipStream_t s) {
    const uint64_t plane = static_cast<uint64_t>(M) * N;
    if (op == 0) launch_reduce_op<0>(P, plane, splits, C, bias, M, N, ldc, sC, batch, s);
    else if (op == 1) launch_reduce_op<1>(P, plane, splits, C, bias, M, N, ldc, sC, batch, s);
    else launch_reduce_op<2>(P, plane, splits, C, bias, M, N, ldc, sC, batch, s);
}

namespace {

// ---- configurations -------------------------------------------------------------

// Tile shapes (BM x BN, waves WM x WN, two 32-wide K blocks per step) of the
// LDS kernel (gemm_q8_kernel). The 256x256 tile keeps one register set in
// flight (PF = 1) to stay within 256 VGPRs.
enum CfgId {
    kC256x128 = 0, kC128x128, kC128x64, kC64x64, kC256x256,  // 8 / 4 / 4 / 4 / 8 waves
    kC192x256,                                                // 8 waves of 96x64
    kC128x128W8,                                              // 8 waves of 32x64
    kNumCfg
};
static_assert(kNumCfg == kGemmBuilds, "mi_tuning_set bounds gemm_cfg by kGemmBuilds");

// Group height for the tile order: the XCD chunks (blocks b with b % 8 == x,
// contiguous in the grouped order) each read the A panels of the rows and the
// W panels of the columns they cover; pick the height that minimises the sum
// over chunks (A panel = BM*K*4 bytes, W panel = BN*K*34/32 bytes).
uint32_t pick_group(uint32_t tm, uint32_t tn, uint32_t BM, uint32_t BN, uint32_t K) {
    const uint64_t tiles = static_cast<uint64_t>(tm) * tn;
    if (tiles <= 8 || tiles > 65536) return tm;
    const double pa = static_cast<double>(BM) * K * 4, pw = static_cast<double>(BN) * K * 34.0 / 32.0;
    uint32_t best = tm;
    double best_cost = 1e300;
    for (uint32_t gm = 1;; gm *= 2) {
        const uint32_t g = std::min(gm, tm);
        const uint64_t per = tiles / 8, extra = tiles % 8;
        double cost = 0;
        uint64_t start = 0;
        for (uint32_t x = 0; x < 8; ++x) {
            const uint64_t len = per + (x < extra ? 1 : 0);
            // rows / columns touched by grouped-order positions [start, start + len)
            uint32_t rmin = tm, rmax = 0, cmin = tn, cmax = 0;
            uint64_t pos = start;
            while (pos < start + len) {
                const uint64_t gsz = static_cast<uint64_t>(g) * tn;
                const uint64_t grp = pos / gsz, off = pos % gsz;
                const uint32_t rows_in = std::min<uint32_t>(g, tm - static_cast<uint32_t>(grp) * g);
                const uint64_t take = std::min<uint64_t>(start + len - pos, static_cast<uint64_t>(rows_in) * tn - off);
                const uint32_t c0 = static_cast<uint32_t>(off / rows_in), c1 = static_cast<uint32_t>((off + take - 1) / rows_in);
                const uint32_t r0 = static_cast<uint32_t>(grp) * g;
                const uint32_t rlast = take >= rows_in ? r0 + rows_in - 1 : std::max(r0 + static_cast<uint32_t>(off % rows_in), r0 + static_cast<uint32_t>((off + take - 1) % rows_in));
                const uint32_t rfirst = take >= rows_in ? r0 : std::min(r0 + static_cast<uint32_t>(off % rows_in), r0 + static_cast<uint32_t>((off + take - 1) % rows_in));
                rmin = std::min(rmin, rfirst);
                rmax = std::max(rmax, rlast);
                cmin = std::min(cmin, c0);
                cmax = std::max(cmax, c1);
                pos += take;
            }
            if (len) cost += (rmax - rmin + 1) * pa + (cmax - cmin + 1) * pw;
            start += len;
        }
        // near-equal cross-XCD costs: prefer a group height near 4 (32 resident
        // workgroups per XCD then form a 4 x 8 block: reuse inside the XCD)
        const auto dist = [](uint32_t v) { return v > 4 ? v / 4 : 4 / v; };
        if (cost < best_cost * 0.999 || (cost <= best_cost * 1.001 && dist(g) < dist(best))) {
            best_cost = std::min(cost, best_cost);
            best = g;
        }
        if (g >= tm) break;
    }
    return best;
}

// The partial planes of a K split: the kernel's C becomes the workspace
// (row stride N, split planes M * N apart, batch items splits planes apart).
GemmArgs partial_args(const GemmArgs& a, uint32_t splits, float* ws) {
    GemmArgs p = a;
    p.C = ws;
    p.ldc = a.N;
    p.split_stride = static_cast<uint64_t>(a.M) * a.N;
    p.sC = p.split_stride * splits;
    return p;
}

// Adds the partial planes into C in split order (reduce op from the epilogue / mode).
template <int EPI>
void finish_split(const GemmArgs& a, uint32_t splits, const float* ws, uint32_t batch, hipStream_t s) {
    const int op = EPI == kEpiResidual ? 2 : a.mode == 0 ? 0 : 1;
    launch_splitk_reduce(ws, splits, a.C, a.bias, a.M, a.N, a.ldc, a.sC, batch, op, s);
}

// SPLIT = false: a build without a K-split variant (requested splits are ignored).
// splits > 1 needs ws: batch * splits * M * N floats (split_workspace_floats).
template <int BM, int BN, int WM, int WN, int KB, int WK, bool KTAIL, int PF = 2, int EPI = kEpiPlain,
          bool SPLIT = true, bool AH = false, bool PP = false>
void launch_cfg(const GemmArgs& a0, uint32_t batch, uint32_t splits, float* ws, hipStream_t s) {
    GemmArgs a = a0;
    // GEGLU: BN / 2 outputs per tile, and the epilogue needs the whole K sum
    a.tiles_n = EPI == kEpiGeglu ? ceil_div(a.F, BN / 2) : ceil_div(a.N, BN);
    if (EPI == kEpiGeglu || !SPLIT || !ws) splits = 1;
    a.tiles_m = ceil_div(a.M, BM);
    a.group_m = pick_group(a.tiles_m, a.tiles_n, BM, BN, a.K);
    a.ksteps = ceil_div(a.K, 32 * KB);
    const unsigned tiles = ceil_div(a.M, BM) * a.tiles_n;
    if (splits > 1) {
        a.steps_per_split = ceil_div(a.ksteps, splits);
        splits = ceil_div(a.ksteps, a.steps_per_split);
    }
    if (splits > 1) {
        if constexpr (EPI != kEpiGeglu && SPLIT) {
            const GemmArgs p = partial_args(a, splits, ws);
            gemm_q8_kernel<BM, BN, WM, WN, KB, WK, true, KTAIL, PF, kEpiPlain, AH, PP>
                <<<dim3(tiles, splits, batch), WM * WN * 64, 0, s>>>(p);
            finish_split<EPI>(a, splits, ws, batch, s);
        }
    } else {
        a.steps_per_split = a.ksteps;
        gemm_q8_kernel<BM, BN, WM, WN, KB, WK, false, KTAIL, PF, EPI, AH, PP>
            <<<dim3(tiles, 1, batch), WM * WN * 64, 0, s>>>(a);
    }
}

template <int WK, int EPI = kEpiPlain, bool AH = false>
void launch(int cfg, const GemmArgs& a, uint32_t batch, uint32_t splits, float* ws, hipStream_t s) {
    switch (cfg) {
        case kC256x128:
            // ping-pong K loop (PP): 2048x3840x1280 34.3 vs 36.0 us, 2048x1280x5120 in
            // three K splits 50.7 vs 53.6 (one-barrier loop; fp16 A 3-4% faster)
            launch_cfg<256, 128, 4, 2, 2, WK, false, 2, EPI, true, AH, true>(a, batch, splits, ws, s);
            break;
        case kC128x128:
            // one register set: the loop then issues most of a step's MFMAs before
            // converting the next step's loads (8192x640x2560 58 vs 68 us with two
            // sets, 2048x1280x5120 71 vs 76, 8192x640x640 20 vs 22, the rest equal)
            launch_cfg<128, 128, 2, 2, 2, WK, false, 1, EPI, true, AH>(a, batch, splits, ws, s);
            break;
        case kC192x256:
            // two wave groups alternating MFMA and staging halves (PP): 1-3% faster
            // than the one-barrier loop on the shapes the rules give this build
            // (2048x10240x1280 78.6 vs 80.7 us, 2048x3840x1280 36.0 vs 37.2)
            launch_cfg<192, 256, 2, 4, 2, WK, false, 2, EPI, true, AH, true>(a, batch, splits, ws, s);
            break;
        case kC128x128W8:
            // grids of one workgroup per CU: two waves per SIMD instead of one
            launch_cfg<128, 128, 4, 2, 2, WK, false, 2, EPI, true, AH>(a, batch, splits, ws, s);
            break;
        case kC128x64: launch_cfg<128, 64, 2, 2, 2, WK, false, 2, EPI, true, AH>(a, batch, splits, ws, s); break;
        case kC256x256:
            // The split layout's and the GEGLU epilogue's 256x256 builds need
            // more than the 256 VGPRs of a wave at two waves per SIMD: the
            // compiler spills LDS addresses inside the K loop, and every
            // scratch reload waits for all global loads in flight. They run
            // 256x128 tiles instead.
            if constexpr (WK == kSplit || EPI == kEpiGeglu)
                launch_cfg<256, 128, 4, 2, 2, WK, false, 2, EPI, true, AH>(a, batch, splits, ws, s);
            else
                launch_cfg<256, 256, 4, 2, 2, WK, false, 1, EPI, true, AH>(a, batch, splits, ws, s);
            break;
        default: launch_cfg<64, 64, 2, 2, 2, WK, false, 2, EPI, true, AH>(a, batch, splits, ws, s); break;
    }
}

// General K (K % 64 != 0): one block column per step, 64x64 tiles; the split
// layout with K % 32 != 0 also zero-fills the partial last step.
template <int WK, int EPI = kEpiPlain, bool AH = false>
void launch_general(const GemmArgs& a, uint32_t batch, uint32_t splits, float* ws, hipStream_t s) {
    if (a.K % 32 == 0) launch_cfg<64, 64, 2, 2, 1, WK, false, 2, EPI, true, AH>(a, batch, splits, ws, s);
    else launch_cfg<64, 64, 2, 2, 1, WK, true, 2, EPI, true, AH>(a, batch, splits, ws, s);
}

constexpr int kCUs = 256;

struct Plan {
    int cfg;
    uint32_t splits;
};

// Picks the tile and K split for a shape (rules from per-shape sweeps of every
// tile build on MI355X over the SDXL shapes, timed interleaved): the 192x256
// tile (8 waves, one workgroup per CU) where it yields a wave or more of
// long-K tiles over more than 640 columns (at N = 640 the 128x128 tile is
// faster: 8192x640x2560 61.6 vs 66.0 us), or 256x128 where that fills more of
// a single round; among the grids of at least 160 128x128 tiles, 256x128 (8
// waves, ping-pong) where it makes 160 tiles or more, else 128x128 (4 waves,
// two workgroups per CU), as 8 waves of 32x64 when the grid has fewer tiles
// than CUs and no K split (one workgroup per CU: two waves per SIMD instead
// of one; 2048x1280x1280 17.6 vs 21.8 us, 2048x1280x5120 unsplit 60.5 vs
// 89.5); 64x64 for the rest.
// With a workspace (allow_split), long-K (>= 4096) 128x128 grids of fewer
// tiles than CUs run as 256x128 tiles (8 waves) with K split into the most
// parts (>= 1024 k each) that keep one round (2048x1280x5120: 80 tiles x 3 =
// 240 workgroups, 52.3 us against 54.1 us for 128x128 tiles in 3 parts with
// fp32 A and 45.6 against 48.6 with fp16 A; 128x128 in 3 parts had beaten 2
// and 4 parts, 55.2 against 67.7 and 69.4 us), and small 64x64 grids split K
// until ~256 workgroups run.
Plan choose(uint32_t M, uint32_t N, uint32_t K, uint32_t batch, bool allow_split) {
    Plan p{kC64x64, 1};
    // mi_tuning_set("gemm_cfg", "<cfg>[:<splits>]") pins a build (tuning sweeps, tests)
    const int forced = tuning().gemm_cfg.load(std::memory_order_relaxed);
    if (forced >= 0) {
        p.cfg = forced < kNumCfg ? forced : kC64x64;
        p.splits = allow_split ? static_cast<uint32_t>(std::max(1, tuning().gemm_splits.load(std::memory_order_relaxed)))
                               : 1u;
        return p;
    }
    auto tiles = [&](uint32_t bm, uint32_t bn) {
        return static_cast<uint64_t>(ceil_div(M, bm)) * ceil_div(N, bn) * batch;
    };
    const uint64_t t192 = tiles(192, 256), t128 = tiles(128, 128), t64 = tiles(64, 64), t256 = tiles(256, 128);
    if (t192 >= 120 && K >= 1280 && N > 640) {
        // under one round, 256x128 tiles fill more CUs where they still fit one
        // (the block's joint Q/K/V 2048x3840x1280: 240 against 165 tiles, 30.9
        // against 32.7 us with fp16 A)
        p.cfg = t192 < kCUs && t256 > t192 && t256 <= kCUs ? kC256x128 : kC192x256;
    } else if (t128 >= 160) {
        p.cfg = kC128x128;
        if (t256 >= 160) {
            // grids of at least 160 256x128 tiles: the 8-wave ping-pong build
            // (8192x640x2560 48.4 vs 50.9 us, 8192x640x640 17.1 vs 17.8,
            // 8192x5120x640 90.5 vs 91.7; with fp16 A 5-9% faster)
            p.cfg = kC256x128;
        } else if (allow_split && t128 < kCUs && K >= 4096) {
            p.cfg = kC256x128;
            p.splits = static_cast<uint32_t>(std::max<uint64_t>(2, std::min<uint64_t>(kCUs / t256, K / 1024)));
        } else if (t128 < kCUs) {
            p.cfg = kC128x128W8;
        }
    } else {
        p.cfg = kC64x64;
        if (allow_split && t64 < 2 * kCUs) {
            const uint64_t want = (kCUs + t64 - 1) / t64;
            uint32_t sp = 1;
            while (sp * 2 <= want && sp * 2 * 128 <= K) sp *= 2;
            p.splits = sp;
        }
    }
    return p;
}

// Floats of workspace a K-split plan uses: one [M, N] partial plane per split
// and batch item.
uint64_t split_floats(uint32_t M, uint32_t N, uint32_t batch, uint32_t splits) {
    return splits > 1 ? static_cast<uint64_t>(batch) * splits * M * N : 0;
}

// The plan for a call: a split plan only when the caller's workspace holds
// its partials, else the best plan without a split.
Plan plan_for(uint32_t M, uint32_t N, uint32_t K, uint32_t batch, const void* ws, uint64_t ws_bytes) {
    Plan p = choose(M, N, K, batch, ws != nullptr);
    if (p.splits > 1 && split_floats(M, N, batch, p.splits) * 4 > ws_bytes) p = choose(M, N, K, batch, false);
    return p;
}

template <int WK, int EPI = kEpiPlain, bool AH = false>
void dispatch(const GemmArgs& a, uint32_t batch, const Plan& p, float* ws, hipStream_t s) {
    if (a.K % 64 != 0) launch_general<WK, EPI, AH>(a, batch, p.splits, ws, s);
    else launch<WK, EPI, AH>(p.cfg, a, batch, p.splits, ws, s);
}

// ---- any-K kernel (split layout) ---------------------------------------------------
//
// The reference's scalar gemm_nt_q8 accepts any K and any row stride
// (gemm_nt_q8.comp:52-80 stages element by element with bounds checks). Shapes
// the tiled kernels do not take (K % 4 != 0, lda or sA not a multiple of 4, A
// not 16-byte aligned) run here: 64 x 64 tiles, four waves of one 32 x 32 MFMA
// tile, 32 k per step, every element staged with its own bounds check
// (zero past K). The arithmetic is the tiled kernels': A rounded to fp16, the
// weight fp16(q * s), fp32 MFMA sums.
__global__ __launch_bounds__(256) void gemm_q8_any_kernel(GemmArgs a) {
    constexpr int LD = 40;  // halves per staged row: 32 k + 16-byte pad
    __shared__ __attribute__((aligned(16))) _Float16 As[64 * LD];
    __shared__ __attribute__((aligned(16))) _Float16 Ws[64 * LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t n0 = blockIdx.x * 64, m0 = blockIdx.y * 64;
    const float* A = a.A + static_cast<uint64_t>(blockIdx.z) * a.sA;
    const int8_t* q = reinterpret_cast<const int8_t*>(a.W);
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    // this thread stages row (tid / 4) of both tiles, k = 8 (tid % 4) .. + 7
    const uint32_t sr = tid >> 2, sk = (tid & 3) * 8;
    const uint32_t am = min(m0 + sr, a.M - 1), wr = min(n0 + sr, a.N - 1);
    for (uint32_t k0 = 0; k0 < a.K; k0 += 32) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t k = k0 + sk + e;
            float av = 0.0f, wv = 0.0f;
            if (k < a.K) {
                av = A[static_cast<uint64_t>(am) * a.lda + k];
                const uint64_t f = static_cast<uint64_t>(wr) * a.K + k;
                wv = static_cast<float>(q[f]) * a.scales[f >> 5];
            }
            As[sr * LD + sk + e] = static_cast<_Float16>(av);
            Ws[sr * LD + sk + e] = static_cast<_Float16>(wv);
        }
        __syncthreads();
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            const half8 af = *reinterpret_cast<const half8*>(&As[(wm * 32 + l32) * LD + 16 * sl + 8 * g]);
            const half8 bf = *reinterpret_cast<const half8*>(&Ws[(wn * 32 + l32) * LD + 16 * sl + 8 * g]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    // lane holds column n = l32 and rows 8 (r / 4) + 4 g + r % 4 of the wave's tile
    const uint32_t n = n0 + wn * 32 + l32;
    if (n >= a.N) return;
    float* C = a.C + static_cast<uint64_t>(blockIdx.z) * a.sC;
    const float b = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t m = m0 + wm * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m >= a.M) continue;
        float* c = C + static_cast<uint64_t>(m) * a.ldc + n;
        if (a.mode == 0) *c = a.bias ? acc[r] + b : acc[r];
        else if (a.mode == 1) *c = *c + acc[r];
        else *c = *c + (a.bias ? acc[r] + b : acc[r]);
    }
}

// vec_a: the tiled kernels' A path (16-byte loads) -- A 16-byte aligned, lda
// and sA multiples of 4; otherwise A only needs 4-byte alignment (the any-K
// kernel of the split layout).
// a_half: A is fp16 (the 16-byte path then needs lda and sA multiples of 8).
int validate(const char* fn, const void* A, const void* W, const void* C, uint32_t M, uint32_t N, uint32_t K,
             uint32_t mode, uint32_t& lda, uint32_t& ldc, uint32_t batch, uint64_t sA, uint64_t sC, bool vec_a,
             bool a_half = false) {
    if (!A || !W || !C) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (mode > 2)
        return fail(MI_ERR_INVALID_ARG, "%s: mode %u (0 = store, 1 = accumulate, 2 = accumulate + bias)", fn, mode);
    if (batch == 0) return fail(MI_ERR_INVALID_ARG, "%s: batch 0", fn);
    if (batch > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: batch %u > 65535", fn, batch);
    if (lda == 0) lda = K;
    if (ldc == 0) ldc = N;
    if (lda < K || ldc < N) return fail(MI_ERR_INVALID_ARG, "%s: lda %u < K %u or ldc %u < N %u", fn, lda, K, ldc, N);
    const uint32_t av = a_half ? 8 : 4;  // elements per 16-byte unit
    if (vec_a && (!aligned(A, 16) || lda % av || sA % av))
        return fail(MI_ERR_ALIGNMENT, "%s: A must be 16-byte aligned, lda and sA multiples of %u", fn, av);
    if (!aligned(A, 4)) return fail(MI_ERR_ALIGNMENT, "%s: A must be 4-byte aligned", fn);
    if (!aligned(C, 4)) return fail(MI_ERR_ALIGNMENT, "%s: C must be 4-byte aligned", fn);
    // per-workgroup A offsets are 32-bit: a 256-row panel must stay below 4 GiB
    if (static_cast<uint64_t>(lda) * 4 * 256 >= (uint64_t(1) << 32))
        return fail(MI_ERR_UNSUPPORTED, "%s: lda=%u too large", fn, lda);
    return MI_OK;
}

// Workspace of a *_ws call: 16-byte aligned, disjoint from every operand.
int check_ws(const char* fn, const void* ws, uint64_t ws_bytes, const void* A, uint64_t abytes, const void* W,
             uint64_t wbytes, const void* C, uint64_t cbytes, const float* bias, uint32_t N) {
    if (!ws || ws_bytes == 0) return MI_OK;
    if (!aligned(ws, 16)) return fail(MI_ERR_ALIGNMENT, "%s: workspace must be 16-byte aligned", fn);
    if (overlaps(ws, ws_bytes, A, abytes) || overlaps(ws, ws_bytes, W, wbytes) || overlaps(ws, ws_bytes, C, cbytes) ||
        overlaps(ws, ws_bytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: workspace overlaps an operand", fn);
    return MI_OK;
}

// fixed_ws: `ws` is the library's fixed-size scratch (the no-allocation
// entry): a plan whose K-split partials exceed it is an error, not a reason to
// run unsplit, so that the entry's results always equal the workspace entry's.
// a_half: A holds fp16 values (mi_gemm_nt_q8_0_f16a), else fp32.
int gemm_blocks(const char* fn, const void* A, const void* W, const float* bias, float* C, uint32_t M, uint32_t N,
                uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sC,
                void* ws, uint64_t ws_bytes, hipStream_t stream, bool fixed_ws = false, bool a_half = false) {
    if (M == 0 || N == 0) return MI_OK;
    if (K % 32) return fail(MI_ERR_UNSUPPORTED, "%s: K=%u is not a multiple of 32 (Q8_0 block)", fn, K);
    int st = validate(fn, A, W, C, M, N, K, mode, lda, ldc, batch, sA, sC, true, a_half);
    if (st) return st;
    if (!aligned(W, 16)) return fail(MI_ERR_ALIGNMENT, "%s: W must be 16-byte aligned", fn);
    const uint64_t wbytes = static_cast<uint64_t>(N) * (K / 32) * 34;
    if (wbytes + 16 >= (uint64_t(1) << 32)) return fail(MI_ERR_UNSUPPORTED, "%s: weight >= 4 GiB", fn);
    const uint64_t cbytes = (static_cast<uint64_t>(batch - 1) * sC + static_cast<uint64_t>(M - 1) * ldc + N) * 4;
    const uint64_t abytes =
        (static_cast<uint64_t>(batch - 1) * sA + static_cast<uint64_t>(M - 1) * lda + K) * (a_half ? 2 : 4);
    if (overlaps(C, cbytes, A, abytes) || overlaps(C, cbytes, W, wbytes) || overlaps(C, cbytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: C overlaps an input", fn);
    st = check_ws(fn, ws, ws_bytes, A, abytes, W, wbytes, C, cbytes, bias, N);
    if (st) return st;
    if (K == 0) {
        if (mode == 0 || (mode == 2 && bias)) launch_fill(C, bias, M, N, ldc, sC, batch, mode == 2, stream);
        return check_launch(fn);
    }
    if (fixed_ws) {
        const Plan want = choose(M, N, K, batch, true);
        const uint64_t need = split_floats(M, N, batch, want.splits) * 4;
        if (need > ws_bytes)
            return fail(MI_ERR_UNSUPPORTED,
                        "%s: M=%u N=%u K=%u batch=%u plans %u K splits whose partials need %llu bytes of scratch; "
                        "the maximum is %llu bytes (use mi_gemm_nt_q8_0_ws with a larger workspace)",
                        fn, M, N, K, batch, want.splits, static_cast<unsigned long long>(need),
                        static_cast<unsigned long long>(ws_bytes));
    }
    GemmArgs a = make_args(static_cast<const float*>(A), static_cast<const uint8_t*>(W), nullptr, bias, C, M, N, K,
                           mode, lda, ldc, sA, sC, (K / 32) * 34);
    const Plan p = plan_for(M, N, K, batch, ws, ws_bytes);
    float* wsf = static_cast<float*>(ws);
    if (a_half) {
        if (mode == 2) dispatch<kBlocks34, kEpiResidual, true>(a, batch, p, wsf, stream);
        else dispatch<kBlocks34, kEpiPlain, true>(a, batch, p, wsf, stream);
    } else {
        if (mode == 2) dispatch<kBlocks34, kEpiResidual>(a, batch, p, wsf, stream);
        else dispatch<kBlocks34>(a, batch, p, wsf, stream);
    }
    return check_launch(fn);
}

int gemm_split(const char* fn, const float* A, const uint32_t* payload, const float* scales, const float* bias,
               float* C, uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
               uint32_t batch, uint64_t sA, uint64_t sC, void* ws, uint64_t ws_bytes, hipStream_t stream) {
    if (M == 0 || N == 0) return MI_OK;
    const uint32_t lda_e = lda ? lda : K;
    // the tiled kernels stage A 16 bytes at a time; other shapes take the any-K kernel
    const bool tiled = K % 4 == 0 && lda_e % 4 == 0 && sA % 4 == 0 && aligned(A, 16);
    int st = validate(fn, A, payload, C, M, N, K, mode, lda, ldc, batch, sA, sC, false);
    if (st) return st;
    if (!scales) return fail(MI_ERR_INVALID_ARG, "%s: null scales", fn);
    if (!aligned(payload, 4) || !aligned(scales, 4)) return fail(MI_ERR_ALIGNMENT, "%s: payload/scales alignment", fn);
    const uint64_t nk = static_cast<uint64_t>(N) * K;
    if (nk + 16 >= (uint64_t(1) << 32)) return fail(MI_ERR_UNSUPPORTED, "%s: weight >= 4 GiB", fn);
    const uint64_t cbytes = (static_cast<uint64_t>(batch - 1) * sC + static_cast<uint64_t>(M - 1) * ldc + N) * 4;
    const uint64_t abytes = (static_cast<uint64_t>(batch - 1) * sA + static_cast<uint64_t>(M - 1) * lda + K) * 4;
    if (overlaps(C, cbytes, A, abytes) || overlaps(C, cbytes, payload, nk) ||
        overlaps(C, cbytes, scales, (nk + 31) / 32 * 4) || overlaps(C, cbytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: C overlaps an input", fn);
    st = check_ws(fn, ws, ws_bytes, A, abytes, payload, nk, C, cbytes, bias, N);
    if (st) return st;
    if (K == 0) {
        if (mode == 0 || (mode == 2 && bias)) launch_fill(C, bias, M, N, ldc, sC, batch, mode == 2, stream);
        return check_launch(fn);
    }
    GemmArgs a = make_args(A, reinterpret_cast<const uint8_t*>(payload), scales, bias, C, M, N, K, mode, lda, ldc, sA,
                           sC, 0);
    if (!tiled) {
        gemm_q8_any_kernel<<<dim3(ceil_div(N, 64), ceil_div(M, 64), batch), 256, 0, stream>>>(a);
        return check_launch(fn);
    }
    const Plan p = plan_for(M, N, K, batch, ws, ws_bytes);
    if (mode == 2) dispatch<kSplit, kEpiResidual>(a, batch, p, static_cast<float*>(ws), stream);
    else dispatch<kSplit>(a, batch, p, static_cast<float*>(ws), stream);
    return check_launch(fn);
}

// ---- no-allocation entry -------------------------------------------------------------
//
// Scratch of mi_gemm_nt_q8_0_noalloc: the K-split partial planes live in this
// file-scope device array instead of a caller workspace. The runtime gives
// each GPU its own copy when the code object loads there, and it stays until
// the process ends. Host code never passes `scratch` itself to a kernel (on
// the host the name is only a stand-in, not a device address): the entry
// looks up the device address once per GPU with hipGetSymbolAddress and uses
// that pointer everywhere. Every call on a GPU shares its copy, so calls that
// overlap on one GPU (different streams without ordering) race. Nothing in it
// must start at zero: each split stores every element of its partial plane
// before the reduce kernel reads it.
constexpr uint64_t kScratchBytes = MI_GEMM_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) float scratch[kScratchBytes / 4];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current GPU's scratch, looked up on its first use.
// The lookup can load the code object on that GPU, which has no place inside
// a stream capture: with `capturing` set and no address yet, the call fails
// instead (mi_gemm_noalloc_init does the lookup beforehand).
int scratch_on_current_device(const char* fn, void** out, hipStream_t stream = nullptr, bool check_capture = false) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(MI_ERR_UNSUPPORTED, "%s: device index %d >= %d", fn, dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev] && check_capture) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: hipStreamIsCapturing: %s", fn, hipGetErrorString(e));
        if (cs != hipStreamCaptureStatusNone)
            return fail(MI_ERR_UNSUPPORTED, "%s: first call on device %d inside a stream capture: call "
                        "mi_gemm_noalloc_init() on the device before capturing", fn, dev);
    }
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(MI_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_gemm_nt_q8_0_noalloc(const float* A, const void* W, const float* bias, float* C, uint32_t M,
                                       uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
                                       uint32_t batch, uint64_t sA, uint64_t sC, void* stream) {
    const char* fn = "mi_gemm_nt_q8_0_noalloc";
    if (M == 0 || N == 0) return MI_OK;
    void* ws = nullptr;
    const int st = scratch_on_current_device(fn, &ws, static_cast<hipStream_t>(stream), true);
    if (st) return st;
    return gemm_blocks(fn, A, W, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC, ws, kScratchBytes,
                       static_cast<hipStream_t>(stream), true);
}

extern "C" int mi_gemm_noalloc_init(void) {
    void* ws = nullptr;
    return scratch_on_current_device("mi_gemm_noalloc_init", &ws);
}

extern "C" int mi_gemm_nt_q8_0(const float* A, const void* W, const float* bias, float* C, uint32_t M, uint32_t N,
                               uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA,
                               uint64_t sC, void* stream) {
    return gemm_blocks("mi_gemm_nt_q8_0", A, W, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC, nullptr, 0,
                       static_cast<hipStream_t>(stream));
}

extern "C" int mi_gemm_nt_q8_0_ws(const float* A, const void* W, const float* bias, float* C, uint32_t M, uint32_t N,
                                  uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA,
                                  uint64_t sC, void* workspace, uint64_t workspace_bytes, void* stream) {
    return gemm_blocks("mi_gemm_nt_q8_0_ws", A, W, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC, workspace,
                       workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int mi_gemm_nt_q8_split(const float* A, const uint32_t* payload, const float* scales, const float* bias,
                                   float* C, uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda,
                                   uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sC, void* stream) {
    return gemm_split("mi_gemm_nt_q8_split", A, payload, scales, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC,
                      nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int mi_gemm_nt_q8_split_ws(const float* A, const uint32_t* payload, const float* scales,
                                      const float* bias, float* C, uint32_t M, uint32_t N, uint32_t K, uint32_t mode,
                                      uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sC,
                                      void* workspace, uint64_t workspace_bytes, void* stream) {
    return gemm_split("mi_gemm_nt_q8_split_ws", A, payload, scales, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC,
                      workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" uint64_t mi_gemm_nt_q8_workspace_bytes(uint32_t M, uint32_t N, uint32_t K, uint32_t batch) {
    if (M == 0 || N == 0 || K == 0 || batch == 0) return 0;
    const Plan p = choose(M, N, K, batch, true);
    return split_floats(M, N, batch, p.splits) * 4;
}

namespace mi {
namespace {
int gemm_geglu(const char* fn, const void* A, const void* W, const float* bias, void* G, uint32_t M, uint32_t F,
               uint32_t K, uint32_t lda, uint32_t ldg, hipStream_t stream, bool a_half, bool g_half) {
    if (M == 0 || F == 0) return MI_OK;
    if (K == 0 || K % 32) return fail(MI_ERR_UNSUPPORTED, "%s: K=%u must be a positive multiple of 32", fn, K);
    if (F > (1u << 30)) return fail(MI_ERR_UNSUPPORTED, "%s: F=%u too large", fn, F);
    const uint32_t N = 2 * F;
    uint32_t ldc = ldg, mode = 0;
    int st = validate(fn, A, W, G, M, F, K, mode, lda, ldc, 1, 0, 0, true, a_half);
    if (st) return st;
    if (!aligned(W, 16)) return fail(MI_ERR_ALIGNMENT, "%s: W must be 16-byte aligned", fn);
    if (g_half && !aligned(G, 8)) return fail(MI_ERR_ALIGNMENT, "%s: G must be 8-byte aligned", fn);
    const uint64_t wbytes = static_cast<uint64_t>(N) * (K / 32) * 34;
    if (wbytes + 16 >= (uint64_t(1) << 32)) return fail(MI_ERR_UNSUPPORTED, "%s: weight >= 4 GiB", fn);
    const uint64_t gbytes = (static_cast<uint64_t>(M - 1) * ldc + F) * (g_half ? 2 : 4);
    const uint64_t abytes = (static_cast<uint64_t>(M - 1) * lda + K) * (a_half ? 2 : 4);
    if (overlaps(G, gbytes, A, abytes) || overlaps(G, gbytes, W, wbytes) || overlaps(G, gbytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: G overlaps an input", fn);
    GemmArgs a = make_args(static_cast<const float*>(A), static_cast<const uint8_t*>(W), nullptr, bias,
                           static_cast<float*>(G), M, N, K, 0, lda, ldc, 0, 0, (K / 32) * 34);
    a.F = F;
    a.out_half = g_half ? 1u : 0u;
    if (g_half)  // 8-byte stores of four fp16 outputs
        a.cvec = aligned(G, 8) && ldc % 4 == 0 ? 1u : 0u;
    // the GEGLU epilogue needs the whole K sum: never split
    const Plan p = plan_for(M, N, K, 1, nullptr, 0);
    if (a_half) dispatch<kBlocks34, kEpiGeglu, true>(a, 1, p, nullptr, stream);
    else dispatch<kBlocks34, kEpiGeglu>(a, 1, p, nullptr, stream);
    return check_launch(fn);
}
}  // namespace
}  // namespace mi

extern "C" int mi_gemm_nt_q8_0_geglu(const float* A, const void* W, const float* bias, float* G, uint32_t M, uint32_t F,
                                     uint32_t K, uint32_t lda, uint32_t ldg, void* stream) {
    return gemm_geglu("mi_gemm_nt_q8_0_geglu", A, W, bias, G, M, F, K, lda, ldg, static_cast<hipStream_t>(stream),
                      false, false);
}

extern "C" int mi_gemm_nt_q8_0_geglu_f16(const void* A, const void* W, const float* bias, void* G, uint32_t M,
                                         uint32_t F, uint32_t K, uint32_t lda, uint32_t ldg, void* stream) {
    return gemm_geglu("mi_gemm_nt_q8_0_geglu_f16", A, W, bias, G, M, F, K, lda, ldg,
                      static_cast<hipStream_t>(stream), true, true);
}

namespace mi {
namespace {
// C (fp16) = A . W^T (+ bias), one RNE rounding of the fp32 result; A fp32 or
// fp16 (a_half). Mode 0 only and never split (no workspace), so the result is
// the rounding of the unsplit fp32 GEMM's bits.
int gemm_f16out(const char* fn, const void* A, bool a_half, const void* W, const float* bias, void* C, uint32_t M,
                uint32_t N, uint32_t K, uint32_t lda, uint32_t ldc, hipStream_t stream) {
    if (M == 0 || N == 0) return MI_OK;
    if (K == 0 || K % 32) return fail(MI_ERR_UNSUPPORTED, "%s: K=%u must be a positive multiple of 32", fn, K);
    uint32_t mode = 0;
    int st = validate(fn, A, W, C, M, N, K, mode, lda, ldc, 1, 0, 0, true, a_half);
    if (st) return st;
    if (!aligned(W, 16)) return fail(MI_ERR_ALIGNMENT, "%s: W must be 16-byte aligned", fn);
    const uint64_t wbytes = static_cast<uint64_t>(N) * (K / 32) * 34;
    if (wbytes + 16 >= (uint64_t(1) << 32)) return fail(MI_ERR_UNSUPPORTED, "%s: weight >= 4 GiB", fn);
    const uint64_t cbytes = (static_cast<uint64_t>(M - 1) * ldc + N) * 2;
    const uint64_t abytes = (static_cast<uint64_t>(M - 1) * lda + K) * (a_half ? 2 : 4);
    if (overlaps(C, cbytes, A, abytes) || overlaps(C, cbytes, W, wbytes) || overlaps(C, cbytes, bias, uint64_t(N) * 4))
        return fail(MI_ERR_ALIASING, "%s: C overlaps an input", fn);
    GemmArgs a = make_args(static_cast<const float*>(A), static_cast<const uint8_t*>(W), nullptr, bias,
                           static_cast<float*>(C), M, N, K, 0, lda, ldc, 0, 0, (K / 32) * 34);
    a.out_half = 1u;
    a.cvec = aligned(C, 8) && ldc % 4 == 0 ? 1u : 0u;  // 8-byte stores of four fp16 outputs
    a.bvec = 0u;
    const Plan p = plan_for(M, N, K, 1, nullptr, 0);
    if (a_half) dispatch<kBlocks34, kEpiPlain, true>(a, 1, p, nullptr, stream);
    else dispatch<kBlocks34, kEpiPlain>(a, 1, p, nullptr, stream);
    return check_launch(fn);
}
}  // namespace
}  // namespace mi

extern "C" int mi_gemm_nt_q8_0_f16o(const void* A, uint32_t a_dtype, const void* W, const float* bias, void* C,
                                    uint32_t M, uint32_t N, uint32_t K, uint32_t lda, uint32_t ldc, void* stream) {
    if (a_dtype != MI_F32 && a_dtype != MI_F16)
        return fail(MI_ERR_INVALID_ARG, "mi_gemm_nt_q8_0_f16o: a_dtype %u (MI_F32 or MI_F16)", a_dtype);
    return gemm_f16out("mi_gemm_nt_q8_0_f16o", A, a_dtype == MI_F16, W, bias, C, M, N, K, lda, ldc,
                       static_cast<hipStream_t>(stream));
}

extern "C" int mi_gemm_nt_q8_0_f16a(const void* A, const void* W, const float* bias, float* C, uint32_t M, uint32_t N,
                                    uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA,
                                    uint64_t sC, void* workspace, uint64_t workspace_bytes, void* stream) {
    return gemm_blocks("mi_gemm_nt_q8_0_f16a", A, W, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC, workspace,
                       workspace_bytes, static_cast<hipStream_t>(stream), false, true);
}
