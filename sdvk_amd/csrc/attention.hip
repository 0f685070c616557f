// attention.hip -- fused attention for gfx950: O = softmax(Q K^T * scale + mask) V
//
// Reference behaviour: src/Modules/GPU/fused_attn.cpp:34-61 (support predicate,
// scale 1/sqrt(hd)), shaders/fused_attn_tiled.comp and fused_attn.comp (causal
// and Tk bounds masks, O = 0 when the running sum is 0). The reference's two
// kernels (tiled for Tk >= 256, per-key butterfly otherwise) become one kernel
// here; the algorithm is our own:
//
//   * a workgroup owns 128 queries of one (batch, head): 4 waves x 32 queries;
//   * K and V tiles of 64 keys are staged in LDS as fp16 (double-buffered, the
//     next tile's global loads in flight during the current tile's math);
//   * each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_f16 so that a lane
//     owns one query and 32 of the tile's keys: the row max and row sum are
//     in-register reductions plus one exchange with the partner lane (lane ^ 32);
//   * online softmax in fp32 in the exp2 domain (scale * log2 e folded into one
//     FMA per score), masked scores are -inf, all-masked rows give O = 0. The
//     running max is raised lazily (only when a tile exceeds it by 2^8), so
//     the O / l rescale is skipped on most tiles; masks are applied only on
//     boundary tiles (a wave-uniform branch);
//   * O^T = V^T P^T on the same MFMA: P stays in registers (the S^T output
//     layout is, key for key, the B-operand layout the PV product needs); V is
//     stored in LDS grouped by the PV step that consumes each key, so each A
//     fragment is one 16-byte read; the row sums of P come from the same MFMA
//     (an all-ones A operand) in the fp32-input kernel, and from v_dot2_f32_f16
//     on the fp16 P values in the fp16 kernel (VALU instead of a fifth of its
//     MFMAs);
//   * fp32 inputs (the reference layout) are carried as fp16 hi + lo pairs
//     (x = hi + lo to 2^-22): S = K_hi Q_hi + K_lo Q_hi + K_hi Q_lo and
//     O = V_hi P + V_lo P, so only P is rounded to fp16. fp16 inputs take one
//     MFMA per product.
#include "common.hpp"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace mi {
namespace {

constexpr int kBQ = 128;   // queries per workgroup
constexpr int kBKV = 64;   // keys per tile
constexpr int kKld = 72;   // K tile LDS row stride (halves): 64 d + 8 pad
// V tile LDS layout [G][d][8 keys] with the G stride padded from 64 to 66
// 16-byte units: the staging stores (16 lanes = 16 key groups of one d block)
// then spread over the banks instead of hitting one bank in four.
constexpr int kVG = 66;
constexpr int kThreads = 256;
// floats per key-split piece in the workspace: O rows [kBQ][64], then the running max and the row sum of
// each of the kBQ queries
constexpr uint32_t kPartFloats = kBQ * 64 + 2 * kBQ;

struct AttnArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    uint32_t Tq, Tk, heads, hd;
    int causal;
    uint64_t ldq, ldk, ldv, ldo, sq, sk, sv, so;
    const int32_t* kv_len;
    float c;  // scale * log2(e)
    int ostage;  // output rows and head columns 16-byte aligned: store O through LDS (store_o_rows)
    int precise;  // P's fp16 residual as a second PV product on every tile (mi_attn_precision)
    // Key-split plan of the fp16 kernel (mi_fused_attention_ws): the first nfull query blocks run
    // whole; each later one runs as `pieces` workgroups over consecutive key-tile ranges that write
    // unnormalised partials to `part` (kPartFloats floats per piece), merged by attn_merge_kernel.
    uint32_t nfull, pieces;
    float* part;
};

// 8 consecutive elements as fp16 (hi); for fp32 sources also the residual
// lo = fp16(x - hi), so that hi + lo carries x to 2^-22 relative.
template <typename T>
__device__ __forceinline__ void load8(const T* p, bool vec, int valid, half8& hi, half8& lo) {
    if constexpr (sizeof(T) == 2) {
        if (vec) {
            hi = *reinterpret_cast<const half8*>(p);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) hi[i] = i < valid ? p[i] : static_cast<_Float16>(0.0f);
        }
    } else {
        float x[8];
        if (vec) {
            floatx4 a = reinterpret_cast<const floatx4*>(p)[0];
            floatx4 b = reinterpret_cast<const floatx4*>(p)[1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = a[i];
                x[4 + i] = b[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = i < valid ? p[i] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hi[i] = static_cast<_Float16>(x[i]);
            lo[i] = static_cast<_Float16>(x[i] - static_cast<float>(hi[i]));
        }
    }
}

__device__ __forceinline__ half8 zero8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }

// 4 consecutive elements as fp16 (hi) and, for fp32 sources, the residual lo.
template <typename T>
__device__ __forceinline__ void load4(const T* p, bool vec, int valid, half4& hi, half4& lo) {
    if constexpr (sizeof(T) == 2) {
        if (vec) {
            hi = *reinterpret_cast<const half4*>(p);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) hi[i] = i < valid ? p[i] : static_cast<_Float16>(0.0f);
        }
    } else {
        floatx4 x;
        if (vec) {
            x = *reinterpret_cast<const floatx4*>(p);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = i < valid ? p[i] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hi[i] = static_cast<_Float16>(x[i]);
            lo[i] = static_cast<_Float16>(x[i] - static_cast<float>(hi[i]));
        }
    }
}

// A buffer offset past every record: the load returns zeros. Valid offsets
// stay below it (run() bounds a 64-row tile's extent to 2^30 bytes).
constexpr uint32_t kOob = 0x80000000u;

// Bytes of rows kv0 .. min(kv0 + 64, L) - 1 of a [*, ld] tensor (the last row
// counted up to hd): the record size of one tile's buffer resource, so rows
// at or past L read as zeros.
__device__ __forceinline__ uint32_t tile_bytes(uint32_t kv0, uint32_t L, uint64_t ld, uint32_t hd, uint32_t esz) {
    if (kv0 >= L) return 0u;
    const uint32_t rows = min(L - kv0, 64u);
    return static_cast<uint32_t>(((rows - 1) * ld + hd) * esz);
}

// Four outputs o * inv as fp16: the fp32 products rounded once each (RNE),
// the values an fp32 output would round to in a consumer that stages it as
// fp16 (the block's out-projection GEMM). The empty register constraint keeps the rounding
// from fusing into the multiply (a mixed-precision multiply rounds the exact
// product once, which can differ).
__device__ __forceinline__ half4 half4_of(float a, float b, float c, float d) {
    floatx4 v = {a, b, c, d};
    asm volatile("" : "+v"(v));
    return half4{static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1]), static_cast<_Float16>(v[2]),
                 static_cast<_Float16>(v[3])};
}

// 16 bytes per lane from a buffer into LDS (lane l's bytes land at lds + 16 l).
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
}

// Transposing LDS read: within each 16-lane group, lane i returns element i % 4
// of the 8-byte pieces addressed by lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12.
__device__ __forceinline__ half4 lds_read_tr16(const _Float16* p) {
    typedef __fp16 fp16x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) fp16x4*)(const_cast<_Float16*>(p))));
}

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Writes one wave's O^T accumulators (32 queries x 64 d, times inv) as output
// rows. In the MFMA layout a lane holds 4-element runs of one query's row, so
// a direct store touches 32 rows with 8 or 16 bytes each per instruction; here
// the wave transposes through its own LDS region (32 rows, the 16-byte chunks
// of row q XOR-swizzled by q) and then stores 16 bytes per lane, whole rows
// per instruction. Rows at or past nrows and chunks at or past hd are skipped.
// Needs 16-byte aligned rows and head offsets; lds: 32 * 64 * sizeof(TO) bytes.
template <typename TO>
__device__ __forceinline__ void store_o_rows(const floatx16* o, float inv, char* lds, TO* Ob, int nrows, int hd,
                                             uint64_t ldo, int lane) {
    constexpr int E = sizeof(TO), RB = 64 * E, NC = RB / 16;
    const int q = lane & 31, g = lane >> 5;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int run = 0; run < 4; ++run) {
            const int byte = (32 * u + 8 * run + 4 * g) * E;
            char* p = lds + q * RB + (((byte >> 4) ^ (q & (NC - 1))) << 4) + (byte & 15);
            if constexpr (E == 4) {
                *reinterpret_cast<floatx4*>(p) =
                    floatx4{o[u][4 * run] * inv, o[u][4 * run + 1] * inv, o[u][4 * run + 2] * inv, o[u][4 * run + 3] * inv};
            } else {
                *reinterpret_cast<half4*>(p) = half4_of(o[u][4 * run] * inv, o[u][4 * run + 1] * inv,
                                                        o[u][4 * run + 2] * inv, o[u][4 * run + 3] * inv);
            }
        }
    __builtin_amdgcn_wave_barrier();
    constexpr int RPI = 64 / NC;  // rows per store instruction
    const int c = lane % NC, r0 = lane / NC;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
        const int r = i * RPI + r0;
        const floatx4 v = *reinterpret_cast<const floatx4*>(lds + r * RB + ((c ^ (r & (NC - 1))) << 4));
        if (r < nrows && c * (16 / E) < hd)
            *reinterpret_cast<floatx4*>(reinterpret_cast<char*>(Ob + static_cast<uint64_t>(r) * ldo) + c * 16) = v;
    }
}

// Lazy rescaling threshold (exp2 domain): the running max is only raised when
// a tile's max exceeds it by more than this, so P = exp2(s - m) <= 2^8 stays
// far inside fp16 range while the O / l rescale runs on few tiles.
constexpr float kLazy = 8.0f;
// The fp16 kernel checks the same bound after the exponentials: a lane's sum
// of a tile's P values bounds each of them, so a sum <= 2^kLazy keeps every
// P <= 2^kLazy.
constexpr float kLazySum = 256.0f;

template <typename TI, typename TO, bool VEC>
__global__ __launch_bounds__(kThreads) void attn_kernel(AttnArgs a) {
    constexpr bool kSplit = sizeof(TI) == 4;  // fp32 inputs: hi + lo planes
    constexpr int NP = kSplit ? 2 : 1;
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2][NP][kBKV * kKld];
    __shared__ __attribute__((aligned(16))) _Float16 Vs[2][NP][8 * kVG * 8];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const uint32_t b = blockIdx.z, h = blockIdx.y;
    const uint32_t qcta = blockIdx.x * kBQ;
    const uint32_t qwave = qcta + wave * 32;     // first query of this wave
    const uint32_t qi = qwave + l32;             // this lane's query
    const int hd = static_cast<int>(a.hd);

    uint32_t L = a.Tk;
    if (a.kv_len) {
        int32_t l = a.kv_len[b];
        L = l < 0 ? 0u : (static_cast<uint32_t>(l) < a.Tk ? static_cast<uint32_t>(l) : a.Tk);
    }
    uint32_t kend = L;
    if (a.causal) kend = min(kend, qcta + kBQ);  // keys past the CTA's last query are all masked
    // Tiles [0, kfull) need no mask for any query of this wave.
    uint32_t kfull = L / kBKV * kBKV;
    if (a.causal) kfull = min(kfull, (qwave + 1) / kBKV * kBKV);

    const TI* Qp = static_cast<const TI*>(a.q) + b * a.sq + static_cast<uint64_t>(h) * a.hd;
    const TI* Kp = static_cast<const TI*>(a.k) + b * a.sk + static_cast<uint64_t>(h) * a.hd;
    const TI* Vp = static_cast<const TI*>(a.v) + b * a.sv + static_cast<uint64_t>(h) * a.hd;

    // Q^T fragments (B operand): d = 16 s + 8 g .. +8 of query qi
    half8 qf[4], qlo[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int d0 = 16 * s + 8 * g;
        const int valid = hd - d0;
        qf[s] = zero8();
        qlo[s] = zero8();
        if (qi < a.Tq && valid > 0) load8(Qp + static_cast<uint64_t>(qi) * a.ldq + d0, VEC, valid, qf[s], qlo[s]);
    }

    // Staging. K: chunks of 8 d (thread handles chunks tid and tid + 256: key =
    // c / 8, d0 = 8 (c % 8)), stored row-major. V: a 4-key x 4-d block per
    // thread (key group kg = tid % 16, d0 = 4 (tid / 16)), transposed in
    // registers and stored as [G][d][8] halves, G = (t, sp, g) the PV MFMA step
    // and lane half that consumes the key: key 32t + 16sp + 8j + 4g + i sits in
    // slot 4j + i, so a PV fragment is one 16-byte read and the stores are four
    // 8-byte writes.
    half8 kreg[2][NP];
    half4 vreg[4][NP];
    const int vkg = tid & 15, vd0 = (tid >> 4) * 4;
    // Vector path: K/V rows through buffer resources whose base advances with
    // the tile (scalar work only) and whose size ends at key L-1, so rows past
    // the valid keys read as zeros (hardware range check) with no lane guards.
    // Chunks at d >= hd take an offset past every record (the load returns
    // zeros) instead of reading the neighbouring head's columns.
    const bool kin = (tid & 7) * 8 < hd;
    const uint32_t k_off0 = kin ? ((tid >> 3) * static_cast<uint32_t>(a.ldk) + (tid & 7) * 8) * sizeof(TI) : kOob;
    const uint32_t k_off1 = kin ? k_off0 + 32u * static_cast<uint32_t>(a.ldk) * sizeof(TI) : kOob;
    const uint32_t v_off = vd0 < hd ? (vkg * 4 * static_cast<uint32_t>(a.ldv) + vd0) * sizeof(TI) : kOob;
    const uint32_t v_row = static_cast<uint32_t>(a.ldv) * sizeof(TI);
    auto load_tile = [&](uint32_t kv0) {
        if constexpr (VEC) {
            const uint32_t kbytes = tile_bytes(kv0, L, a.ldk, a.hd, sizeof(TI));
            const uint32_t vbytes = tile_bytes(kv0, L, a.ldv, a.hd, sizeof(TI));
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<TI*>(Kp + static_cast<uint64_t>(kv0) * a.ldk), 0, static_cast<int>(kbytes), 0x00020000);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<TI*>(Vp + static_cast<uint64_t>(kv0) * a.ldv), 0, static_cast<int>(vbytes), 0x00020000);
            if constexpr (sizeof(TI) == 2) {
                kreg[0][0] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, k_off0, 0, 0));
                kreg[1][0] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, k_off1, 0, 0));
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    vreg[i][0] = __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(rv, v_off + i * v_row, 0, 0));
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t off = i ? k_off1 : k_off0;
                    const floatx4 x0 = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
                    const floatx4 x1 = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, off + 16, 0, 0));
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kreg[i][0][e] = static_cast<_Float16>(x0[e]);
                        kreg[i][0][4 + e] = static_cast<_Float16>(x1[e]);
                        kreg[i][NP - 1][e] = static_cast<_Float16>(x0[e] - static_cast<float>(kreg[i][0][e]));
                        kreg[i][NP - 1][4 + e] = static_cast<_Float16>(x1[e] - static_cast<float>(kreg[i][0][4 + e]));
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const floatx4 x = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rv, v_off + i * v_row, 0, 0));
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        vreg[i][0][e] = static_cast<_Float16>(x[e]);
                        vreg[i][NP - 1][e] = static_cast<_Float16>(x[e] - static_cast<float>(vreg[i][0][e]));
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int c = tid + i * kThreads;
                const uint32_t key = kv0 + (c >> 3);
                const int d0 = (c & 7) * 8;
                const int valid = hd - d0;
                half8 klo = zero8();
                kreg[i][0] = zero8();
                if (key < L && valid > 0) load8(Kp + static_cast<uint64_t>(key) * a.ldk + d0, VEC, valid, kreg[i][0], klo);
                if constexpr (kSplit) kreg[i][NP - 1] = klo;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t key = kv0 + vkg * 4 + i;
                const int valid = hd - vd0;
                half4 vlo = half4{0, 0, 0, 0};
                vreg[i][0] = half4{0, 0, 0, 0};
                if (key < L && valid > 0) load4(Vp + static_cast<uint64_t>(key) * a.ldv + vd0, VEC, valid, vreg[i][0], vlo);
                if constexpr (kSplit) vreg[i][NP - 1] = vlo;
            }
        }
    };
    auto store_tile = [&](int st) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kThreads;
            const int key = c >> 3, d0 = (c & 7) * 8;
#pragma unroll
            for (int pl = 0; pl < NP; ++pl) *reinterpret_cast<half8*>(&Ks[st][pl][key * kKld + d0]) = kreg[i][pl];
        }
        // keys 4 vkg .. +3: t = vkg / 8, sp = (vkg / 4) % 2, j = (vkg / 2) % 2, g = vkg % 2
        const int vG = (vkg >> 3) * 4 + ((vkg >> 2) & 1) * 2 + (vkg & 1);
        const int vslot = ((vkg >> 1) & 1) * 4;
#pragma unroll
        for (int pl = 0; pl < NP; ++pl)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                *reinterpret_cast<half4*>(&Vs[st][pl][(vG * kVG + vd0 + e) * 8 + vslot]) =
                    half4{vreg[0][pl][e], vreg[1][pl][e], vreg[2][pl][e], vreg[3][pl][e]};
    };

    // o[0..1]: O^T for d in [0, 32) and [32, 64); o[2]: the row sums of P,
    // computed by the same MFMA with an all-ones A operand (every row of that
    // 32x32 tile holds sum_k P[q, k] for the lane's query q).
    floatx16 o[3];
#pragma unroll
    for (int u = 0; u < 3; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[u][r] = 0.0f;
    float m = -INFINITY;
    const half8 ones = {1, 1, 1, 1, 1, 1, 1, 1};

    const uint32_t ntiles = (kend + kBKV - 1) / kBKV;
    if (ntiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();

    for (uint32_t it = 0; it < ntiles; ++it) {
        const int st = it & 1;
        const uint32_t kv0 = it * kBKV;
        // next tile's loads first (clamped: the last trip re-reads its own tile)
        load_tile(min(it + 1, ntiles - 1) * kBKV);
        __builtin_amdgcn_sched_barrier(0);

        // S^T tile: rows = keys kv0 + 32 t + 8(r/4) + 4 g + r%4, column = query qi
        floatx16 sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[t][r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int off = (32 * t + l32) * kKld + 16 * s + 8 * g;
                half8 kf = *reinterpret_cast<const half8*>(&Ks[st][0][off]);
                sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], sc[t], 0, 0, 0);
                if constexpr (kSplit) {
                    half8 kl = *reinterpret_cast<const half8*>(&Ks[st][NP - 1][off]);
                    sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qf[s], sc[t], 0, 0, 0);
                    sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qlo[s], sc[t], 0, 0, 0);
                }
            }
        }

        if (kv0 >= kfull) {  // wave-uniform: a boundary tile (key padding / Tk end / causal)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t key = kv0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (key >= L || (a.causal && key > qi)) sc[t][r] = -INFINITY;
                }
        }

        float mx = sc[0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[t][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mt = mx * a.c;  // tile max, exp2 domain (same in both lanes of a query)
        if (__any(mt > m + kLazy)) {
            const float m_new = fmaxf(m, mt);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
            m = m_new;
#pragma unroll
            for (int u = 0; u < 3; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[u][r] *= alpha;
        }
        const float m_use = m == -INFINITY ? 0.0f : m;

#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) {
                half8 pf;
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    pf[i] = static_cast<_Float16>(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][8 * sp + i], a.c, -m_use)));
                o[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, pf, o[2], 0, 0, 0);
                const int G = t * 4 + sp * 2 + g;
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int d = 32 * u + l32;
#pragma unroll
                    for (int pl = 0; pl < NP; ++pl) {
                        const half8 vf = *reinterpret_cast<const half8*>(&Vs[st][pl][(G * kVG + d) * 8]);
                        o[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[u], 0, 0, 0);
                    }
                }
            }
        }
        if (a.precise || (a.causal && kv0 >= kfull)) {
            // causal diagonal tile (or every tile under MI_ATTN_PRECISE): P's
            // fp16 residual as a second product (the first queries of a causal
            // launch average a handful of keys; see attn_f16_kernel)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int sp = 0; sp < 2; ++sp) {
                    half8 plo;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][8 * sp + i], a.c, -m_use));
                        plo[i] = static_cast<_Float16>(e - static_cast<float>(static_cast<_Float16>(e)));
                    }
                    o[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, plo, o[2], 0, 0, 0);
                    const int G = t * 4 + sp * 2 + g;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int d = 32 * u + l32;
#pragma unroll
                        for (int pl = 0; pl < NP; ++pl) {
                            const half8 vf = *reinterpret_cast<const half8*>(&Vs[st][pl][(G * kVG + d) * 8]);
                            o[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, plo, o[u], 0, 0, 0);
                        }
                    }
                }
            }
        }

        store_tile(st ^ 1);
        __syncthreads();
    }

    const float lt = o[2][0];
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    constexpr int kWaveBytes = 32 * 64 * static_cast<int>(sizeof(TO));
    if constexpr (VEC && static_cast<int>(sizeof(Ks)) >= (kThreads / 64) * kWaveBytes) {
        if (a.ostage) {  // through LDS (the K stages, free after every wave's last tile)
            __syncthreads();
            const int nrows = qwave >= a.Tq ? 0 : static_cast<int>(min(a.Tq - qwave, 32u));
            TO* Ob = static_cast<TO*>(a.o) + b * a.so + static_cast<uint64_t>(qwave) * a.ldo + static_cast<uint64_t>(h) * a.hd;
            store_o_rows<TO>(o, inv, reinterpret_cast<char*>(&Ks[0][0][0]) + wave * kWaveBytes, Ob, nrows, hd, a.ldo, lane);
            return;
        }
    }
    if (qi >= a.Tq) return;
    TO* Op = static_cast<TO*>(a.o) + b * a.so + static_cast<uint64_t>(qi) * a.ldo + static_cast<uint64_t>(h) * a.hd;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int run = 0; run < 4; ++run) {
            const int d0 = 32 * u + 8 * run + 4 * g;
            if (VEC && d0 + 4 <= hd) {
                if constexpr (sizeof(TO) == 4) {
                    *reinterpret_cast<floatx4*>(Op + d0) =
                        floatx4{o[u][4 * run] * inv, o[u][4 * run + 1] * inv, o[u][4 * run + 2] * inv, o[u][4 * run + 3] * inv};
                } else {
                    *reinterpret_cast<half4*>(Op + d0) = half4_of(o[u][4 * run] * inv, o[u][4 * run + 1] * inv,
                                                                  o[u][4 * run + 2] * inv, o[u][4 * run + 3] * inv);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d0 + e < hd) Op[d0 + e] = static_cast<TO>(o[u][4 * run + e] * inv);
            }
        }
}


// ---- fp16 inputs: software-pipelined kernel --------------------------------
//
// Same math as attn_kernel, arranged so that matrix and vector work overlap
// inside each wave (a wave issues in order, so an MFMA only hides VALU work
// placed between MFMAs; waves sharing a SIMD do not overlap them): iteration
// j issues the S MFMAs of tile j+1 between the exp2 / fp16 packing / row sum
// of tile j, then the PV MFMAs of tile j between the scale of tile j+1. The
// lazy-rescale test needs no row max per tile: it runs on the tile's row sums
// after the exponentials (a sum over 2^8 is rare and sends the wave through a
// rescale that recomputes the tile's P). Every LDS fragment of an iteration is
// read up front.
//
// K and V tiles travel from memory straight into LDS (buffer loads with the
// LDS-DMA bit: no registers, no conversion, no LDS store instructions), as
// row-major [64 keys][64 d] fp16 with the eight 16-byte chunks of key row k
// stored at slot chunk ^ f(k) (a bank-conflict-free XOR swizzle for the
// fragment reads below). K fragments are plain 16-byte reads; V fragments come
// from ds_read_b64_tr_b16, whose 16-lane transpose turns four 8-byte row
// pieces into four consecutive keys at one d per lane -- exactly the key order
// of P in registers. K runs one tile ahead of V (K tiles j+1, j+2; V tiles j,
// j+1), so one barrier per tile keeps both double buffers race-free. The
// workgroup has NW waves of 32 queries; blocks are mapped so that the
// workgroups of one (batch, head) share an XCD (and its L2).
// RESID: which tiles add P's fp16 residual as a second PV product, at compile
// time (a runtime test of the flag inside the loop cost non-causal launches
// 2.4%): kResidNone; kResidDiagonal, a causal launch's diagonal tiles;
// kResidAll, every tile (MI_ATTN_PREC_SPLIT).
constexpr int kResidNone = 0, kResidDiagonal = 1, kResidAll = 2;
// BURST: the burst-ordered loop (below) built for three waves per SIMD
// (168 registers): a third workgroup per CU for grids of more than two per CU.
template <typename TO, int NW, int RESID, int BURST = 0>
__global__ __launch_bounds__(64 * NW, BURST ? 3 : 1) void attn_f16_kernel(AttnArgs a, uint32_t qtiles) {
    static_assert(!BURST || (RESID == kResidNone && NW == 4), "burst build: 4 waves, one PV product per tile");
    constexpr int BQ = 32 * NW;
    constexpr int DMA_IT = 8 / NW;  // 1 KB (8-row) DMA pieces per wave per tile, for K and for V
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2][kBKV * 64];
    __shared__ __attribute__((aligned(16))) _Float16 Vs[2][kBKV * 64];

    // block -> query block (and key range of a piece)
    unsigned blk;
    uint32_t piece = 0;
    bool split = false;
    if (a.pieces > 1 && blockIdx.x >= a.nfull) {
        const unsigned j = xcd_swizzle(blockIdx.x - a.nfull, gridDim.x - a.nfull);
        blk = a.nfull + j / a.pieces;
        piece = j % a.pieces;
        split = true;
    } else {
        blk = xcd_swizzle(blockIdx.x, a.pieces > 1 ? a.nfull : gridDim.x);
    }
    const uint32_t qt = blk % qtiles, bh = blk / qtiles;
    const uint32_t h = bh % a.heads, b = bh / a.heads;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, g = lane >> 5;
    const uint32_t qcta = qt * BQ, qwave = qcta + wave * 32, qi = qwave + l32;
    const int hd = static_cast<int>(a.hd);

    uint32_t L = a.Tk;
    if (a.kv_len) {
        int32_t l = a.kv_len[b];
        L = l < 0 ? 0u : (static_cast<uint32_t>(l) < a.Tk ? static_cast<uint32_t>(l) : a.Tk);
    }
    uint32_t kend = L;
    if (a.causal) kend = min(kend, qcta + BQ);
    uint32_t kfull = L / kBKV * kBKV;
    if (a.causal) kfull = min(kfull, (qwave + 1) / kBKV * kBKV);
    const uint32_t ntiles_all = (kend + kBKV - 1) / kBKV;
    // key tiles [t0, ntiles) of this workgroup (a piece: its share, in piece order)
    const uint32_t t0 = split ? ntiles_all * piece / a.pieces : 0u;
    const uint32_t ntiles = split ? ntiles_all * (piece + 1) / a.pieces : ntiles_all;

    const _Float16* Qp = static_cast<const _Float16*>(a.q) + b * a.sq + static_cast<uint64_t>(h) * a.hd;
    const _Float16* Kp = static_cast<const _Float16*>(a.k) + b * a.sk + static_cast<uint64_t>(h) * a.hd;
    const _Float16* Vp = static_cast<const _Float16*>(a.v) + b * a.sv + static_cast<uint64_t>(h) * a.hd;

    // Q rows of this wave go through LDS like the K tiles (4 DMA pieces of 8
    // rows: 128-byte row segments per instruction instead of 32 rows x 32 bytes)
    __shared__ __attribute__((aligned(16))) _Float16 Qs[BQ * 64];
    half8 qf[4];

    // Chunk slots: K row k keeps chunk c at slot c ^ ((k / 2) % 8), V row k at
    // c ^ 4 ((k / 2) % 2) (conflict-free for the K reads and the transposing V
    // reads). DMA piece p of a tile is key rows 8p .. 8p+7; lane l of the wave
    // writes slot l % 8 of row 8p + l / 8, so it fetches that slot's chunk.
    // Chunks at d >= hd and rows at or past L read as zeros.
    uint32_t k_dma[DMA_IT], v_dma[DMA_IT];
#pragma unroll
    for (int ii = 0; ii < DMA_IT; ++ii) {
        const uint32_t row = 8 * (wave * DMA_IT + ii) + (lane >> 3), slot = lane & 7;
        const uint32_t ck = slot ^ ((row >> 1) & 7), cv = slot ^ (((row >> 1) & 1) << 2);
        k_dma[ii] = static_cast<int>(ck * 8) < hd ? (row * static_cast<uint32_t>(a.ldk) + ck * 8) * 2u : kOob;
        v_dma[ii] = static_cast<int>(cv * 8) < hd ? (row * static_cast<uint32_t>(a.ldv) + cv * 8) * 2u : kOob;
    }
    auto dma_k = [&](uint32_t kv0, int st) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>(Kp + static_cast<uint64_t>(kv0) * a.ldk), 0,
            static_cast<int>(tile_bytes(kv0, L, a.ldk, a.hd, 2)), 0x00020000);
#pragma unroll
        for (int ii = 0; ii < DMA_IT; ++ii)
            lds_dma16(r, &Ks[st][(wave * DMA_IT + ii) * 512], k_dma[ii]);
    };
    auto dma_v = [&](uint32_t kv0, int st) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>(Vp + static_cast<uint64_t>(kv0) * a.ldv), 0,
            static_cast<int>(tile_bytes(kv0, L, a.ldv, a.hd, 2)), 0x00020000);
#pragma unroll
        for (int ii = 0; ii < DMA_IT; ++ii)
            lds_dma16(r, &Vs[st][(wave * DMA_IT + ii) * 512], v_dma[ii]);
    };
    // The DMA writes land asynchronously: wait for this wave's before the
    // barrier that hands the tile to the other waves.
    auto dma_wait = [] { wait_vmcnt0(); };

    half8 kf[2][4], vf[2][2][2];
    auto read_k = [&](int st) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int row = 32 * t + l32;
#pragma unroll
            for (int s = 0; s < 4; ++s)
                kf[t][s] = *reinterpret_cast<const half8*>(&Ks[st][row * 64 + (((2 * s + g) ^ ((row >> 1) & 7)) * 8)]);
        }
    };
    // V^T fragment (PV step t, sp; d block u): lane l = 16G + i needs d = 32u +
    // l%32 and keys 32t + 16sp + 8rd + 4(l/32) + 0..3 for rd = 0, 1. Lane i of
    // the 16-lane group supplies the 8-byte piece of key (base + i/4) at d =
    // 32u + 16(G%2) + 4(i%4); the transpose hands it keys base..base+3 at d.
    const int v_key = lane >> 2 & 3, v_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto read_v = [&](int st) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int sp = 0; sp < 2; ++sp)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    half4 hv[2];
#pragma unroll
                    for (int rd = 0; rd < 2; ++rd) {
                        const int key = 32 * t + 16 * sp + 8 * rd + 4 * g + v_key;
                        const int d = 32 * u + v_d;
                        const int off = key * 64 + (((d >> 3) ^ (((key >> 1) & 1) << 2)) * 8) + (d & 7);
                        hv[rd] = lds_read_tr16(&Vs[st][off]);
                    }
                    vf[t][sp][u] = half8{hv[0][0], hv[0][1], hv[0][2], hv[0][3], hv[1][0], hv[1][1], hv[1][2], hv[1][3]};
                }
    };
    // S^T = K Q^T: rows (keys) kv0 + 32t + 8(r/4) + 4g + r%4, column = query qi
    auto qk = [&](floatx16 (&sc)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[t][r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s) sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][s], qf[s], sc[t], 0, 0, 0);
        }
    };
    auto mask = [&](floatx16 (&sc)[2], uint32_t kv0) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t key = kv0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
                if (key >= L || (a.causal && key > qi)) sc[t][r] = -INFINITY;
            }
    };
    auto lane_max = [&](const floatx16 (&sc)[2]) {
        float m0 = fmaxf(sc[0][0], sc[0][1]), m1 = fmaxf(sc[1][0], sc[1][1]);
#pragma unroll
        for (int r = 2; r < 16; r += 2) {  // v_max3_f32 chains
            m0 = fmaxf(fmaxf(m0, sc[0][r]), sc[0][r + 1]);
            m1 = fmaxf(fmaxf(m1, sc[1][r]), sc[1][r + 1]);
        }
        const float mx = fmaxf(m0, m1);
        // the partner lane (lane ^ 32) holds the query's other 32 keys. (Not
        // v_permlane32_swap with mx as both operands: the compiler then takes
        // the two results for equal and keeps this half's max only.)
        return fmaxf(mx, __shfl_xor(mx, 32));
    };
    // exp2 + fp16 pack of key block t (keys 32t .. 32t + 31 of the tile)
    auto exp_half = [&](const floatx16 (&sc)[2], half8 (&pf)[2][2], int t) {
#pragma unroll
        for (int sp = 0; sp < 2; ++sp)
#pragma unroll
            for (int i = 0; i < 8; ++i) pf[t][sp][i] = static_cast<_Float16>(__builtin_amdgcn_exp2f(sc[t][8 * sp + i]));
    };
    auto exp_pack = [&](const floatx16 (&sc)[2], half8 (&pf)[2][2]) {
        exp_half(sc, pf, 0);
        exp_half(sc, pf, 1);
    };

    floatx16 o[2];  // O^T for d in [0, 32), [32, 64)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[u][r] = 0.0f;
    // Row sum of P over this lane's 32 keys of every tile (the partner lane,
    // lane ^ 32, holds the query's other 32): the fp16 P values the PV product
    // uses, summed in fp32 two at a time by v_dot2_f32_f16 (p0 * 1 + p1 * 1),
    // on the VALU instead of an all-ones MFMA operand.
    float lsum = 0.0f, m = 0.0f;
    const half2 one2 = {1, 1};
    auto tile_sum = [&](const half8 (&pf)[2][2]) {
        float ts = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int sp = 0; sp < 2; ++sp)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ts = __builtin_amdgcn_fdot2(half2{pf[t][sp][2 * i], pf[t][sp][2 * i + 1]}, one2, ts, false);
        return ts;
    };
    // Adds tile j's row sum (ts, from its fp16 P in pf, computed from the
    // scaled scores sc) after the lazy-rescale test: when some lane's sum
    // exceeds 2^8 (rare), the running max rises by the tile's excess over it
    // (the same amount in both lanes of a query), O and l are rescaled and
    // the tile's P are recomputed.
    auto settle = [&](floatx16 (&sc)[2], half8 (&pf)[2][2], float ts) {
        if (__any(ts > kLazySum)) {
            const float d = fmaxf(lane_max(sc), 0.0f);
            const float alpha = __builtin_amdgcn_exp2f(-d);
            m += d;
            lsum *= alpha;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[u][r] *= alpha;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[t][r] -= d;
            exp_pack(sc, pf);
            ts = tile_sum(pf);
        }
        lsum += ts;
    };
    auto pv = [&](const half8 (&pf)[2][2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int sp = 0; sp < 2; ++sp)
#pragma unroll
                for (int u = 0; u < 2; ++u) o[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[t][sp][u], pf[t][sp], o[u], 0, 0, 0);
    };
    // Causal diagonal tiles: the rows of the first queries average a handful
    // of keys, so their |O| is several times the output's RMS and P's fp16
    // rounding (2^-11 of each weight) would reach the 2e-3 x RMS bar. On those
    // tiles P also enters as the fp16 residual exp2(s) - fp16(exp2(s)): O gets
    // V P_lo as a second product and l the residuals' sum, which leaves P's
    // error at ~2^-22. Other tiles (and non-causal launches) keep one product.
    auto pv_residual = [&](const floatx16 (&sc)[2], const half8 (&pf)[2][2]) {
        half8 plo[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int sp = 0; sp < 2; ++sp)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    plo[t][sp][i] = static_cast<_Float16>(__builtin_amdgcn_exp2f(sc[t][8 * sp + i]) -
                                                          static_cast<float>(pf[t][sp][i]));
        lsum += tile_sum(plo);
        pv(plo);
    };

    if (t0 < ntiles) {
        // prologue: K tiles t0, t0+1 and V tile t0 in LDS; S of tile t0; the
        // running max starts at that tile's max (every query has a valid key in
        // it: key 0 < L and key 0 <= qi under the causal mask for t0 = 0, and
        // key-split plans have no mask)
        {
            const uint32_t nq = qwave < a.Tq ? min(a.Tq - qwave, 32u) : 0u;
            const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<_Float16*>(Qp + static_cast<uint64_t>(qwave) * a.ldq), 0,
                nq ? static_cast<int>(((nq - 1) * a.ldq + a.hd) * 2) : 0, 0x00020000);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t row = 8 * p + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
                lds_dma16(rq, &Qs[wave * 2048 + p * 512],
                          static_cast<int>(c * 8) < hd ? (row * static_cast<uint32_t>(a.ldq) + c * 8) * 2u : kOob);
            }
        }
        dma_k(t0 * kBKV, t0 & 1);
        dma_v(t0 * kBKV, t0 & 1);
        if (t0 + 1 < ntiles) dma_k((t0 + 1) * kBKV, (t0 + 1) & 1);
        dma_wait();
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; ++s)
            qf[s] = *reinterpret_cast<const half8*>(&Qs[wave * 2048 + l32 * 64 + (((2 * s + g) ^ ((l32 >> 1) & 7)) * 8)]);
        read_k(t0 & 1);
        floatx16 s0[2];
        qk(s0);
        if (t0 * kBKV >= kfull) mask(s0, t0 * kBKV);
        const float mx0 = lane_max(s0);
        m = mx0 == -INFINITY ? 0.0f : mx0 * a.c;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) s0[t][r] = __builtin_fmaf(s0[t][r], a.c, -m);
        // P of the tile's first 32 keys; each iteration computes the second
        // half in phase A and the next tile's first half in phase B, which
        // splits the exp2 work between the two MFMA phases
        half8 pf[2][2];
        exp_half(s0, pf, 0);
        if constexpr (BURST != 0) {  // the burst loop takes tile t0's whole P
            exp_half(s0, pf, 1);
            settle(s0, pf, tile_sum(pf));
        }
        __syncthreads();  // every wave has read K tile t0 before it is overwritten

        // One pipelined iteration; boundary tiles (key padding, Tk end, causal
        // diagonal) take the masked instantiation so that neither body branches
        // between its two phases.
        auto step = [&](uint32_t j, auto masked) {
            constexpr bool kMasked = decltype(masked)::value;
            const uint32_t kv1 = (j + 1) * kBKV;
            const bool more = j + 2 < ntiles;
            read_k((j + 1) & 1);
            read_v(j & 1);
            __builtin_amdgcn_sched_barrier(0);
            // into the stages read in the previous iteration (free after its barrier)
            if (more) dma_k(kv1 + kBKV, j & 1);
            dma_v(kv1, (j + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);

            // phase A: S of tile j+1 (8 MFMA) || exp2 + fp16 pack of tile j's
            // second half, row sum of tile j
            floatx16 s1[2];
            qk(s1);
            exp_half(s0, pf, 1);
            const float ts = tile_sum(pf);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            settle(s0, pf, ts);
            if constexpr (RESID == kResidAll) {
                pv_residual(s0, pf);
            } else if constexpr (RESID == kResidDiagonal) {
                if (j * kBKV >= kfull) pv_residual(s0, pf);
            }

            // phase B: PV of tile j (8 MFMA) || mask + scale of tile j+1, exp2 +
            // fp16 pack of its first half
            pv(pf);
            if constexpr (kMasked) mask(s1, kv1);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) s1[t][r] = __builtin_fmaf(s1[t][r], a.c, -m);
            half8 pn[2][2];
            exp_half(s1, pn, 0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kMasked ? 15 : 7, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 2; ++t) s0[t] = s1[t];
#pragma unroll
            for (int sp = 0; sp < 2; ++sp) pf[0][sp] = pn[0][sp];
            dma_wait();
            __syncthreads();
        };
        // BURST: iteration j issues its 16 MFMAs back to back (S of tile j+1,
        // then PV of tile j, whose P the previous iteration completed), then
        // the whole softmax of tile j+1 on the VALU, so one wave's MFMAs can
        // run under another wave's vector work; the loop keeps fewer values
        // live (168 registers: three waves per SIMD). Same operations in the
        // same order per tile as the interleaved loop: the same bits.
        auto step_burst = [&](uint32_t j, auto masked) {
            constexpr bool kMasked = decltype(masked)::value;
            const uint32_t kv1 = (j + 1) * kBKV;
            const bool more = j + 2 < ntiles;
            read_k((j + 1) & 1);
            read_v(j & 1);
            __builtin_amdgcn_sched_barrier(0);
            if (more) dma_k(kv1 + kBKV, j & 1);
            dma_v(kv1, (j + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            floatx16 s1[2];
            qk(s1);
            pv(pf);  // (the burst build has one PV product per tile: RESID == kResidNone)
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kMasked) mask(s1, kv1);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) s1[t][r] = __builtin_fmaf(s1[t][r], a.c, -m);
            exp_pack(s1, pf);
            settle(s1, pf, tile_sum(pf));
#pragma unroll
            for (int t = 0; t < 2; ++t) s0[t] = s1[t];
            dma_wait();
            __syncthreads();
        };
        for (uint32_t j = t0; j + 1 < ntiles; ++j) {
            if constexpr (BURST != 0) {
                if ((j + 1) * kBKV >= kfull) step_burst(j, std::true_type{});
                else step_burst(j, std::false_type{});
            } else {
                if ((j + 1) * kBKV >= kfull) step(j, std::true_type{});
                else step(j, std::false_type{});
            }
        }
        // last tile
        read_v((ntiles - 1) & 1);
        if constexpr (BURST == 0) {
            exp_half(s0, pf, 1);
            settle(s0, pf, tile_sum(pf));
        }
        if constexpr (RESID == kResidAll) {
            pv_residual(s0, pf);
        } else if constexpr (RESID == kResidDiagonal) {
            if ((ntiles - 1) * kBKV >= kfull) pv_residual(s0, pf);
        }
        pv(pf);
    }

    // the query's row sum: this lane's 32 keys of every tile plus the partner
    // lane's (one rounding, the same in both lanes: fp32 addition commutes)
    const float lt = lsum + __shfl_xor(lsum, 32);
    if (split) {
        // a piece: the unnormalised O rows (fp32, through the K / V stages like the
        // output), the running max and the row sum of each query, for attn_merge_kernel
        __syncthreads();
        constexpr int kWB = 32 * 64 * 4;
        constexpr int kStage = static_cast<int>(sizeof(Ks));
        char* st = wave * kWB < kStage ? reinterpret_cast<char*>(&Ks[0][0]) + wave * kWB
                                       : reinterpret_cast<char*>(&Vs[0][0]) + (wave * kWB - kStage);
        float* P = a.part + static_cast<uint64_t>((blk - a.nfull) * a.pieces + piece) * kPartFloats;
        store_o_rows<float>(o, 1.0f, st, P + wave * 32 * 64, 32, 64, 64, lane);
        if (lane < 32) {
            P[kBQ * 64 + wave * 32 + lane] = m;
            P[kBQ * 64 + kBQ + wave * 32 + lane] = lt;
        }
        return;
    }
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (a.ostage) {
        // every wave is done with the K / V stages: each takes 32 * 64 * sizeof(TO)
        // bytes of them (waves 0, 1 of Ks and 2, 3 of Vs for fp32 output)
        __syncthreads();
        constexpr int kWaveBytes = 32 * 64 * static_cast<int>(sizeof(TO));
        constexpr int kStage = static_cast<int>(sizeof(Ks));
        char* st = wave * kWaveBytes < kStage ? reinterpret_cast<char*>(&Ks[0][0]) + wave * kWaveBytes
                                              : reinterpret_cast<char*>(&Vs[0][0]) + (wave * kWaveBytes - kStage);
        const int nrows = qwave >= a.Tq ? 0 : static_cast<int>(min(a.Tq - qwave, 32u));
        TO* Ob = static_cast<TO*>(a.o) + b * a.so + static_cast<uint64_t>(qwave) * a.ldo + static_cast<uint64_t>(h) * a.hd;
        store_o_rows<TO>(o, inv, st, Ob, nrows, hd, a.ldo, lane);
        return;
    }
    if (qi >= a.Tq) return;
    TO* Op = static_cast<TO*>(a.o) + b * a.so + static_cast<uint64_t>(qi) * a.ldo + static_cast<uint64_t>(h) * a.hd;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int run = 0; run < 4; ++run) {
            const int d0 = 32 * u + 8 * run + 4 * g;
            if (d0 >= hd) continue;
            if constexpr (sizeof(TO) == 4) {
                *reinterpret_cast<floatx4*>(Op + d0) =
                    floatx4{o[u][4 * run] * inv, o[u][4 * run + 1] * inv, o[u][4 * run + 2] * inv, o[u][4 * run + 3] * inv};
            } else {
                *reinterpret_cast<half4*>(Op + d0) = half4_of(o[u][4 * run] * inv, o[u][4 * run + 1] * inv,
                                                              o[u][4 * run + 2] * inv, o[u][4 * run + 3] * inv);
            }
        }
}


// Adds the key-split pieces of a query block (mi_fused_attention_ws): O = sum_i 2^(m_i - M) O_i /
// sum_i 2^(m_i - M) l_i with M = max_i m_i, pieces in order (a call repeats bit for bit). Four
// workgroups per split query block; thread t of a workgroup takes query t / 8 of its 32 and the 8
// columns 8 (t % 8) of the head, so a warp-wide access covers whole 256-byte partial rows and whole
// output rows (one 16-byte store per thread for fp16 output when rows are 16-byte aligned).
// NP > 0: exactly NP pieces (the 2- and 4-piece plans), unrolled so that all loads issue together.
template <typename TO, int NP = 0>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a, uint32_t qtiles) {
    const uint32_t rb = blockIdx.x / 4, blk = a.nfull + rb;
    const uint32_t qt = blk % qtiles, bh = blk / qtiles;
    const uint32_t h = bh % a.heads, b = bh / a.heads;
    const int q = static_cast<int>(blockIdx.x % 4) * 32 + static_cast<int>(threadIdx.x >> 3);
    const int c = static_cast<int>(threadIdx.x & 7) * 8;
    const uint32_t qi = qt * kBQ + q;
    const int hd = static_cast<int>(a.hd);
    if (qi >= a.Tq || c >= hd) return;
    const float* P = a.part + static_cast<uint64_t>(rb) * a.pieces * kPartFloats;
    float M = -INFINITY;
    float l = 0.0f;
    floatx4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (NP > 0) {
        // NP pieces exactly: every load first (one memory round trip), then
        // the same operations in the same order as the loops of any count
        float mi[NP], li[NP];
        floatx4 r0[NP], r1[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const float* Pi = P + i * kPartFloats;
            mi[i] = Pi[kBQ * 64 + q];
            li[i] = Pi[kBQ * 64 + kBQ + q];
            r0[i] = reinterpret_cast<const floatx4*>(Pi + q * 64 + c)[0];
            r1[i] = reinterpret_cast<const floatx4*>(Pi + q * 64 + c)[1];
        }
#pragma unroll
        for (int i = 0; i < NP; ++i) M = fmaxf(M, mi[i]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const float sc = mi[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mi[i] - M);
            l += sc * li[i];
            acc0 += sc * r0[i];
            acc1 += sc * r1[i];
        }
    } else {
        for (uint32_t i = 0; i < a.pieces; ++i) M = fmaxf(M, P[i * kPartFloats + kBQ * 64 + q]);
        for (uint32_t i = 0; i < a.pieces; ++i) {
            const float* Pi = P + i * kPartFloats;
            const float mi = Pi[kBQ * 64 + q];
            const float sc = mi == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mi - M);
            l += sc * Pi[kBQ * 64 + kBQ + q];
            const floatx4* row = reinterpret_cast<const floatx4*>(Pi + q * 64 + c);
            acc0 += sc * row[0];
            acc1 += sc * row[1];
        }
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    acc0 *= inv;
    acc1 *= inv;
    TO* Op = static_cast<TO*>(a.o) + b * a.so + static_cast<uint64_t>(qi) * a.ldo + static_cast<uint64_t>(h) * a.hd + c;
    if constexpr (sizeof(TO) == 2) {
        const half4 v0 = half4_of(acc0[0], acc0[1], acc0[2], acc0[3]), v1 = half4_of(acc1[0], acc1[1], acc1[2], acc1[3]);
        const half8 v = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        if (a.ostage) {
            *reinterpret_cast<half8*>(Op) = v;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) Op[e] = v[e];
        }
    } else {
        if (a.ostage) {
            reinterpret_cast<floatx4*>(Op)[0] = acc0;
            reinterpret_cast<floatx4*>(Op)[1] = acc1;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                Op[e] = acc0[e];
                Op[4 + e] = acc1[e];
            }
        }
    }
}

// Waves per workgroup of the fp16 kernel: 4 (128 queries), or 2 when one
// 64-query block holds every query. Measured on MI355X, 4-wave workgroups are
// as fast or faster on every grid size, small ones included (160-256 blocks of
// 128 queries: 23% faster than twice as many 2-wave workgroups).
// mi_tuning_set("attn_nw", "2" | "4") pins one (tuning sweeps).
int f16_waves(const AttnArgs& a, uint32_t /*batch*/) {
    const int forced = tuning().attn_nw.load(std::memory_order_relaxed);
    return forced == 2 || forced == 4 ? forced : a.Tq <= 64 ? 2 : 4;
}

// Compute units of the current device (queried once per device).
uint32_t cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return static_cast<uint32_t>(n);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return static_cast<uint32_t>(n);
}

// Key split of the grid's last partial round (mi_fused_attention_ws): with W
// 4-wave query blocks and S = 2 per CU resident at once, W = r S + rest runs
// r full rounds and then `rest` blocks alone on part of the GPU. Those rest
// blocks instead run as `pieces` workgroups each over consecutive key-tile
// ranges, one piece per CU (pieces = CUs / rest, >= 8 tiles each, at most 8),
// so the last round fills the GPU for a fraction of a round; attn_merge_kernel
// adds the pieces. Measured on MI355X (graph-timed, interleaved): 2 x 10 heads
// x 4096 (128 rest blocks) unsplit 119.4 us, 2 pieces 104.7, 4 pieces 106.6,
// 8 pieces 110.3; 2 x 9 heads (64 rest) unsplit 116.4, 2 / 4 / 8 pieces 119.5 /
// 110.0 / 113.4; 2 x 12 heads (256 rest: no plan, CUs / rest = 1) 131 unsplit
// against 141 in 2 pieces.
// Only unmasked, non-causal fp16 launches split. mi_tuning_set("attn_split",
// "<rest>:<pieces>") forces a plan (tests; "0" turns the split off).
struct SplitPlan {
    uint32_t nfull = 0, pieces = 1, rest = 0;
};

SplitPlan plan_split(const AttnArgs& a, uint32_t batch) {
    SplitPlan p;
    if (a.causal || a.kv_len || a.Tk == 0 || f16_waves(a, batch) != 4) return p;
    const uint64_t W = static_cast<uint64_t>(ceil_div(a.Tq, kBQ)) * a.heads * batch;
    const uint32_t nt = ceil_div(a.Tk, kBKV);
    uint64_t rest = 0, pieces = 1;
    const int forced_rest = tuning().attn_split_rest.load(std::memory_order_relaxed);
    if (forced_rest >= 0) {
        rest = static_cast<uint64_t>(forced_rest);
        pieces = static_cast<uint64_t>(tuning().attn_split_pieces.load(std::memory_order_relaxed));
        rest = rest < W ? rest : W;
        if (pieces > nt) pieces = nt;
    } else {
        const uint64_t S = 2ull * cu_count();
        if (W <= S || W % S == 0) return p;
        rest = W % S;
        pieces = cu_count() / rest;
        if (pieces > nt / 8) pieces = nt / 8;
        if (pieces > 8) pieces = 8;
    }
    if (rest == 0 || pieces < 2) return p;
    p.rest = static_cast<uint32_t>(rest);
    p.pieces = static_cast<uint32_t>(pieces);
    p.nfull = static_cast<uint32_t>(W - rest);
    return p;
}

uint64_t split_bytes(const SplitPlan& p) { return static_cast<uint64_t>(p.rest) * p.pieces * kPartFloats * 4; }

// The burst build (three 4-wave workgroups per CU) for fp16-precision,
// non-causal launches whose grid holds more than two workgroups per CU; the
// interleaved build (two per CU) otherwise. Measured on MI355X (graph-timed,
// interleaved runs, us, interleaved / burst): 2 x 10 x 4096^2 with its key
// split 102.5 / 100.4, cross 2 x 10 x 4096 x 77 9.59 / 7.62; with at most two
// workgroups per CU the burst loop has no second wave to overlap with
// (2 x 20 x 1024^2 21.1 / 22.4). mi_tuning_set("attn_simd_waves", "2" | "3")
// pins one (fp16-precision non-causal launches only).
bool use_burst(const AttnArgs& a, uint64_t grid) {
    if (a.precise || a.causal) return false;
    const int forced = tuning().attn_simd_waves.load(std::memory_order_relaxed);
    if (forced == 2 || forced == 3) return forced == 3;
    return grid > 2ull * cu_count();
}

template <typename TO>
void launch_f16(const AttnArgs& a, uint32_t batch, hipStream_t s) {
    const uint32_t q4 = ceil_div(a.Tq, 128u), q2 = ceil_div(a.Tq, 64u);
    const uint64_t groups = static_cast<uint64_t>(a.heads) * batch;
    if (a.pieces > 1) {  // a key-split plan (4-wave workgroups)
        const uint32_t rest = static_cast<uint32_t>(q4 * groups - a.nfull);
        const unsigned grid = a.nfull + rest * a.pieces;
        if (a.precise) attn_f16_kernel<TO, 4, kResidAll><<<grid, 256, 0, s>>>(a, q4);
        else if (use_burst(a, grid)) attn_f16_kernel<TO, 4, kResidNone, 1><<<grid, 256, 0, s>>>(a, q4);
        else attn_f16_kernel<TO, 4, kResidNone><<<grid, 256, 0, s>>>(a, q4);
        if (a.pieces == 2) attn_merge_kernel<TO, 2><<<rest * 4, 256, 0, s>>>(a, q4);
        else if (a.pieces == 4) attn_merge_kernel<TO, 4><<<rest * 4, 256, 0, s>>>(a, q4);
        else attn_merge_kernel<TO><<<rest * 4, 256, 0, s>>>(a, q4);
        return;
    }
    const bool nw4 = f16_waves(a, batch) == 4;
    const unsigned g4 = static_cast<unsigned>(q4 * groups), g2 = static_cast<unsigned>(q2 * groups);
    if (a.precise) {
        if (nw4) attn_f16_kernel<TO, 4, kResidAll><<<g4, 256, 0, s>>>(a, q4);
        else attn_f16_kernel<TO, 2, kResidAll><<<g2, 128, 0, s>>>(a, q2);
    } else if (a.causal) {
        if (nw4) attn_f16_kernel<TO, 4, kResidDiagonal><<<g4, 256, 0, s>>>(a, q4);
        else attn_f16_kernel<TO, 2, kResidDiagonal><<<g2, 128, 0, s>>>(a, q2);
    } else {
        if (nw4 && use_burst(a, g4)) attn_f16_kernel<TO, 4, kResidNone, 1><<<g4, 256, 0, s>>>(a, q4);
        else if (nw4) attn_f16_kernel<TO, 4, kResidNone><<<g4, 256, 0, s>>>(a, q4);
        else attn_f16_kernel<TO, 2, kResidNone><<<g2, 128, 0, s>>>(a, q2);
    }
}

template <typename TI, typename TO>
void launch_typed(const AttnArgs& a, uint32_t batch, bool vec, hipStream_t s) {
    dim3 grid(ceil_div(a.Tq, kBQ), a.heads, batch);
    if (vec) attn_kernel<TI, TO, true><<<grid, kThreads, 0, s>>>(a);
    else attn_kernel<TI, TO, false><<<grid, kThreads, 0, s>>>(a);
}

// need: when set, only the workspace bytes a split plan would use are stored
// (no launch); ws / ws_bytes: the caller's workspace (mi_fused_attention_ws).
int run(const mi_attn_args& x, hipStream_t s, const char* fn, void* ws = nullptr, uint64_t ws_bytes = 0,
        uint64_t* need = nullptr) {
    if (!x.q || !x.k || !x.v || !x.out) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (x.in_dtype != MI_F32 && x.in_dtype != MI_F16) return fail(MI_ERR_INVALID_ARG, "%s: in_dtype %d", fn, x.in_dtype);
    if (x.out_dtype != MI_F32 && x.out_dtype != MI_F16) return fail(MI_ERR_INVALID_ARG, "%s: out_dtype %d", fn, x.out_dtype);
    if (x.batch == 0) return fail(MI_ERR_INVALID_ARG, "%s: batch 0", fn);
    if (x.precision != MI_ATTN_PREC_AUTO && x.precision != MI_ATTN_PREC_FP16 && x.precision != MI_ATTN_PREC_SPLIT)
        return fail(MI_ERR_INVALID_ARG, "%s: precision %d", fn, x.precision);
    if (!mi_fused_attn_supported(x.C, x.heads))
        return fail(MI_ERR_UNSUPPORTED, "%s: unsupported C=%u heads=%u (need heads | C and C/heads <= 64)", fn, x.C, x.heads);
    if (x.batch > 65535 || x.heads > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: batch/heads > 65535", fn);
    if (x.Tq == 0) return MI_OK;
    const uint64_t ldq = x.ldq ? x.ldq : x.C, ldk = x.ldk ? x.ldk : x.C, ldv = x.ldv ? x.ldv : x.C,
                   ldo = x.ldo ? x.ldo : x.C;
    if (ldq < x.C || ldk < x.C || ldv < x.C || ldo < x.C) return fail(MI_ERR_INVALID_ARG, "%s: token stride < C", fn);
    // a 64-row K/V tile must span under 2^30 bytes (32-bit buffer offsets)
    if (ldq * 64 * 4 >= (1ull << 30) || ldk * 64 * 4 >= (1ull << 30) || ldv * 64 * 4 >= (1ull << 30))
        return fail(MI_ERR_UNSUPPORTED, "%s: Q/K/V token stride too large", fn);
    const uint64_t sq = x.sq ? x.sq : x.Tq * ldq, sk = x.sk ? x.sk : x.Tk * ldk, sv = x.sv ? x.sv : x.Tk * ldv,
                   so = x.so ? x.so : x.Tq * ldo;
    const uint64_t ei = x.in_dtype == MI_F32 ? 4 : 2, eo = x.out_dtype == MI_F32 ? 4 : 2;
    const uint64_t obytes = ((x.batch - 1) * so + (x.Tq - 1) * ldo + x.C) * eo;
    const uint64_t qbytes = ((x.batch - 1) * sq + (x.Tq - 1) * ldq + x.C) * ei;
    const uint64_t kbytes = x.Tk ? ((x.batch - 1) * sk + (x.Tk - 1) * ldk + x.C) * ei : 0;
    const uint64_t vbytes = x.Tk ? ((x.batch - 1) * sv + (x.Tk - 1) * ldv + x.C) * ei : 0;
    if (overlaps(x.out, obytes, x.q, qbytes) || overlaps(x.out, obytes, x.k, kbytes) ||
        overlaps(x.out, obytes, x.v, vbytes))
        return fail(MI_ERR_ALIASING, "%s: out overlaps q, k or v", fn);
    if (!aligned(x.q, ei) || !aligned(x.k, ei) || !aligned(x.v, ei) || !aligned(x.out, eo))
        return fail(MI_ERR_ALIGNMENT, "%s: tensors must be aligned to their element size", fn);

    AttnArgs a;
    a.q = x.q; a.k = x.k; a.v = x.v; a.o = x.out;
    a.Tq = x.Tq; a.Tk = x.Tk; a.heads = x.heads; a.hd = x.C / x.heads;
    a.causal = x.causal ? 1 : 0;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
    a.sq = sq; a.sk = sk; a.sv = sv; a.so = so;
    a.kv_len = x.kv_len;
    const float scale = x.scale != 0.0f ? x.scale : 1.0f / sqrtf(static_cast<float>(a.hd));
    a.c = scale * 1.4426950408889634f;
    a.ostage = aligned(x.out, 16) && (ldo * eo) % 16 == 0 && (so * eo) % 16 == 0 && (a.hd * eo) % 16 == 0 &&
               tuning().attn_direct_store.load(std::memory_order_relaxed) == 0;
    a.precise = x.precision == MI_ATTN_PREC_SPLIT || (x.precision == MI_ATTN_PREC_AUTO && x.out_dtype == MI_F32);

    // 16-byte vector path: every 8-element chunk of every row is 16-byte aligned.
    const uintptr_t vin = 8 * ei, vout = 4 * eo;
    const bool vec = a.hd % 8 == 0 && aligned(x.q, 16) && aligned(x.k, 16) && aligned(x.v, 16) &&
                     aligned(x.out, vout) && (ldq * ei) % 16 == 0 && (ldk * ei) % 16 == 0 && (ldv * ei) % 16 == 0 &&
                     (sq * ei) % 16 == 0 && (sk * ei) % 16 == 0 && (sv * ei) % 16 == 0 && (ldo * eo) % vout == 0 &&
                     (so * eo) % vout == 0 && (a.hd * ei) % vin == 0;
    // fp16 inputs on the vector path: the pipelined kernel (one workgroup per
    // 64 or 128 queries of one (batch, head), 1-D grid)
    const bool fast = vec && x.in_dtype == MI_F16 &&
                      static_cast<uint64_t>(ceil_div(x.Tq, 64u)) * x.heads * x.batch < (1ull << 31);
    a.nfull = 0;
    a.pieces = 1;
    a.part = nullptr;
    if (fast && (need || ws)) {
        const SplitPlan p = plan_split(a, x.batch);
        const uint64_t bytes = p.pieces > 1 ? split_bytes(p) : 0;
        if (need) {
            *need = bytes;
            return MI_OK;
        }
        if (bytes && ws_bytes >= bytes) {
            if (!aligned(ws, 16)) return fail(MI_ERR_ALIGNMENT, "%s: workspace must be 16-byte aligned", fn);
            if (overlaps(ws, bytes, x.out, obytes) || overlaps(ws, bytes, x.q, qbytes) ||
                overlaps(ws, bytes, x.k, kbytes) || overlaps(ws, bytes, x.v, vbytes))
                return fail(MI_ERR_ALIASING, "%s: workspace overlaps q, k, v or out", fn);
            a.nfull = p.nfull;
            a.pieces = p.pieces;
            a.part = static_cast<float*>(ws);
        }
    } else if (need) {
        *need = 0;
        return MI_OK;
    }
    if (fast && x.out_dtype == MI_F16) launch_f16<_Float16>(a, x.batch, s);
    else if (fast) launch_f16<float>(a, x.batch, s);
    else if (x.in_dtype == MI_F16 && x.out_dtype == MI_F16) launch_typed<_Float16, _Float16>(a, x.batch, vec, s);
    else if (x.in_dtype == MI_F16) launch_typed<_Float16, float>(a, x.batch, vec, s);
    else if (x.out_dtype == MI_F16) launch_typed<float, _Float16>(a, x.batch, vec, s);
    else launch_typed<float, float>(a, x.batch, vec, s);
    return check_launch(fn);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_fused_attn_supported(uint32_t C, uint32_t heads) {
    if (!C || !heads || C % heads) return 0;
    uint32_t hd = C / heads;
    return hd > 0 && hd <= 64 ? 1 : 0;
}

extern "C" int mi_fused_attention(const float* q, const float* k, const float* v, float* out, uint32_t Tq,
                                  uint32_t Tk, uint32_t C, uint32_t heads, int causal, void* stream) {
    mi_attn_args x{};
    x.q = q; x.k = k; x.v = v; x.out = out;
    x.batch = 1; x.Tq = Tq; x.Tk = Tk; x.C = C; x.heads = heads; x.causal = causal;
    x.in_dtype = MI_F32; x.out_dtype = MI_F32;
    return run(x, static_cast<hipStream_t>(stream), "mi_fused_attention");
}

extern "C" int mi_fused_attention_ex(const mi_attn_args* args, void* stream) {
    if (!args) return fail(MI_ERR_INVALID_ARG, "mi_fused_attention_ex: null args");
    return run(*args, static_cast<hipStream_t>(stream), "mi_fused_attention_ex");
}

extern "C" uint64_t mi_fused_attention_ws_bytes(const mi_attn_args* args) {
    if (!args) return 0;
    uint64_t need = 0;
    return run(*args, nullptr, "mi_fused_attention_ws_bytes", nullptr, 0, &need) == MI_OK ? need : 0;
}

extern "C" int mi_fused_attention_ws(const mi_attn_args* args, void* workspace, uint64_t workspace_bytes,
                                     void* stream) {
    if (!args) return fail(MI_ERR_INVALID_ARG, "mi_fused_attention_ws: null args");
    return run(*args, static_cast<hipStream_t>(stream), "mi_fused_attention_ws", workspace, workspace_bytes);
}
