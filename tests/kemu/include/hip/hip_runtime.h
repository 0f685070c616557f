// Host stand-in for <hip/hip_runtime.h> used only by the kernel emulator
// (tests/kemu): HIP's device dialect and the gfx950 builtins the library's
// kernels call, mapped onto the fiber runtime of kemu.hpp. Every builtin is
// restated from its documented behaviour (AMD ISA / LLVM AMDGPU docs); an
// argument the kernels never use (DPP row masks, MFMA broadcast controls,
// strided buffers) is rejected instead of emulated.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <tuple>
#include <type_traits>

#include "../../kemu.hpp"

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ __attribute__((section("kemu_lds"))) static
#define __restrict__ __restrict

struct dim3 {
    uint32_t x, y, z;
    constexpr dim3(uint32_t x_ = 1, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
};

#define threadIdx (::kemu::thread_idx())
#define blockIdx (::kemu::g_block_idx)
#define blockDim (::kemu::g_block_dim)
#define gridDim (::kemu::g_grid_dim)
#define __syncthreads() ::kemu::syncthreads()

// ---- runtime API (host side of the library) --------------------------------------
typedef enum hipError_t { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2 } hipError_t;
typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;
typedef enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4
} hipMemcpyKind;
#define hipEventDisableTiming 0x2u
#define hipHostMallocDefault 0x0u

inline hipError_t hipGetLastError() { return hipSuccess; }
// File-scope __device__ arrays are host globals here: a symbol's device address
// is its host address, on the one emulated device 0.
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
// The emulated device reports an MI355X's 256 compute units.
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t attr, int) {
    *v = attr == hipDeviceAttributeMultiprocessorCount ? 256 : 0;
    return hipSuccess;
}
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
    *p = const_cast<void*>(sym);
    return hipSuccess;
}
// The emulator records no graphs: no stream is ever capturing.
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* st) {
    *st = hipStreamCaptureStatusNone;
    return hipSuccess;
}

inline const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "emulated HIP error"; }
// Asynchronous copies are deferred: they run at the event synchronisation that
// covers them, before the next kernel launch, or at kemu_sync(), so a source
// reused before its copy is known to be done is caught.
struct ihipEvent_t {
    uint64_t seq;
};
inline hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
    ::kemu::enqueue_copy(d, s, n);
    return hipSuccess;
}
inline hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
    *p = std::malloc(n ? n : 1);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipHostFree(void* p) {
    ::kemu::flush_copies(~0ull);
    std::free(p);
    return hipSuccess;
}
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
    *e = new ihipEvent_t{0};
    return hipSuccess;
}
inline hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
    e->seq = ::kemu::copy_seq();
    return hipSuccess;
}
inline hipError_t hipEventSynchronize(hipEvent_t e) {
    ::kemu::flush_copies(e->seq);
    return hipSuccess;
}
inline hipError_t hipEventDestroy(hipEvent_t e) {
    delete e;
    return hipSuccess;
}

// ---- device math / bit helpers ---------------------------------------------------
inline float __uint_as_float(uint32_t u) { return __builtin_bit_cast(float, u); }
inline uint32_t __float_as_uint(float f) { return __builtin_bit_cast(uint32_t, f); }
inline float __int_as_float(int u) { return __builtin_bit_cast(float, u); }
inline int __float_as_int(float f) { return __builtin_bit_cast(int, f); }
template <class T, class U>
inline typename std::common_type<T, U>::type min(T a, U b) {
    typedef typename std::common_type<T, U>::type R;
    return static_cast<R>(a) < static_cast<R>(b) ? static_cast<R>(a) : static_cast<R>(b);
}
template <class T, class U>
inline typename std::common_type<T, U>::type max(T a, U b) {
    typedef typename std::common_type<T, U>::type R;
    return static_cast<R>(a) < static_cast<R>(b) ? static_cast<R>(b) : static_cast<R>(a);
}
// fp32 atomics: work-items run one at a time, so a plain read-modify-write is atomic
inline float unsafeAtomicAdd(float* p, float v) {
    const float o = *p;
    *p = o + v;
    return o;
}
inline float atomicAdd(float* p, float v) { return unsafeAtomicAdd(p, v); }

namespace kemu {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef uint32_t u3v __attribute__((ext_vector_type(3)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

// ---- buffer resources ------------------------------------------------------------
// Raw buffer (stride 0): a dword at byte offset o (voffset + soffset) is read
// when o + 4 <= num_records, else reads as 0 / is not written. Cases whose
// outcome would depend on details the kernels must not rely on are errors:
// a dword straddling num_records, and a dword that is out of range only
// because of the scalar offset (some generations leave soffset out of the
// check).
struct Rsrc {
    unsigned char* base;
    uint32_t num;
};
inline Rsrc make_rsrc(const void* p, int stride, int num, int) {
    if (stride != 0) die("make_buffer_rsrc: strided buffers are not emulated");
    return Rsrc{static_cast<unsigned char*>(const_cast<void*>(p)), static_cast<uint32_t>(num)};
}
inline bool in_range(const Rsrc& r, uint32_t voff, uint32_t soff, uint32_t at, uint32_t size, const char* what) {
    const uint64_t o = static_cast<uint64_t>(voff) + soff + at;
    const uint64_t ov = static_cast<uint64_t>(voff) + at;
    const bool in = o + size <= r.num;
    if (!in && o < r.num) die("%s: access [%llu, +%u) straddles num_records %u", what, (unsigned long long)o, size, r.num);
    if (!in && ov + size <= r.num)
        die("%s: voffset %u in range, voffset + soffset %u out of range (num_records %u)", what, voff, soff, r.num);
    return in;
}
template <int N>
inline void buf_load(const Rsrc& r, uint32_t voff, uint32_t soff, uint32_t* out, const char* what) {
    int n_in = 0;
    for (int d = 0; d < N; ++d) {
        if (in_range(r, voff, soff, 4u * d, 4, what)) {
            std::memcpy(&out[d], r.base + static_cast<uint64_t>(voff) + soff + 4u * d, 4);
            ++n_in;
        } else {
            out[d] = 0;
        }
    }
    if (n_in != 0 && n_in != N) die("%s: %d of %d dwords in range (partial loads are not relied on)", what, n_in, N);
}
inline uint32_t buffer_load_b32(Rsrc r, uint32_t v, uint32_t s, int) {
    uint32_t x;
    buf_load<1>(r, v, s, &x, "raw_buffer_load_b32");
    return x;
}
inline u2v buffer_load_b64(Rsrc r, uint32_t v, uint32_t s, int) {
    uint32_t x[2];
    buf_load<2>(r, v, s, x, "raw_buffer_load_b64");
    return u2v{x[0], x[1]};
}
inline u4v buffer_load_b128(Rsrc r, uint32_t v, uint32_t s, int) {
    uint32_t x[4];
    buf_load<4>(r, v, s, x, "raw_buffer_load_b128");
    return u4v{x[0], x[1], x[2], x[3]};
}
inline uint16_t buffer_load_b16(Rsrc r, uint32_t v, uint32_t s, int) {
    uint16_t x = 0;
    if (in_range(r, v, s, 0, 2, "raw_buffer_load_b16")) std::memcpy(&x, r.base + static_cast<uint64_t>(v) + s, 2);
    return x;
}
inline void buffer_store_b32(uint32_t x, Rsrc r, uint32_t v, uint32_t s, int) {
    if (in_range(r, v, s, 0, 4, "raw_buffer_store_b32")) std::memcpy(r.base + static_cast<uint64_t>(v) + s, &x, 4);
}

// ---- VALU bit operations -----------------------------------------------------------
// v_perm_b32: byte i of the result is selected by byte i of sel from the eight
// bytes {a (high), b (low)}; 8..11 replicate a sign bit, 12 gives 0x00, 13+ 0xFF.
inline uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
    const uint64_t in = (static_cast<uint64_t>(a) << 32) | b;
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t s = (sel >> (8 * i)) & 0xffu;
        uint32_t byte;
        if (s < 8) byte = static_cast<uint32_t>(in >> (8 * s)) & 0xffu;
        else if (s < 12) byte = ((in >> (16 * (s - 8) + 15)) & 1u) ? 0xffu : 0u;
        else if (s == 12) byte = 0;
        else byte = 0xffu;
        r |= byte << (8 * i);
    }
    return r;
}
// v_alignbit_b32: low 32 bits of ({a, b} >> (s mod 32))
inline uint32_t alignbit(uint32_t a, uint32_t b, uint32_t s) {
    return static_cast<uint32_t>(((static_cast<uint64_t>(a) << 32) | b) >> (s & 31u));
}

// ---- cross-lane operations ---------------------------------------------------------
struct MfmaIn {
    h8 a, b;
    f16v c;
};
// v_mfma_f32_32x32x16_f16: D = C + A B with A 32x16, B 16x32. Lane l supplies
// A row l % 32 and B column l % 32, eight k each (k = 8 (l / 32) + 0..7; any
// k order is the same product as long as A and B share it); D / C: lane l,
// register r holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
inline void mfma_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void*) {
    float A[32][16], B[16][32], Cm[32][32];
    for (int l = 0; l < 64; ++l) {
        MfmaIn x;
        std::memcpy(&x, ins[l], sizeof x);
        const int i = l % 32, kb = 8 * (l / 32);
        for (int e = 0; e < 8; ++e) {
            A[i][kb + e] = static_cast<float>(x.a[e]);
            B[kb + e][i] = static_cast<float>(x.b[e]);
        }
        for (int r = 0; r < 16; ++r) Cm[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32] = x.c[r];
    }
    for (int l = 0; l < 64; ++l) {
        f16v d;
        for (int r = 0; r < 16; ++r) {
            const int i = 8 * (r / 4) + 4 * (l / 32) + r % 4, j = l % 32;
            double s = Cm[i][j];
            for (int k = 0; k < 16; ++k) s += static_cast<double>(A[i][k]) * B[k][j];
            d[r] = static_cast<float>(s);
        }
        std::memcpy(outs[l], &d, sizeof d);
    }
}
inline f16v mfma_32x32x16_f16(h8 a, h8 b, f16v c, int cbsz, int abid, int blgp) {
    if (cbsz || abid || blgp) die("mfma: broadcast controls are not emulated");
    const MfmaIn x{a, b, c};
    f16v d;
    wave_op("mfma_f32_32x32x16_f16", &x, sizeof x, &d, sizeof d, mfma_fn, nullptr);
    return d;
}

struct DppCtl {
    int ctrl;
};
// DPP quad_perm (ctrl 0x00..0xFF): lane l reads lane 4 (l / 4) + sel(l % 4),
// sel(j) = bits [2j, 2j + 2) of ctrl; row_mirror (0x140): lane l reads lane
// 15 - l within its row of 16; row_half_mirror (0x141): lane 7 - l within its
// half-row of 8. Other DPP controls are not emulated.
template <class T>
inline void dpp_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void* ctx) {
    const int ctrl = static_cast<const DppCtl*>(ctx)->ctrl;
    for (int l = 0; l < 64; ++l) {
        int src;
        if (ctrl == 0x140) src = (l & ~15) + (15 - (l & 15));
        else if (ctrl == 0x141) src = (l & ~7) + (7 - (l & 7));
        else src = (l & ~3) + ((ctrl >> (2 * (l & 3))) & 3);
        std::memcpy(outs[l], ins[src], sizeof(T));
    }
}
template <class T>
inline T mov_dpp(T x, int ctrl, int row_mask, int bank_mask, bool) {
    if (ctrl < 0 || (ctrl > 0xff && ctrl != 0x140 && ctrl != 0x141) || row_mask != 0xf || bank_mask != 0xf)
        die("mov_dpp: only full-mask quad_perm, row_mirror and row_half_mirror are emulated");
    const DppCtl c{ctrl};
    T y;
    wave_op("mov_dpp", &x, sizeof x, &y, sizeof y, dpp_fn<T>, &c);
    return y;
}

template <class T>
inline void first_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void*) {
    for (int l = 0; l < 64; ++l) std::memcpy(outs[l], ins[0], sizeof(T));
}
template <class T>
inline T readfirstlane(T x) {
    T y;
    wave_op("readfirstlane", &x, sizeof x, &y, sizeof y, first_fn<T>, nullptr);
    return y;
}

struct ShflCtl {
    int mask, width;
};
template <class T>
inline void xor_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void* ctx) {
    const ShflCtl c = *static_cast<const ShflCtl*>(ctx);
    for (int l = 0; l < 64; ++l) {
        const int src = l ^ c.mask;
        const bool same_group = (src / c.width) == (l / c.width);
        std::memcpy(outs[l], ins[same_group ? src : l], sizeof(T));
    }
}
template <class T>
inline T shfl_xor(T v, int mask, int width = 64) {
    const ShflCtl c{mask, width};
    T y;
    wave_op("shfl_xor", &v, sizeof v, &y, sizeof y, xor_fn<T>, &c);
    return y;
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i returns element
// i % 4 of the 8-byte pieces addressed by lanes i / 4 + 4 j (j = 0..3) of its
// group, as element j.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
inline void tr16_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void*) {
    for (int l = 0; l < 64; ++l) {
        const int grp = l & ~15, i = l & 15;
        h4 r;
        for (int j = 0; j < 4; ++j) {
            const _Float16* p;
            std::memcpy(&p, ins[grp + i / 4 + 4 * j], sizeof p);
            r[j] = p[i % 4];
        }
        std::memcpy(outs[l], &r, sizeof r);
    }
}
template <class P>
inline h4 ds_read_tr16_b64(P* p) {
    const void* q = static_cast<const void*>(p);
    if (reinterpret_cast<uintptr_t>(q) % 8) die("ds_read_tr16_b64: address not 8-byte aligned");
    h4 r;
    wave_op("ds_read_tr16_b64", &q, sizeof q, &r, sizeof r, tr16_fn, nullptr);
    return r;
}

// v_permlane32_swap: returns {old with lanes 32..63 replaced by src's lanes
// 0..31, src with lanes 0..31 replaced by old's lanes 32..63}.
inline void swap32_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void*) {
    for (int l = 0; l < 64; ++l) {
        uint32_t in_l[2], o[2];
        std::memcpy(in_l, ins[l], 8);
        uint32_t other[2];
        std::memcpy(other, ins[l ^ 32], 8);
        o[0] = l < 32 ? in_l[0] : other[1];
        o[1] = l < 32 ? other[0] : in_l[1];
        std::memcpy(outs[l], o, 8);
    }
}
inline u2v permlane32_swap(uint32_t old, uint32_t src, bool fi, bool bc) {
    if (fi || bc) die("permlane32_swap: fetch-inactive / bound-ctrl not emulated");
    const uint32_t in[2] = {old, src};
    uint32_t o[2];
    wave_op("permlane32_swap", in, 8, o, 8, swap32_fn, nullptr);
    return u2v{o[0], o[1]};
}

// buffer_load_dword* ... lds: lane l's `size` bytes (range-checked like a
// load) are written to LDS at lds + offset + size * l.
inline void buffer_load_lds(Rsrc r, void* lds, int size, uint32_t voff, uint32_t soff, int offset, int) {
    if (size != 4 && size != 12 && size != 16) die("buffer_load_lds: size %d", size);
    uint32_t x[4];
    switch (size) {
        case 4: buf_load<1>(r, voff, soff, x, "raw_ptr_buffer_load_lds"); break;
        case 12: buf_load<3>(r, voff, soff, x, "raw_ptr_buffer_load_lds"); break;
        default: buf_load<4>(r, voff, soff, x, "raw_ptr_buffer_load_lds"); break;
    }
    dma_enqueue(static_cast<unsigned char*>(lds) + offset + static_cast<size_t>(size) * lane_id(), x, size);
}

// s_waitcnt: only the vector-memory count matters here (loads into registers
// complete at once in this emulation; LDS DMA writes wait in a queue).
// gfx9 encoding: vmcnt = imm[3:0] | imm[15:14] << 4.
inline void s_waitcnt(int imm) { dma_wait_vmcnt((imm & 0xF) | (((imm >> 14) & 3) << 4)); }

// wave vote: nonzero in every lane when the predicate holds in any lane
inline void any_fn(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void*) {
    int r = 0;
    for (int l = 0; l < 64; ++l) {
        int x;
        std::memcpy(&x, ins[l], sizeof x);
        r |= x != 0;
    }
    for (int l = 0; l < 64; ++l) std::memcpy(outs[l], &r, sizeof r);
}
inline int vote_any(int pred) {
    int r;
    wave_op("any", &pred, sizeof pred, &r, sizeof r, any_fn, nullptr);
    return r;
}

// v_mbcnt_lo / _hi: base + the set bits of mask that belong to lanes below
// this one, in lanes 0-31 (lo) or 32-63 (hi)
inline unsigned mbcnt_lo(unsigned mask, unsigned base) {
    const int l = lane_id();
    const unsigned below = l >= 32 ? mask : mask & ((1u << l) - 1u);
    return base + static_cast<unsigned>(__builtin_popcount(below));
}
inline unsigned mbcnt_hi(unsigned mask, unsigned base) {
    const int l = lane_id() - 32;
    const unsigned below = l <= 0 ? 0u : mask & ((1u << l) - 1u);
    return base + static_cast<unsigned>(__builtin_popcount(below));
}

// v_dot2_f32_f16: a.x * b.x + a.y * b.y + c, rounded once to fp32 (the fp16
// products and their sum with c are exact in double for the kernels' operands).
typedef _Float16 kemu_h2 __attribute__((ext_vector_type(2)));
inline float fdot2(kemu_h2 a, kemu_h2 b, float c, bool clamp) {
    if (clamp) die("fdot2: clamp not emulated");
    const double r = static_cast<double>(a[0]) * static_cast<double>(b[0]) +
                     static_cast<double>(a[1]) * static_cast<double>(b[1]) + static_cast<double>(c);
    return static_cast<float>(r);
}

inline void nop_fn(const unsigned char (*)[256], unsigned char (*)[256], const void*) {}
inline void wave_barrier() { wave_op("wave_barrier", nullptr, 0, nullptr, 0, nop_fn, nullptr); }

// ---- launches ----------------------------------------------------------------------
template <class... P, class... A>
inline void launch(const char* name, void (*k)(P...), dim3 grid, dim3 block, size_t, hipStream_t, A&&... args) {
    std::tuple<typename std::decay<P>::type...> t(static_cast<typename std::decay<P>::type>(args)...);
    auto f = [&]() { std::apply(k, t); };
    BodyOf<decltype(f)> body(std::move(f));
    run_grid(name, dim3v{grid.x, grid.y, grid.z}, dim3v{block.x, block.y, block.z}, body);
}

}  // namespace kemu

inline int __any(int pred) { return ::kemu::vote_any(pred); }
template <class T>
inline T __shfl_xor(T v, int mask, int width = 64) {
    return ::kemu::shfl_xor(v, mask, width);
}

#define __amdgpu_buffer_rsrc_t ::kemu::Rsrc
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, num, flags) ::kemu::make_rsrc((p), (stride), (num), (flags))
#define __builtin_amdgcn_raw_buffer_load_b16 ::kemu::buffer_load_b16
#define __builtin_amdgcn_raw_buffer_load_b32 ::kemu::buffer_load_b32
#define __builtin_amdgcn_raw_buffer_load_b64 ::kemu::buffer_load_b64
#define __builtin_amdgcn_raw_buffer_load_b128 ::kemu::buffer_load_b128
#define __builtin_amdgcn_raw_buffer_store_b32 ::kemu::buffer_store_b32
#define __builtin_amdgcn_mfma_f32_32x32x16_f16 ::kemu::mfma_32x32x16_f16
#define __builtin_amdgcn_mov_dpp ::kemu::mov_dpp
#define __builtin_amdgcn_readfirstlane ::kemu::readfirstlane
#define __builtin_amdgcn_mbcnt_lo ::kemu::mbcnt_lo
#define __builtin_amdgcn_mbcnt_hi ::kemu::mbcnt_hi
#define __builtin_amdgcn_wave_barrier ::kemu::wave_barrier
#define __builtin_amdgcn_perm ::kemu::perm
#define __builtin_amdgcn_alignbit ::kemu::alignbit
#define __builtin_amdgcn_exp2f exp2f
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define __builtin_amdgcn_ds_read_tr16_b64_v4f16 ::kemu::ds_read_tr16_b64
#define __builtin_amdgcn_permlane32_swap ::kemu::permlane32_swap
#define __builtin_amdgcn_fdot2 ::kemu::fdot2
#define __builtin_amdgcn_raw_ptr_buffer_load_lds ::kemu::buffer_load_lds
#define __builtin_amdgcn_sched_barrier(...) ((void)0)
#define __builtin_amdgcn_sched_group_barrier(...) ((void)0)
#define __builtin_amdgcn_s_waitcnt ::kemu::s_waitcnt
#define __builtin_amdgcn_s_setprio(...) ((void)0)
