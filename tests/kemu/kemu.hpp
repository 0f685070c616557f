// kemu.hpp -- CPU emulation of the gfx950 execution model used by the
// library's kernels, for tests only. The product's .hip sources are compiled
// for the host against include/hip/hip_runtime.h (this directory), which maps
// HIP's device dialect onto this runtime:
//
//   * a workgroup is run as blockDim fibers (one per work-item) on one OS
//     thread; __syncthreads() is a fiber barrier over the work-items that have
//     not exited;
//   * a wavefront is 64 consecutive work-items; every cross-lane operation
//     (MFMA, DPP, readfirstlane, shuffles, wave barrier) is a rendezvous of the
//     wave's 64 lanes: each lane deposits its operand, the last to arrive
//     computes the result for all lanes. A wave operation reached by some lanes
//     and not others, or with exited lanes, is reported as an error;
//   * __shared__ arrays live in one linker section that is filled with 0xFF
//     (a NaN pattern) before every workgroup, so a read of LDS that was never
//     written shows up in the results;
//   * buffer resources range-check every dword like the hardware's raw buffer
//     loads (out of range: loads return 0, stores are dropped);
//   * a DMA load into LDS writes LDS only when an s_waitcnt vmcnt of the
//     issuing work-item retires it (or the work-item exits);
//   * device memory is host memory; tests allocate it with kemu_alloc, which
//     places the buffer against a PROT_NONE guard page, so an access past its
//     end faults and the fault handler names the kernel, workgroup and lane.
//
// Work-items between two synchronisation points run one after another, in an
// order set by kemu_set_order (bit 0: lanes of a wave in reverse; bit 1: waves
// in reverse; bit 2: wave-major, each wave runs ahead to its next barrier
// before the next wave starts), so a missing barrier between a write and
// another work-item's read changes the results under some order.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <tuple>
#include <type_traits>
#include <utility>

namespace kemu {

struct dim3v {
    uint32_t x, y, z;
};

struct Thread;
extern Thread* g_cur;
extern dim3v g_block_idx, g_block_dim, g_grid_dim;
const dim3v& thread_idx();

[[noreturn]] void die(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// ---- synchronisation -----------------------------------------------------------
void syncthreads();
// Rendezvous of the current wave: copies `in` (n_in bytes) into the lane's
// slot; the last lane to arrive runs fn(ins, outs) over all 64 lanes; then
// copies the lane's n_out bytes of output back into `out`.
typedef void (*WaveFn)(const unsigned char (*ins)[256], unsigned char (*outs)[256], const void* ctx);
void wave_op(const char* name, const void* in, size_t n_in, void* out, size_t n_out, WaveFn fn, const void* ctx);
int lane_id();

// ---- LDS DMA (buffer_load ... lds) ----------------------------------------------------
// The LDS write of a DMA load lands when the issuing work-item's
// s_waitcnt vmcnt(n) retires it (oldest first, until n remain), or when the
// work-item exits -- not at a barrier (the hardware's s_barrier does not wait
// for vector memory), so a read of a DMA target that no wait covers sees the
// old LDS contents.
void dma_enqueue(void* lds_dst, const void* data, int size);
void dma_wait_vmcnt(int n);

// ---- deferred copies -------------------------------------------------------------
void enqueue_copy(void* dst, const void* src, size_t n);
uint64_t copy_seq();                 // sequence number after the last enqueued copy
void flush_copies(uint64_t upto);    // runs the copies numbered below `upto`

// ---- launches ------------------------------------------------------------------
struct Body {
    virtual void run() = 0;
    virtual ~Body() {}
};
void run_grid(const char* name, dim3v grid, dim3v block, Body& body);

template <class F>
struct BodyOf : Body {
    F f;
    explicit BodyOf(F&& x) : f(std::move(x)) {}
    void run() override { f(); }
};

}  // namespace kemu

extern "C" {
void* kemu_alloc(size_t bytes, int guard_front);
void kemu_free(void* p);
void kemu_set_order(int order, int reverse_blocks);
uint64_t kemu_launches(void);
uint64_t kemu_blocks_run(void);  // workgroups emulated so far
void kemu_set_sample(const char* spec);  // run only some workgroups (kemu.cpp)
void kemu_last_grid(uint32_t* xyz);      // grid (x, y, z) and work-items per block of the last launch
                                        // (a K-split reduce pass is not recorded)
void kemu_sync(void);  // runs every deferred copy
const char* kemu_last_kernel(void);
}
