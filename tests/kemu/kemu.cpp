// kemu.cpp -- fiber runtime of the kernel emulator (see kemu.hpp). Test
// infrastructure: linked only into the emulation build of the library that
// tests/kemu/kemu_build.py makes for CPU-side checks of kernel indexing.
#include "kemu.hpp"

#include <signal.h>
#include <sys/mman.h>
#include <ucontext.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <string>
#include <vector>

extern "C" __attribute__((weak)) char __start_kemu_lds[];
extern "C" __attribute__((weak)) char __stop_kemu_lds[];

namespace kemu {
namespace {

enum State { kRun = 0, kBarrier = 1, kWave = 2, kDone = 3 };

struct Wave {
    int live = 0;
    int arrived = 0;
    const char* op = nullptr;
    unsigned char in[64][256];
    unsigned char out[64][256];
};

}  // namespace

struct PendingDma {
    void* dst;
    unsigned char data[16];
    int size;
};

struct Thread {
    ucontext_t ctx;
    dim3v idx;
    int linear = 0, lane = 0, wave = 0;
    int state = kRun;
    std::deque<PendingDma> dma;  // LDS DMA writes not yet retired by a vmcnt wait
};

namespace {

struct Block {
    std::vector<Thread> th;
    std::vector<Wave> waves;
    int live = 0;
    int at_barrier = 0;
    Body* body = nullptr;
};

Block* g_blk = nullptr;
ucontext_t g_sched;
std::vector<char*> g_stacks;
constexpr size_t kStack = 512 << 10;
constexpr size_t kPage = 4096;
// scheduling order (kemu_set_order): lanes of a wave in reverse order; waves
// in reverse order; wave-major (a wave runs ahead to its next barrier before
// the next wave starts) instead of one wave operation per wave per pass
enum { kRevLanes = 1, kRevWaves = 2, kWaveMajor = 4 };
int g_order = 0, g_rev_blocks = 0;
uint64_t g_launches = 0, g_blocks_run = 0;
// workgroup sampling (kemu_set_sample): the first rule whose kernel text is
// part of the launched kernel's name picks, per grid dimension, every index
// (all) or a list (negative entries count from the end; an empty list runs
// no workgroup of that kernel)
struct SampleRule {
    std::string kernel;
    bool all[3] = {true, true, true};
    std::vector<long> idx[3];
};
std::vector<SampleRule> g_sample;
const char* g_kernel = "";
std::map<void*, std::pair<void*, size_t>> g_allocs;
bool g_handler = false;
struct Copy {
    void* dst;
    const void* src;
    size_t n;
};
std::deque<Copy> g_copies;
uint64_t g_copy_base = 0;  // sequence number of g_copies.front()
char g_altstack[1 << 16];

void on_fault(int sig, siginfo_t* si, void*) {
    const Thread* t = g_cur;
    fprintf(stderr, "kemu: signal %d (fault address %p) in kernel %s, block (%u,%u,%u), thread %d\n", sig,
            si ? si->si_addr : nullptr, g_kernel, g_block_idx.x, g_block_idx.y, g_block_idx.z, t ? t->linear : -1);
    fflush(stderr);
    _exit(71);
}

void install_handler() {
    if (g_handler) return;
    g_handler = true;
    stack_t ss{};
    ss.ss_sp = g_altstack;
    ss.ss_size = sizeof g_altstack;
    sigaltstack(&ss, nullptr);
    struct sigaction sa{};
    sa.sa_sigaction = on_fault;
    sa.sa_flags = SA_SIGINFO | SA_ONSTACK;
    sigaction(SIGSEGV, &sa, nullptr);
    sigaction(SIGBUS, &sa, nullptr);
}

char* stack_for(size_t i) {
    while (g_stacks.size() <= i) {
        // one PROT_NONE page below each stack: an overflow faults instead of
        // overwriting the neighbouring fiber's frames
        char* m = static_cast<char*>(
            mmap(nullptr, kStack + kPage, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0));
        if (m == MAP_FAILED) die("cannot map a fiber stack");
        mprotect(m, kPage, PROT_NONE);
        g_stacks.push_back(m + kPage);
    }
    return g_stacks[i];
}

void release_barrier(Block& b) {
    for (Thread& t : b.th)
        if (t.state == kBarrier) t.state = kRun;
    b.at_barrier = 0;
}

void yield_to_scheduler(Thread* t) { swapcontext(&t->ctx, &g_sched); }

void retire_dma(Thread* t, size_t keep) {
    while (t->dma.size() > keep) {
        const PendingDma& d = t->dma.front();
        std::memcpy(d.dst, d.data, static_cast<size_t>(d.size));
        t->dma.pop_front();
    }
}

void thread_entry() {
    g_blk->body->run();
    Thread* t = g_cur;
    retire_dma(t, 0);
    Block& b = *g_blk;
    Wave& w = b.waves[t->wave];
    t->state = kDone;
    --b.live;
    --w.live;
    if (w.arrived) die("a lane exited while lanes of its wave wait in %s", w.op);
    if (b.at_barrier && b.at_barrier == b.live) release_barrier(b);
    // returning resumes the scheduler (uc_link)
}

void run_block(Block& b) {
    const int n = static_cast<int>(b.th.size());
    for (int i = 0; i < n; ++i) {
        Thread& t = b.th[i];
        getcontext(&t.ctx);
        t.ctx.uc_stack.ss_sp = stack_for(i);
        t.ctx.uc_stack.ss_size = kStack;
        t.ctx.uc_link = &g_sched;
        makecontext(&t.ctx, thread_entry, 0);
        t.state = kRun;
    }
    if (__start_kemu_lds && __stop_kemu_lds > __start_kemu_lds)
        std::memset(__start_kemu_lds, 0xff, static_cast<size_t>(__stop_kemu_lds - __start_kemu_lds));
    const int nw = static_cast<int>(b.waves.size());
    auto run_thread = [&](Thread& t) {
        g_cur = &t;
        swapcontext(&g_sched, &t.ctx);
    };
    // one pass over the wave's runnable lanes; returns whether any ran
    auto pass_wave = [&](int w) {
        bool any = false;
        const int lo = 64 * w, hi = std::min(n, lo + 64);
        for (int ii = lo; ii < hi; ++ii) {
            Thread& t = b.th[(g_order & kRevLanes) ? hi - 1 - (ii - lo) : ii];
            if (t.state != kRun) continue;
            any = true;
            run_thread(t);
        }
        return any;
    };
    while (b.live > 0) {
        bool ran = false;
        for (int wi = 0; wi < nw; ++wi) {
            const int w = (g_order & kRevWaves) ? nw - 1 - wi : wi;
            if (g_order & kWaveMajor) {
                // this wave runs until every lane waits at a barrier or has exited
                while (pass_wave(w)) ran = true;
            } else {
                ran |= pass_wave(w);
            }
        }
        if (!ran) {
            int bar = 0, wv = 0;
            for (const Thread& t : b.th) {
                bar += t.state == kBarrier;
                wv += t.state == kWave;
            }
            g_cur = nullptr;
            die("deadlock: %d work-items at a barrier, %d in cross-lane operations", bar, wv);
        }
    }
    g_cur = nullptr;
}

}  // namespace

Thread* g_cur = nullptr;
dim3v g_block_idx{0, 0, 0}, g_block_dim{1, 1, 1}, g_grid_dim{1, 1, 1};
// the last launch other than a K-split reduce pass (kemu_last_grid / kemu_last_kernel)
const char* g_rec_kernel = "";
dim3v g_rec_grid{1, 1, 1}, g_rec_block{1, 1, 1};

const dim3v& thread_idx() { return g_cur->idx; }
int lane_id() { return g_cur->lane; }

void die(const char* fmt, ...) {
    fprintf(stderr, "kemu: kernel %s, block (%u,%u,%u), thread %d: ", g_kernel, g_block_idx.x, g_block_idx.y,
            g_block_idx.z, g_cur ? g_cur->linear : -1);
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fputc('\n', stderr);
    fflush(stderr);
    _exit(70);
}

void dma_enqueue(void* lds_dst, const void* data, int size) {
    if (size <= 0 || size > 16) die("LDS DMA of %d bytes", size);
    PendingDma d{lds_dst, {}, size};
    std::memcpy(d.data, data, static_cast<size_t>(size));
    g_cur->dma.push_back(d);
}
void dma_wait_vmcnt(int n) { retire_dma(g_cur, static_cast<size_t>(n < 0 ? 0 : n)); }

void enqueue_copy(void* dst, const void* src, size_t n) { g_copies.push_back(Copy{dst, src, n}); }
uint64_t copy_seq() { return g_copy_base + g_copies.size(); }
void flush_copies(uint64_t upto) {
    while (!g_copies.empty() && g_copy_base < upto) {
        const Copy c = g_copies.front();
        g_copies.pop_front();
        ++g_copy_base;
        std::memmove(c.dst, c.src, c.n);
    }
}

void syncthreads() {
    Block& b = *g_blk;
    Thread* t = g_cur;
    if (++b.at_barrier == b.live) {
        release_barrier(b);
        return;
    }
    t->state = kBarrier;
    yield_to_scheduler(t);
}

void wave_op(const char* name, const void* in, size_t n_in, void* out, size_t n_out, WaveFn fn, const void* ctx) {
    Thread* t = g_cur;
    Wave& w = g_blk->waves[t->wave];
    if (w.live != 64) die("%s with %d live lanes in the wave", name, w.live);
    if (n_in > 256 || n_out > 256) die("%s: operand too large", name);
    if (w.arrived == 0) w.op = name;
    else if (std::strcmp(w.op, name) != 0) die("lanes of one wave are in different cross-lane operations (%s, %s)", w.op, name);
    if (n_in) std::memcpy(w.in[t->lane], in, n_in);
    if (++w.arrived == w.live) {
        fn(w.in, w.out, ctx);
        w.arrived = 0;
        for (Thread& x : g_blk->th)
            if (x.wave == t->wave && x.state == kWave) x.state = kRun;
    } else {
        t->state = kWave;
        yield_to_scheduler(t);
    }
    if (n_out) std::memcpy(out, w.out[t->lane], n_out);
}

void run_grid(const char* name, dim3v grid, dim3v block, Body& body) {
    install_handler();
    flush_copies(~0ull);  // stream order: earlier copies complete before the kernel runs
    ++g_launches;
    g_kernel = name;
    const uint64_t nthreads = static_cast<uint64_t>(block.x) * block.y * block.z;
    if (nthreads == 0 || nthreads > 1024) die("block of %llu work-items", static_cast<unsigned long long>(nthreads));
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) die("empty grid");
    if (grid.y > 65535 || grid.z > 65535) die("grid (%u,%u,%u) beyond the launch limits", grid.x, grid.y, grid.z);
    g_grid_dim = grid;
    g_block_dim = block;
    // the routing record skips the K-split reduce pass that follows a split GEMM
    if (!std::strstr(name, "splitk_reduce")) {
        g_rec_kernel = name;
        g_rec_grid = grid;
        g_rec_block = block;
    }
    Block b;
    b.body = &body;
    b.th.resize(nthreads);
    b.waves.resize((nthreads + 63) / 64);
    const SampleRule* rule = nullptr;
    for (const SampleRule& r : g_sample)
        if (r.kernel == "*" || std::strstr(name, r.kernel.c_str())) {
            rule = &r;
            break;
        }
    const uint32_t dims[3] = {grid.x, grid.y, grid.z};
    auto sampled = [&](const dim3v& bi) {
        if (!rule) return true;
        const uint32_t at[3] = {bi.x, bi.y, bi.z};
        for (int d = 0; d < 3; ++d) {
            if (rule->all[d]) continue;
            bool hit = false;
            for (long v : rule->idx[d]) hit |= (v < 0 ? static_cast<long>(dims[d]) + v : v) == static_cast<long>(at[d]);
            if (!hit) return false;
        }
        return true;
    };
    const uint64_t nblocks = static_cast<uint64_t>(grid.x) * grid.y * grid.z;
    for (uint64_t bi = 0; bi < nblocks; ++bi) {
        const uint64_t lin = g_rev_blocks ? nblocks - 1 - bi : bi;
        g_block_idx = dim3v{static_cast<uint32_t>(lin % grid.x), static_cast<uint32_t>(lin / grid.x % grid.y),
                            static_cast<uint32_t>(lin / grid.x / grid.y)};
        if (!sampled(g_block_idx)) continue;
        ++g_blocks_run;
        for (uint64_t i = 0; i < nthreads; ++i) {
            Thread& t = b.th[i];
            t.linear = static_cast<int>(i);
            t.idx = dim3v{static_cast<uint32_t>(i % block.x), static_cast<uint32_t>(i / block.x % block.y),
                          static_cast<uint32_t>(i / block.x / block.y)};
            t.lane = static_cast<int>(i % 64);
            t.wave = static_cast<int>(i / 64);
        }
        for (size_t w = 0; w < b.waves.size(); ++w) {
            b.waves[w].live = static_cast<int>(std::min<uint64_t>(64, nthreads - 64 * w));
            b.waves[w].arrived = 0;
        }
        b.live = static_cast<int>(nthreads);
        b.at_barrier = 0;
        g_blk = &b;
        run_block(b);
        g_blk = nullptr;
    }
}

}  // namespace kemu

using namespace kemu;

extern "C" void* kemu_alloc(size_t bytes, int guard_front) {
    const size_t body = bytes ? (bytes + kPage - 1) / kPage * kPage : kPage;
    char* base = static_cast<char*>(
        mmap(nullptr, body + 2 * kPage, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
    if (base == MAP_FAILED) return nullptr;
    mprotect(base, kPage, PROT_NONE);
    mprotect(base + kPage + body, kPage, PROT_NONE);
    char* p;
    if (guard_front) {
        p = base + kPage;
    } else {
        // the 16-byte-rounded end of the buffer touches the guard page
        const size_t span = (bytes + 15) / 16 * 16;
        p = base + kPage + body - span;
    }
    g_allocs[p] = {base, body + 2 * kPage};
    return p;
}

extern "C" void kemu_free(void* p) {
    auto it = g_allocs.find(p);
    if (it == g_allocs.end()) return;
    munmap(it->second.first, it->second.second);
    g_allocs.erase(it);
}

extern "C" void kemu_set_order(int order, int reverse_blocks) {
    g_order = order;
    g_rev_blocks = reverse_blocks;
}

extern "C" uint64_t kemu_launches(void) { return g_launches; }
extern "C" uint64_t kemu_blocks_run(void) { return g_blocks_run; }
extern "C" void kemu_last_grid(uint32_t* xyz) {
    xyz[0] = g_rec_grid.x;
    xyz[1] = g_rec_grid.y;
    xyz[2] = g_rec_grid.z;
    xyz[3] = g_rec_block.x * g_rec_block.y * g_rec_block.z;
}

// spec: rules separated by ';', each "kernel|x|y|z" (kernel "*": any) where a dimension is '*'
// (every index), '-' (none) or comma-separated indices (negative: from the
// end). An empty spec runs every workgroup of every kernel.
extern "C" void kemu_set_sample(const char* spec) {
    g_sample.clear();
    std::string s = spec ? spec : "";
    size_t pos = 0;
    while (pos < s.size()) {
        size_t end = s.find(';', pos);
        if (end == std::string::npos) end = s.size();
        const std::string item = s.substr(pos, end - pos);
        pos = end + 1;
        if (item.empty()) continue;
        std::vector<std::string> f;
        size_t a = 0;
        for (size_t b; (b = item.find('|', a)) != std::string::npos; a = b + 1) f.push_back(item.substr(a, b - a));
        f.push_back(item.substr(a));
        if (f.size() != 4 || f[0].empty()) die("kemu_set_sample: bad rule '%s'", item.c_str());
        SampleRule r;
        r.kernel = f[0];
        for (int d = 0; d < 3; ++d) {
            const std::string& v = f[d + 1];
            if (v == "*") continue;
            r.all[d] = false;
            if (v == "-") continue;
            size_t c = 0;
            while (c <= v.size()) {
                size_t e = v.find(',', c);
                if (e == std::string::npos) e = v.size();
                char* stop = nullptr;
                const std::string num = v.substr(c, e - c);
                const long x = std::strtol(num.c_str(), &stop, 10);
                if (num.empty() || *stop) die("kemu_set_sample: bad index '%s' in '%s'", num.c_str(), item.c_str());
                r.idx[d].push_back(x);
                c = e + 1;
            }
        }
        g_sample.push_back(std::move(r));
    }
}
extern "C" void kemu_sync(void) { flush_copies(~0ull); }
extern "C" const char* kemu_last_kernel(void) { return g_rec_kernel; }
