// C++ caller of libmi_sdvk.so with GPU work, through include/mi_sdvk.h and the
// HIP runtime alone: the reference's two harnesses restated against the C-ABI.
//
//   gpu_harness gemm <outdir>   tests/gemm_q8_bench.cpp:59-109,141-156 -- the
//       correctness case (M = N = 100, K = 96, A = i8/127, B int8, scales
//       0.01, inputs from std::mt19937(7) like the reference) through every
//       kernel name of kVariants (gemm_nt_q8, gemm_nt_q8_v, _v_bm128, _v_bk32,
//       _v_bm128_bk32: one C-ABI entry, mi_gemm_nt_q8_split, serves them all),
//       plus K = 90 (any K, the scalar gemm_nt_q8's range) and the 34-byte
//       block entry; then the reference's timing table (its five shapes, best
//       of 3, hipEvents on the launch stream).
//   gpu_harness attn <outdir>   tests/fused_attn_test.cpp:74-126 -- its four
//       shapes (causal self, 77-key cross, hd = 40, hd = 64 cross) with inputs
//       from std::mt19937(20261101) U(-1, 1), through mi_fused_attention (fp32
//       [T, C], the reference's FusedAttnArgs), and its latency lines.
//
// Inputs and outputs are written to <outdir> as raw little-endian arrays so
// that the Python test checks them against the CPU oracle (the harness itself
// only prints the reference harness's relative error against its own CPU loop,
// as the reference does). Exit status: 0 when every call returned MI_OK.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "mi_sdvk.h"

namespace {

int g_fail = 0;

#define HIP_OK(x)                                                                    \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));             \
            std::exit(3);                                                            \
        }                                                                            \
    } while (0)

void check(int st, const char* what) {
    if (st != MI_OK) {
        std::printf("FAIL %s: %s (%s)\n", what, mi_status_string(st), mi_last_error());
        ++g_fail;
    }
}

template <typename T>
void save(const std::string& dir, const char* name, const std::vector<T>& v) {
    const std::string p = dir + "/" + name + ".bin";
    FILE* f = std::fopen(p.c_str(), "wb");
    if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) {
        std::fprintf(stderr, "cannot write %s\n", p.c_str());
        std::exit(4);
    }
    std::fclose(f);
}

template <typename T>
T* to_device(const std::vector<T>& v) {
    void* p = nullptr;
    HIP_OK(hipMalloc(&p, std::max<size_t>(v.size() * sizeof(T), 16)));
    HIP_OK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    return static_cast<T*>(p);
}

template <typename T>
std::vector<T> from_device(const T* p, size_t n) {
    std::vector<T> v(n);
    HIP_OK(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
    return v;
}

double rel_max(const std::vector<float>& got, const std::vector<float>& ref) {
    double max_abs = 0, max_ref = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        max_abs = std::max(max_abs, std::fabs(static_cast<double>(got[i]) - ref[i]));
        max_ref = std::max(max_ref, std::fabs(static_cast<double>(ref[i])));
    }
    return max_abs / std::max(1e-9, max_ref);
}

// The reference's correctness case: its generator, its CPU loop, every kernel name.
void gemm_case(const std::string& dir, uint32_t K, const char* tag) {
    const uint32_t M = 100, N = 100;
    std::mt19937 rng(7);
    std::uniform_int_distribution<int> i8(-127, 127);
    std::vector<float> A(static_cast<size_t>(M) * K);
    std::vector<int8_t> B(static_cast<size_t>(N) * K);
    std::vector<float> S((static_cast<size_t>(N) * K + 31) / 32, 0.01f);
    for (auto& x : A) x = static_cast<float>(i8(rng)) / 127.0f;
    for (auto& x : B) x = static_cast<int8_t>(i8(rng));
    std::vector<float> ref(static_cast<size_t>(M) * N, 0.0f);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t n = 0; n < N; ++n) {
            float acc = 0;
            for (uint32_t k = 0; k < K; ++k)
                acc += A[static_cast<size_t>(m) * K + k] *
                       (static_cast<float>(B[static_cast<size_t>(n) * K + k]) * S[(static_cast<size_t>(n) * K + k) >> 5]);
            ref[static_cast<size_t>(m) * N + n] = acc;
        }
    std::vector<uint32_t> payload((B.size() + 3) / 4, 0u);
    std::memcpy(payload.data(), B.data(), B.size());
    float* dA = to_device(A);
    uint32_t* dB = to_device(payload);
    float* dS = to_device(S);
    float* dC = nullptr;
    HIP_OK(hipMalloc(reinterpret_cast<void**>(&dC), static_cast<size_t>(M) * N * 4));
    save(dir, (std::string(tag) + "_A").c_str(), A);
    save(dir, (std::string(tag) + "_B").c_str(), B);
    save(dir, (std::string(tag) + "_S").c_str(), S);
    // gemm_q8_bench.cpp:33-39: every name is one C-ABI entry with the Pg fields
    // {M, N, K, mode 0, sA 0, sB 0, sC 0, batch 1, lda 0, ldb 0, ldc 0}
    const char* names[] = {"gemm_nt_q8", "gemm_nt_q8_v", "gemm_nt_q8_v_bm128", "gemm_nt_q8_v_bk32",
                           "gemm_nt_q8_v_bm128_bk32"};
    for (const char* name : names) {
        const bool vec = std::strcmp(name, "gemm_nt_q8") != 0;
        if (vec && K % 4) continue;  // the vectorised names need K % 4 == 0 (gemm_nt_q8_v.comp:69,86)
        HIP_OK(hipMemset(dC, 0xff, static_cast<size_t>(M) * N * 4));
        check(mi_gemm_nt_q8_split(dA, dB, dS, nullptr, dC, M, N, K, 0, 0, 0, 1, 0, 0, nullptr), name);
        HIP_OK(hipDeviceSynchronize());
        std::vector<float> got = from_device(dC, static_cast<size_t>(M) * N);
        std::printf("check %-4s %-24s rel=%.3g\n", tag, name, rel_max(got, ref));
        save(dir, (std::string(tag) + "_C_" + name).c_str(), got);
    }
    HIP_OK(hipFree(dA));
    HIP_OK(hipFree(dB));
    HIP_OK(hipFree(dS));
    HIP_OK(hipFree(dC));
}

// The same weights as 34-byte Q8_0 blocks (fp16 d = 0.01 rounded) through the north-star entry.
void gemm_blocks_case(const std::string& dir) {
    const uint32_t M = 100, N = 100, K = 96;
    std::mt19937 rng(7);
    std::uniform_int_distribution<int> i8(-127, 127);
    std::vector<float> A(static_cast<size_t>(M) * K);
    std::vector<int8_t> B(static_cast<size_t>(N) * K);
    for (auto& x : A) x = static_cast<float>(i8(rng)) / 127.0f;
    for (auto& x : B) x = static_cast<int8_t>(i8(rng));
    const uint16_t d16 = 0x211f;  // fp16 nearest to 0.01 (0.01000213623046875)
    std::vector<uint8_t> blocks(static_cast<size_t>(N) * (K / 32) * 34);
    for (size_t b = 0; b < blocks.size() / 34; ++b) {
        std::memcpy(&blocks[b * 34], &d16, 2);
        std::memcpy(&blocks[b * 34 + 2], &B[b * 32], 32);
    }
    float* dA = to_device(A);
    uint8_t* dW = to_device(blocks);
    float* dC = nullptr;
    HIP_OK(hipMalloc(reinterpret_cast<void**>(&dC), static_cast<size_t>(M) * N * 4));
    check(mi_gemm_nt_q8_0(dA, dW, nullptr, dC, M, N, K, 0, 0, 0, 1, 0, 0, nullptr), "mi_gemm_nt_q8_0");
    HIP_OK(hipDeviceSynchronize());
    save(dir, "q80_blocks", blocks);
    save(dir, "q80_C", from_device(dC, static_cast<size_t>(M) * N));
    HIP_OK(hipFree(dA));
    HIP_OK(hipFree(dW));
    HIP_OK(hipFree(dC));
}

// gemm_q8_bench.cpp:111-156: zero-filled operands, best of 3 per shape.
void gemm_timing() {
    struct Shape {
        uint32_t M, N, K;
    };
    const Shape shapes[] = {{9216, 1280, 1280}, {9216, 640, 640}, {9216, 320, 320}, {2304, 1280, 1280}, {576, 1280, 2560}};
    hipStream_t s;
    HIP_OK(hipStreamCreate(&s));
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    std::printf("\n%-22s %12s %10s\n", "shape MxNxK", "best ms", "GFLOP/s");
    for (const Shape& sh : shapes) {
        void *A, *B, *S, *C;
        HIP_OK(hipMalloc(&A, static_cast<size_t>(sh.M) * sh.K * 4));
        HIP_OK(hipMalloc(&B, (static_cast<size_t>(sh.N) * sh.K + 3) / 4 * 4));
        HIP_OK(hipMalloc(&S, (static_cast<size_t>(sh.N) * sh.K + 31) / 32 * 4));
        HIP_OK(hipMalloc(&C, static_cast<size_t>(sh.M) * sh.N * 4));
        HIP_OK(hipMemset(A, 0, static_cast<size_t>(sh.M) * sh.K * 4));
        HIP_OK(hipMemset(B, 0, (static_cast<size_t>(sh.N) * sh.K + 3) / 4 * 4));
        HIP_OK(hipMemset(S, 0, (static_cast<size_t>(sh.N) * sh.K + 31) / 32 * 4));
        double best = 1e30;
        for (int it = 0; it < 4; ++it) {  // the first call warms up
            HIP_OK(hipEventRecord(e0, s));
            check(mi_gemm_nt_q8_split(static_cast<float*>(A), static_cast<uint32_t*>(B), static_cast<float*>(S), nullptr,
                                      static_cast<float*>(C), sh.M, sh.N, sh.K, 0, 0, 0, 1, 0, 0, s),
                  "timing");
            HIP_OK(hipEventRecord(e1, s));
            HIP_OK(hipEventSynchronize(e1));
            float ms = 0;
            HIP_OK(hipEventElapsedTime(&ms, e0, e1));
            if (it > 0) best = std::min(best, static_cast<double>(ms));
        }
        const std::string name = std::to_string(sh.M) + "x" + std::to_string(sh.N) + "x" + std::to_string(sh.K);
        std::printf("%-22s %12.4f %10.0f\n", name.c_str(), best, 2.0 * sh.M * sh.N * sh.K / (best * 1e6));
        HIP_OK(hipFree(A));
        HIP_OK(hipFree(B));
        HIP_OK(hipFree(S));
        HIP_OK(hipFree(C));
    }
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    HIP_OK(hipStreamDestroy(s));
}

int run_gemm(const std::string& dir) {
    gemm_case(dir, 96, "k96");
    gemm_case(dir, 90, "k90");
    gemm_blocks_case(dir);
    gemm_timing();
    return g_fail ? 1 : 0;
}

// fused_attn_test.cpp:74-126: four shapes, one generator for all of them.
int run_attn(const std::string& dir) {
    struct Shape {
        const char* name;
        uint32_t Tq, Tk, C, heads;
        bool causal;
    };
    const Shape shapes[] = {
        {"self T=32 C=320 h=5 causal", 32, 32, 320, 5, true},
        {"cross Tq=32 Tk=77 C=1280 h=20", 32, 77, 1280, 20, false},
        {"self T=64 C=320 h=8 causal hd40", 64, 64, 320, 8, true},
        {"cross Tq=48 Tk=96 C=512 h=8", 48, 96, 512, 8, false},
    };
    std::mt19937 rng(20261101);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    int idx = 0;
    std::vector<double> lat;
    for (const Shape& s : shapes) {
        if (!mi_fused_attn_supported(s.C, s.heads)) {
            std::printf("FAIL %s: not supported\n", s.name);
            ++g_fail;
            continue;
        }
        std::vector<float> q(static_cast<size_t>(s.Tq) * s.C), k(static_cast<size_t>(s.Tk) * s.C),
            v(static_cast<size_t>(s.Tk) * s.C);
        for (auto& x : q) x = dist(rng);
        for (auto& x : k) x = dist(rng);
        for (auto& x : v) x = dist(rng);
        float* dq = to_device(q);
        float* dk = to_device(k);
        float* dv = to_device(v);
        float* dout = nullptr;
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&dout), q.size() * 4));
        check(mi_fused_attention(dq, dk, dv, dout, s.Tq, s.Tk, s.C, s.heads, s.causal ? 1 : 0, nullptr), s.name);
        HIP_OK(hipDeviceSynchronize());
        std::vector<float> got = from_device(dout, q.size());
        double best = 1e30;
        for (int it = 0; it < 4; ++it) {
            HIP_OK(hipEventRecord(e0, nullptr));
            check(mi_fused_attention(dq, dk, dv, dout, s.Tq, s.Tk, s.C, s.heads, s.causal ? 1 : 0, nullptr), s.name);
            HIP_OK(hipEventRecord(e1, nullptr));
            HIP_OK(hipEventSynchronize(e1));
            float ms = 0;
            HIP_OK(hipEventElapsedTime(&ms, e0, e1));
            if (it > 0) best = std::min(best, static_cast<double>(ms));
        }
        lat.push_back(best);
        std::printf("ran  %-38s\n", s.name);
        const std::string p = "s" + std::to_string(idx++);
        save(dir, (p + "_q").c_str(), q);
        save(dir, (p + "_k").c_str(), k);
        save(dir, (p + "_v").c_str(), v);
        save(dir, (p + "_o").c_str(), got);
        HIP_OK(hipFree(dq));
        HIP_OK(hipFree(dk));
        HIP_OK(hipFree(dv));
        HIP_OK(hipFree(dout));
    }
    std::printf("\nlatency (fused attention only):\n");
    for (size_t i = 0; i < lat.size(); ++i) std::printf("  %-38s %.4f ms\n", shapes[i].name, lat[i]);
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    return g_fail ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    if (argc < 3) {
        std::fprintf(stderr, "usage: gpu_harness gemm|attn <outdir>\n");
        return 2;
    }
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n));
    if (n < 1) {
        std::fprintf(stderr, "no HIP device\n");
        return 3;
    }
    if (std::strcmp(argv[1], "gemm") == 0) return run_gemm(argv[2]);
    if (std::strcmp(argv[1], "attn") == 0) return run_attn(argv[2]);
    return 2;
}
