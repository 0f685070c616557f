// C++ caller of libmi_sdvk.so through include/mi_sdvk.h alone: the host-side
// calls sdvk's C++ would make (status text, argument rejection, the GGUF
// reader), with no GPU work. Built and run by tests/test_abi.py.
// Usage: abi_host <sample.gguf> <prefix>; prints "key value" lines.
#include <cstdio>
#include <cstring>
#include <vector>

#include "mi_sdvk.h"

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    std::printf("version %d\n", mi_version());
    std::printf("status2 %s\n", mi_status_string(MI_ERR_UNSUPPORTED));
    // a rejected call returns a status and leaves a reason; nothing throws or exits
    int st = mi_gemm_nt_q8_0(nullptr, nullptr, nullptr, nullptr, 8, 8, 32, 0, 0, 0, 1, 0, 0, nullptr);
    std::printf("null_gemm %d %s\n", st, std::strstr(mi_last_error(), "null") ? "reason" : "no-reason");
    st = mi_fused_attn_supported(1280, 20);
    std::printf("attn_supported %d %d\n", st, mi_fused_attn_supported(65, 1));
    mi_gguf* g = nullptr;
    st = mi_gguf_open(argv[1], argv[2], &g);
    std::printf("open %d\n", st);
    if (st != MI_OK) return 1;
    uint64_t n = 0, off = 0, size = 0;
    uint32_t ver = 0;
    mi_gguf_info(g, &ver, &n, &off, &size);
    std::printf("info %u %llu %llu %llu\n", ver, (unsigned long long)n, (unsigned long long)off,
                (unsigned long long)size);
    for (uint64_t i = 0; i < n; ++i) {
        mi_gguf_tensor_info t;
        if (mi_gguf_tensor(g, i, &t) != MI_OK) return 1;
        double sum = 0;
        std::vector<float> f(t.n_elems);
        if (mi_gguf_read_f32(g, i, f.data(), f.size()) == MI_OK)
            for (float v : f)
                if (v == v && v - v == 0) sum += v;  // finite values only
        std::printf("tensor %s %u %llu %llu %llu %.9g\n", t.name, t.type, (unsigned long long)t.nbytes,
                    (unsigned long long)t.rows, (unsigned long long)t.cols, sum);
    }
    mi_gguf_meta_info m;
    if (mi_gguf_meta(g, "general.architecture", &m) == MI_OK) std::printf("arch %s\n", m.str);
    uint64_t idx = 0;
    std::printf("find_missing %d\n", mi_gguf_find(g, "no.such.tensor", &idx));
    mi_gguf_close(g);
    return 0;
}
