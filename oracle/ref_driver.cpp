// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A thin C entry layer over the reference's own GGUF reader
// (src/Modules/Model/Gguf.cpp, compiled from /root/reference by oracle/Makefile
// into oracle/_ref/libgguf_ref.so). It writes a one-tensor GGUF v3 file holding
// the given Q8_0 blocks, opens it with ofc::GgufFile and returns what the
// reference decodes:
//   readFloat  (Gguf.cpp:514-523)  -> fp32 dequant
//   readQ8     (Gguf.cpp:530-557)  -> int8 payload + fp32 scales
//   readQ8Into (Gguf.cpp:559-583)  -> the same, streamed
//   fp16ToFp32 (Gguf.cpp:11-35)
// Used only by tests/test_oracle.py to pin oracle/oracle.c against the
// reference implementation.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "Gguf.hpp"

namespace {

void put(std::FILE* f, const void* p, size_t n) { std::fwrite(p, 1, n, f); }

bool write_gguf(const char* path, const uint8_t* blocks, uint64_t rows, uint64_t cols) {
    std::FILE* f = std::fopen(path, "wb");
    if (!f) return false;
    const uint32_t version = 3;
    const uint64_t n_tensors = 1, n_kv = 0;
    put(f, "GGUF", 4);
    put(f, &version, 4);
    put(f, &n_tensors, 8);
    put(f, &n_kv, 8);
    const std::string name = "w";
    const uint64_t len = name.size();
    put(f, &len, 8);
    put(f, name.data(), name.size());
    const uint32_t nd = 2;
    put(f, &nd, 4);
    put(f, &cols, 8);  // dims[0] = row length (fastest)
    put(f, &rows, 8);
    const uint32_t type = 8;  // Q8_0
    put(f, &type, 4);
    const uint64_t off = 0;
    put(f, &off, 8);
    long pos = std::ftell(f);
    while (pos % 32) {
        std::fputc(0, f);
        ++pos;
    }
    put(f, blocks, (size_t)(rows * cols / 32 * 34));
    std::fclose(f);
    return true;
}

}  // namespace

extern "C" float ref_fp16_to_fp32(uint16_t h) { return ofc::fp16ToFp32(h); }

// Returns 0 on success. out: rows*cols floats; payload: rows*cols int8;
// scales: rows*cols/32 floats; payload2/scales2 receive readQ8Into's result.
extern "C" int ref_q8_0_decode(const char* tmp_path, const uint8_t* blocks, uint64_t rows,
                               uint64_t cols, float* out, int8_t* payload, float* scales,
                               int8_t* payload2, float* scales2) {
    if (!write_gguf(tmp_path, blocks, rows, cols)) return 1;
    ofc::GgufFile g;
    std::string err;
    if (!g.open(tmp_path, &err)) return 2;
    std::vector<float> f = g.readFloat("w", &err);
    if (f.size() != rows * cols) return 3;
    std::memcpy(out, f.data(), f.size() * sizeof(float));
    std::vector<int8_t> q;
    std::vector<float> s;
    if (!g.readQ8("w", q, s, &err)) return 4;
    std::memcpy(payload, q.data(), q.size());
    std::memcpy(scales, s.data(), s.size() * sizeof(float));
    if (!g.readQ8Into("w", payload2, scales2, &err)) return 5;
    return 0;
}
