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
// reference implementation. The ref_gguf_* entries below expose the whole
// GgufFile API on any file for tests/test_gguf.py, which compares
// libmi_sdvk.so's mi_gguf_* reader with the reference's.
#include <cstdint>
#include <cstdio>
#include <algorithm>
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

// ---- general GgufFile access (any file) ----------------------------------
// Opens `path` with the reference reader and exposes its table, metadata and
// decoders, so tests can compare libmi_sdvk.so's mi_gguf_* results with the
// reference's on the same files (Gguf.hpp:90-140).
namespace {
void copy_str(const std::string& s, char* dst, int cap) {
    if (!dst || cap <= 0) return;
    const size_t n = std::min<size_t>(s.size(), (size_t)cap - 1);
    std::memcpy(dst, s.data(), n);
    dst[n] = 0;
}
}  // namespace

extern "C" void* ref_gguf_open(const char* path, const char* prefix, char* err, int errcap) {
    auto* g = new ofc::GgufFile;
    std::string e;
    if (!g->open(path, &e, prefix ? std::string(prefix) : std::string())) {
        copy_str(e, err, errcap);
        delete g;
        return nullptr;
    }
    return g;
}

extern "C" void ref_gguf_close(void* h) { delete static_cast<ofc::GgufFile*>(h); }

extern "C" uint32_t ref_gguf_version(void* h) { return static_cast<ofc::GgufFile*>(h)->version(); }
extern "C" uint64_t ref_gguf_count(void* h) { return static_cast<ofc::GgufFile*>(h)->tensorCount(); }
extern "C" uint64_t ref_gguf_data_offset(void* h) { return static_cast<ofc::GgufFile*>(h)->dataOffset(); }

extern "C" int ref_gguf_tensor(void* h, uint64_t i, char* name, int cap, uint32_t* type, uint32_t* ndims,
                               uint64_t* dims4, uint64_t* offset, uint64_t* nbytes, uint64_t* rows, uint64_t* cols) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    if (i >= g->tensorCount()) return 1;
    const ofc::GgufTensor& t = g->tensors()[i];
    copy_str(t.name, name, cap);
    *type = (uint32_t)t.type;
    *ndims = (uint32_t)t.dims.size();
    for (size_t d = 0; d < 4; ++d) dims4[d] = d < t.dims.size() ? t.dims[d] : 1;
    *offset = t.offset;
    *nbytes = t.nbytes;
    const auto sh = t.shape();  // GgufTensor::shape (Gguf.cpp:96-102)
    *rows = sh.first;
    *cols = sh.second;
    return 0;
}

// readFloat: returns the element count written, or -1 with the reason in err
extern "C" int64_t ref_gguf_read_float(void* h, const char* name, float* out, uint64_t cap, char* err, int errcap) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    std::string e;
    std::vector<float> v = g->readFloat(name, &e);
    if (v.empty()) {
        copy_str(e, err, errcap);
        return -1;
    }
    if (v.size() > cap) return -2;
    std::memcpy(out, v.data(), v.size() * sizeof(float));
    return (int64_t)v.size();
}

// readQ8 (into = 0) or readQ8Into (into = 1); 0 on success
extern "C" int ref_gguf_read_q8(void* h, const char* name, int8_t* q, float* s, int into, char* err, int errcap) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    std::string e;
    if (into) {
        if (!g->readQ8Into(name, q, s, &e)) {
            copy_str(e, err, errcap);
            return 1;
        }
        return 0;
    }
    std::vector<int8_t> qq;
    std::vector<float> ss;
    if (!g->readQ8(name, qq, ss, &e)) {
        copy_str(e, err, errcap);
        return 1;
    }
    std::memcpy(q, qq.data(), qq.size());
    std::memcpy(s, ss.data(), ss.size() * sizeof(float));
    return 0;
}

extern "C" int ref_gguf_read_raw(void* h, uint64_t i, uint8_t* out, uint64_t cap) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    if (i >= g->tensorCount()) return 1;
    std::vector<uint8_t> v;
    if (!g->readRaw(g->tensors()[i], v)) return 2;
    if (v.size() > cap) return 3;
    std::memcpy(out, v.data(), v.size());
    return 0;
}

// one metadata value; returns 1 when the key is absent
extern "C" int ref_gguf_meta(void* h, const char* key, uint32_t* type, uint64_t* u, double* f, int* b, char* s,
                             int scap, uint32_t* arr_type, uint64_t* arr_len) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    const ofc::GgufMeta* m = g->meta(key);
    if (!m) return 1;
    *type = m->type;
    *u = m->u;
    *f = m->f;
    *b = m->b ? 1 : 0;
    copy_str(m->s, s, scap);
    *arr_type = m->arrType;
    *arr_len = m->strs.size() + m->u64s.size() + m->fs.size() + m->bools.size();
    return 0;
}

// array items: integers / bools -> u64s, floats -> fs, strings one by one via ref_gguf_meta_str_item
extern "C" int ref_gguf_meta_array(void* h, const char* key, uint64_t* u64s, double* fs, uint64_t cap) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    const ofc::GgufMeta* m = g->meta(key);
    if (!m) return 1;
    for (size_t i = 0; i < m->u64s.size() && i < cap; ++i) u64s[i] = m->u64s[i];
    for (size_t i = 0; i < m->bools.size() && i < cap; ++i) u64s[i] = m->bools[i] ? 1 : 0;
    for (size_t i = 0; i < m->fs.size() && i < cap; ++i) fs[i] = m->fs[i];
    return 0;
}

extern "C" int ref_gguf_meta_str_item(void* h, const char* key, uint64_t i, char* s, int cap) {
    auto* g = static_cast<ofc::GgufFile*>(h);
    const ofc::GgufMeta* m = g->meta(key);
    if (!m || i >= m->strs.size()) return 1;
    copy_str(m->strs[i], s, cap);
    return 0;
}

// typed getters (Gguf.cpp:443-478)
extern "C" uint64_t ref_gguf_get_u64(void* h, const char* key, uint64_t def) {
    return static_cast<ofc::GgufFile*>(h)->getU64(key, def);
}
extern "C" int64_t ref_gguf_get_i64(void* h, const char* key, int64_t def) {
    return static_cast<ofc::GgufFile*>(h)->getI64(key, def);
}
extern "C" double ref_gguf_get_f64(void* h, const char* key, double def) {
    return static_cast<ofc::GgufFile*>(h)->getF64(key, def);
}
extern "C" float ref_gguf_get_f32(void* h, const char* key, float def) {
    return static_cast<ofc::GgufFile*>(h)->getF32(key, def);
}
extern "C" int ref_gguf_get_str(void* h, const char* key, const char* def, char* out, int cap) {
    copy_str(static_cast<ofc::GgufFile*>(h)->getStr(key, def ? def : ""), out, cap);
    return 0;
}
