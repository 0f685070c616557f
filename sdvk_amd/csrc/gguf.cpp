// gguf.cpp -- GGUF container reader and device upload of its weights (host side
// of the Q8_0 path: how a real checkpoint's tensors reach mi_gemm_nt_q8_0 /
// mi_gemm_nt_q8_split).
//
// Reference behaviour: src/Modules/Model/Gguf.hpp / Gguf.cpp (GgufFile: header,
// metadata, tensor table, readFloat / readQ8 / readQ8Into) and the upload loop
// loadGgufUnet + ggdims in src/Modules/Diffusion/sdvkgen.cpp:151-176,549-611.
// The implementation is our own: the file is memory-mapped once and parsed
// with a bounds-checked cursor (no stream seeks per tensor); tensor data is
// read straight from the mapping; device uploads stream through two pinned
// staging buffers owned by the handle, so the host copy of chunk i + 1
// overlaps the DMA of chunk i and a multi-GB checkpoint never has a second
// full host copy.
//
// Conventions kept from the reference (the files and callers already depend
// on them):
//   * GGUF v2 / v3 only; at most 2^24 tensors and 2^24 metadata pairs; strings
//     up to 2^30 bytes; arrays up to 2^32 items; 1..4 dims per tensor;
//   * an optional name prefix keeps only tensors that start with it and strips
//     it (full checkpoints store the UNet as model.diffusion_model.*);
//   * data starts at the first multiple of general.alignment (default 32)
//     after the tensor table; the alignment must be a power of two;
//   * tensor byte size = whole blocks of its type (a partial trailing block is
//     counted whole); unknown types count one byte per element;
//   * readFloat decodes F32, F16, BF16, Q4_0 and Q8_0; Q4_0 is expanded with
//     byte i's low nibble at element 2i and its high nibble at 2i + 1
//     (Gguf.cpp:499-511), d * (nibble - 8);
//   * logical (rows, cols) for uploads: comfy.gguf.orig_shape.<name> when it
//     is an array of >= 2 integers (rows = first, cols = product of the rest),
//     else 1-D -> (n, 1), 2-D -> (dims[1], dims[0]), more dims -> rows = the
//     last dim, cols = product of the others (sdvkgen.cpp:151-176).
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace {

using mi::fail;

// GGUF metadata value types (the container's type ids)
enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kStr = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

// ggml tensor types with a decoder here
enum : uint32_t { kTF32 = 0, kTF16 = 1, kTQ4_0 = 2, kTQ4_1 = 3, kTQ5_0 = 6, kTQ5_1 = 7, kTQ8_0 = 8, kTQ8_1 = 9,
                  kTBF16 = 30 };

uint64_t block_elems(uint32_t t) {
    switch (t) {
        case kTQ4_0: case kTQ4_1: case kTQ5_0: case kTQ5_1: case kTQ8_0: case kTQ8_1: return 32;
        default: return 1;
    }
}

uint64_t block_bytes(uint32_t t) {
    switch (t) {
        case kTF32: return 4;
        case kTF16: case kTBF16: return 2;
        case kTQ4_0: return 18;
        case kTQ4_1: return 20;
        case kTQ5_0: return 22;
        case kTQ5_1: return 24;
        case kTQ8_0: return 34;
        case kTQ8_1: return 36;
        default: return 1;
    }
}

// IEEE binary16 -> binary32, exact for every pattern (subnormals by an exact
// scaling, NaN payloads kept).
float half_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float v = static_cast<float>(m) * 5.9604644775390625e-8f;  // m * 2^-24, exact
        std::memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t le16(const uint8_t* p) { return static_cast<uint16_t>(p[0] | (p[1] << 8)); }

struct Meta {
    uint32_t type = 0;
    uint64_t u = 0;       // integer scalars (signed ones sign-extended)
    double f = 0;         // FLOAT32 / FLOAT64
    bool b = false;
    std::string s;
    uint32_t arr_type = 0;
    std::vector<uint64_t> u64s;
    std::vector<double> fs;
    std::vector<std::string> strs;
    std::vector<uint8_t> bools;
    bool is_num() const { return type != kStr && type != kArray; }
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;  // relative to the data section
    uint64_t nbytes = 0;
    uint64_t n_elems() const {
        uint64_t n = 1;
        for (uint32_t i = 0; i < n_dims; ++i) n *= dims[i];
        return n;
    }
};

// Bounds-checked little-endian cursor over the mapped file.
struct Cursor {
    const uint8_t* p;
    uint64_t size, pos = 0;
    bool take(void* dst, uint64_t n) {
        if (n > size - pos) return false;
        std::memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    template <class T> bool get(T& v) { return take(&v, sizeof(T)); }
    bool str(std::string& s) {
        uint64_t len;
        if (!get(len) || len > (uint64_t(1) << 30) || len > size - pos) return false;
        s.assign(reinterpret_cast<const char*>(p + pos), len);
        pos += len;
        return true;
    }
};

bool read_scalar(Cursor& c, uint32_t type, Meta& m) {
    m.type = type;
    switch (type) {
        case kU8: { uint8_t v; if (!c.get(v)) return false; m.u = v; return true; }
        case kI8: { int8_t v; if (!c.get(v)) return false; m.u = static_cast<uint64_t>(static_cast<int64_t>(v)); return true; }
        case kU16: { uint16_t v; if (!c.get(v)) return false; m.u = v; return true; }
        case kI16: { int16_t v; if (!c.get(v)) return false; m.u = static_cast<uint64_t>(static_cast<int64_t>(v)); return true; }
        case kU32: { uint32_t v; if (!c.get(v)) return false; m.u = v; return true; }
        case kI32: { int32_t v; if (!c.get(v)) return false; m.u = static_cast<uint64_t>(static_cast<int64_t>(v)); return true; }
        case kF32: { float v; if (!c.get(v)) return false; m.f = v; return true; }
        case kBool: { uint8_t v; if (!c.get(v)) return false; m.b = v != 0; return true; }
        case kStr: return c.str(m.s);
        case kU64: case kI64: { uint64_t v; if (!c.get(v)) return false; m.u = v; return true; }
        case kF64: { double v; if (!c.get(v)) return false; m.f = v; return true; }
        default: return false;
    }
}

bool read_array(Cursor& c, uint32_t et, uint64_t count, Meta& m) {
    m.arr_type = et;
    if (count > (uint64_t(1) << 32)) return false;
    Meta one;
    switch (et) {
        case kStr:
            m.strs.reserve(std::min<uint64_t>(count, 1u << 20));
            for (uint64_t i = 0; i < count; ++i) {
                if (!c.str(one.s)) return false;
                m.strs.push_back(std::move(one.s));
            }
            return true;
        case kU8: case kI8: case kU16: case kI16: case kU32: case kI32: case kU64: case kI64:
            m.u64s.reserve(std::min<uint64_t>(count, 1u << 20));
            for (uint64_t i = 0; i < count; ++i) {
                if (!read_scalar(c, et, one)) return false;
                m.u64s.push_back(one.u);
            }
            return true;
        case kF32: case kF64:
            m.fs.reserve(std::min<uint64_t>(count, 1u << 20));
            for (uint64_t i = 0; i < count; ++i) {
                if (!read_scalar(c, et, one)) return false;
                m.fs.push_back(one.f);
            }
            return true;
        case kBool:
            m.bools.reserve(std::min<uint64_t>(count, 1u << 20));
            for (uint64_t i = 0; i < count; ++i) {
                if (!read_scalar(c, et, one)) return false;
                m.bools.push_back(one.b ? 1 : 0);
            }
            return true;
        default: return false;
    }
}

}  // namespace

// The opaque handle of include/mi_sdvk.h.
struct mi_gguf {
    std::string path;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    std::map<std::string, Meta> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, uint64_t> by_name;
    // upload staging: two pinned buffers, each guarded by the event of the
    // last copy that reads it
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool stage_used[2] = {false, false};

    ~mi_gguf() {
        for (int i = 0; i < 2; ++i) {
            if (done[i]) {
                (void)hipEventSynchronize(done[i]);
                (void)hipEventDestroy(done[i]);
            }
            if (stage[i]) (void)hipHostFree(stage[i]);
        }
        if (map) munmap(const_cast<uint8_t*>(map), size);
    }
};

namespace {

constexpr uint64_t kStageBytes = uint64_t(8) << 20;  // per staging buffer

int parse(mi_gguf& g, const char* prefix) {
    const char* fn = "mi_gguf_open";
    Cursor c{g.map, g.size};
    char magic[4];
    if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0)
        return fail(MI_ERR_IO, "%s: %s: bad magic (not a GGUF file)", fn, g.path.c_str());
    uint32_t version;
    if (!c.get(version) || (version != 2 && version != 3))
        return fail(MI_ERR_IO, "%s: %s: unsupported GGUF version", fn, g.path.c_str());
    g.version = version;
    uint64_t n_tensors, n_kv;
    if (!c.get(n_tensors) || !c.get(n_kv)) return fail(MI_ERR_IO, "%s: %s: truncated header", fn, g.path.c_str());
    if (n_tensors > (uint64_t(1) << 24) || n_kv > (uint64_t(1) << 24))
        return fail(MI_ERR_IO, "%s: %s: implausible counts", fn, g.path.c_str());

    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        if (!c.str(key)) return fail(MI_ERR_IO, "%s: truncated kv key", fn);
        uint32_t type;
        if (!c.get(type)) return fail(MI_ERR_IO, "%s: truncated kv type", fn);
        Meta m;
        if (type == kArray) {
            uint32_t et;
            uint64_t count;
            if (!c.get(et) || !c.get(count)) return fail(MI_ERR_IO, "%s: truncated array header", fn);
            m.type = kArray;
            if (!read_array(c, et, count, m)) return fail(MI_ERR_IO, "%s: truncated array items for %s", fn, key.c_str());
        } else if (!read_scalar(c, type, m)) {
            return fail(MI_ERR_IO, "%s: truncated kv value for %s", fn, key.c_str());
        }
        g.meta[key] = std::move(m);
    }

    const std::string pre = prefix ? prefix : "";
    g.tensors.reserve(static_cast<size_t>(n_tensors));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        if (!c.str(t.name)) return fail(MI_ERR_IO, "%s: truncated tensor name", fn);
        if (!c.get(t.n_dims) || t.n_dims == 0 || t.n_dims > 4) return fail(MI_ERR_IO, "%s: bad tensor ndims", fn);
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (!c.get(t.dims[d])) return fail(MI_ERR_IO, "%s: truncated tensor dims", fn);
        if (!c.get(t.type)) return fail(MI_ERR_IO, "%s: truncated tensor type", fn);
        if (!c.get(t.offset)) return fail(MI_ERR_IO, "%s: truncated tensor offset", fn);
        if (!pre.empty()) {
            if (t.name.compare(0, pre.size(), pre) != 0) continue;
            t.name.erase(0, pre.size());
        }
        const uint64_t be = block_elems(t.type), bb = block_bytes(t.type), ne = t.n_elems();
        t.nbytes = (ne / be) * bb + ((ne % be) ? bb : 0);
        if (g.by_name.count(t.name)) return fail(MI_ERR_IO, "%s: duplicate tensor %s", fn, t.name.c_str());
        g.by_name[t.name] = g.tensors.size();
        g.tensors.push_back(std::move(t));
    }

    uint64_t align = 32;
    auto it = g.meta.find("general.alignment");
    if (it != g.meta.end() && it->second.is_num()) align = static_cast<uint32_t>(it->second.u);
    if (align == 0 || (align & (align - 1))) return fail(MI_ERR_IO, "%s: bad alignment", fn);
    g.alignment = static_cast<uint32_t>(align);
    g.data_offset = (c.pos + align - 1) / align * align;
    if (g.data_offset > g.size) return fail(MI_ERR_IO, "%s: data offset beyond EOF", fn);
    return MI_OK;
}

const Tensor* tensor_at(const mi_gguf* g, uint64_t index, const char* fn, int* st) {
    if (!g) {
        *st = fail(MI_ERR_INVALID_ARG, "%s: null handle", fn);
        return nullptr;
    }
    if (index >= g->tensors.size()) {
        *st = fail(MI_ERR_NOT_FOUND, "%s: tensor index %llu >= %zu", fn, static_cast<unsigned long long>(index),
                   g->tensors.size());
        return nullptr;
    }
    return &g->tensors[index];
}

// Tensor bytes inside the mapping, or null when the file is shorter than the
// table claims (the reference's readRaw fails the same way).
const uint8_t* tensor_bytes(const mi_gguf* g, const Tensor& t) {
    const uint64_t start = g->data_offset + t.offset;
    if (t.offset > g->size || start > g->size || t.nbytes > g->size - start) return nullptr;
    return g->map + start;
}

void logical_dims(const mi_gguf* g, const Tensor& t, uint64_t& rows, uint64_t& cols) {
    auto it = g->meta.find("comfy.gguf.orig_shape." + t.name);
    if (it != g->meta.end() && it->second.type == kArray && it->second.u64s.size() >= 2) {
        rows = it->second.u64s[0];
        cols = 1;
        for (size_t i = 1; i < it->second.u64s.size(); ++i) cols *= it->second.u64s[i];
        return;
    }
    if (t.n_dims <= 1) {
        rows = t.dims[0];
        cols = 1;
    } else if (t.n_dims > 2) {
        rows = t.dims[t.n_dims - 1];
        cols = 1;
        for (uint32_t i = 0; i + 1 < t.n_dims; ++i) cols *= t.dims[i];
    } else {
        rows = t.dims[1];
        cols = t.dims[0];
    }
}

bool decodable(uint32_t type) {
    return type == kTF32 || type == kTF16 || type == kTBF16 || type == kTQ4_0 || type == kTQ8_0;
}

// Decodes elements [e0, e1) of tensor data p (readFloat semantics); e0 and e1
// are multiples of the type's block size except at the tensor's end.
void decode_range(uint32_t type, const uint8_t* p, uint64_t e0, uint64_t e1, float* out) {
    switch (type) {
        case kTF32:
            std::memcpy(out, p + e0 * 4, (e1 - e0) * 4);
            return;
        case kTF16:
            for (uint64_t i = e0; i < e1; ++i) out[i - e0] = half_to_float(le16(p + 2 * i));
            return;
        case kTBF16:
            for (uint64_t i = e0; i < e1; ++i) {
                const uint32_t bits = static_cast<uint32_t>(le16(p + 2 * i)) << 16;
                std::memcpy(&out[i - e0], &bits, 4);
            }
            return;
        case kTQ4_0:
            for (uint64_t b = e0 / 32; b < e1 / 32; ++b) {
                const uint8_t* blk = p + b * 18;
                const float d = half_to_float(le16(blk));
                float* o = out + (b * 32 - e0);
                for (int i = 0; i < 16; ++i) {
                    o[2 * i] = d * static_cast<float>((blk[2 + i] & 0x0f) - 8);
                    o[2 * i + 1] = d * static_cast<float>((blk[2 + i] >> 4) - 8);
                }
            }
            return;
        case kTQ8_0:
            for (uint64_t b = e0 / 32; b < e1 / 32; ++b) {
                const uint8_t* blk = p + b * 34;
                const float d = half_to_float(le16(blk));
                float* o = out + (b * 32 - e0);
                for (int i = 0; i < 32; ++i) o[i] = d * static_cast<float>(static_cast<int8_t>(blk[2 + i]));
            }
            return;
        default: return;
    }
}

// Q8_0 blocks [b0, b1) -> int8 payload + fp32 scales (readQ8Into semantics).
void split_range(const uint8_t* p, uint64_t b0, uint64_t b1, int8_t* q, float* s) {
    for (uint64_t b = b0; b < b1; ++b) {
        const uint8_t* blk = p + b * 34;
        s[b - b0] = half_to_float(le16(blk));
        std::memcpy(q + (b - b0) * 32, blk + 2, 32);
    }
}

// Waits until staging buffer i is free and returns it (allocated on first use).
int acquire_stage(mi_gguf* g, int i, const char* fn, void** buf) {
    if (!g->stage[i]) {
        if (hipHostMalloc(&g->stage[i], kStageBytes, hipHostMallocDefault) != hipSuccess) {
            g->stage[i] = nullptr;
            return fail(MI_ERR_HIP, "%s: pinned staging allocation failed", fn);
        }
        if (hipEventCreateWithFlags(&g->done[i], hipEventDisableTiming) != hipSuccess) {
            g->done[i] = nullptr;
            return fail(MI_ERR_HIP, "%s: event creation failed", fn);
        }
    }
    if (g->stage_used[i] && hipEventSynchronize(g->done[i]) != hipSuccess)
        return fail(MI_ERR_HIP, "%s: staging wait failed", fn);
    *buf = g->stage[i];
    return MI_OK;
}

int enqueue_copy(mi_gguf* g, int i, void* dst, const void* src, uint64_t n, hipStream_t s, const char* fn) {
    if (hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipEventRecord(g->done[i], s) != hipSuccess)
        return fail(MI_ERR_HIP, "%s: %s", fn, hipGetErrorString(hipGetLastError()));
    g->stage_used[i] = true;
    return MI_OK;
}

}  // namespace

// ------------------------------------------------------------------- C-ABI --

extern "C" int mi_gguf_open(const char* path, const char* prefix, mi_gguf** out) {
    const char* fn = "mi_gguf_open";
    if (!path || !out) return fail(MI_ERR_INVALID_ARG, "%s: null argument", fn);
    *out = nullptr;
    mi_gguf* g = new (std::nothrow) mi_gguf;
    if (!g) return fail(MI_ERR_INVALID_ARG, "%s: out of host memory", fn);
    g->path = path;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        delete g;
        return fail(MI_ERR_IO, "%s: cannot open %s", fn, path);
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        delete g;
        return fail(MI_ERR_IO, "%s: cannot stat %s", fn, path);
    }
    g->size = static_cast<uint64_t>(sb.st_size);
    if (g->size > 0) {
        void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            delete g;
            return fail(MI_ERR_IO, "%s: cannot map %s", fn, path);
        }
        g->map = static_cast<const uint8_t*>(m);
    }
    close(fd);
    int st;
    try {
        st = parse(*g, prefix);
    } catch (const std::bad_alloc&) {
        st = fail(MI_ERR_IO, "%s: out of host memory while parsing %s", fn, path);
    }
    if (st != MI_OK) {
        delete g;
        return st;
    }
    *out = g;
    return MI_OK;
}

extern "C" void mi_gguf_close(mi_gguf* g) { delete g; }

extern "C" int mi_gguf_info(const mi_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* data_offset,
                            uint64_t* file_size) {
    if (!g) return fail(MI_ERR_INVALID_ARG, "mi_gguf_info: null handle");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (data_offset) *data_offset = g->data_offset;
    if (file_size) *file_size = g->size;
    return MI_OK;
}

extern "C" int mi_gguf_tensor(const mi_gguf* g, uint64_t index, mi_gguf_tensor_info* info) {
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, "mi_gguf_tensor", &st);
    if (!t) return st;
    if (!info) return fail(MI_ERR_INVALID_ARG, "mi_gguf_tensor: null info");
    info->name = t->name.c_str();
    info->type = t->type;
    info->n_dims = t->n_dims;
    for (int i = 0; i < 4; ++i) info->dims[i] = i < static_cast<int>(t->n_dims) ? t->dims[i] : 1;
    info->offset = t->offset;
    info->nbytes = t->nbytes;
    info->n_elems = t->n_elems();
    logical_dims(g, *t, info->rows, info->cols);
    return MI_OK;
}

extern "C" int mi_gguf_find(const mi_gguf* g, const char* name, uint64_t* index) {
    if (!g || !name || !index) return fail(MI_ERR_INVALID_ARG, "mi_gguf_find: null argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return fail(MI_ERR_NOT_FOUND, "mi_gguf_find: tensor not found: %s", name);
    *index = it->second;
    return MI_OK;
}

extern "C" int mi_gguf_meta(const mi_gguf* g, const char* key, mi_gguf_meta_info* info) {
    if (!g || !key || !info) return fail(MI_ERR_INVALID_ARG, "mi_gguf_meta: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return fail(MI_ERR_NOT_FOUND, "mi_gguf_meta: no key %s", key);
    const Meta& m = it->second;
    info->type = m.type;
    info->u = m.u;
    info->f = m.f;
    info->b = m.b ? 1 : 0;
    info->str = m.type == kStr ? m.s.c_str() : nullptr;
    info->str_len = m.type == kStr ? m.s.size() : 0;
    info->arr_type = m.arr_type;
    info->arr_len = m.type != kArray ? 0
                    : !m.strs.empty() ? m.strs.size()
                    : !m.u64s.empty() ? m.u64s.size()
                    : !m.fs.empty()   ? m.fs.size()
                                      : m.bools.size();
    return MI_OK;
}

extern "C" int mi_gguf_meta_array(const mi_gguf* g, const char* key, uint64_t first, uint64_t count, uint64_t* u64s,
                                  double* f64s, const char** strs) {
    if (!g || !key) return fail(MI_ERR_INVALID_ARG, "mi_gguf_meta_array: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return fail(MI_ERR_NOT_FOUND, "mi_gguf_meta_array: no key %s", key);
    const Meta& m = it->second;
    if (m.type != kArray) return fail(MI_ERR_INVALID_ARG, "mi_gguf_meta_array: %s is not an array", key);
    const uint64_t len = m.strs.size() + m.u64s.size() + m.fs.size() + m.bools.size();
    if (first > len || count > len - first)
        return fail(MI_ERR_INVALID_ARG, "mi_gguf_meta_array: items [%llu, %llu) of %llu", static_cast<unsigned long long>(first),
                    static_cast<unsigned long long>(first + count), static_cast<unsigned long long>(len));
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t j = first + i;
        if (!m.u64s.empty()) {
            if (u64s) u64s[i] = m.u64s[j];
        } else if (!m.bools.empty()) {
            if (u64s) u64s[i] = m.bools[j];
        } else if (!m.fs.empty()) {
            if (f64s) f64s[i] = m.fs[j];
        } else if (!m.strs.empty()) {
            if (strs) strs[i] = m.strs[j].c_str();
        }
    }
    return MI_OK;
}

extern "C" int mi_gguf_read_raw(const mi_gguf* g, uint64_t index, void* dst, uint64_t dst_bytes) {
    const char* fn = "mi_gguf_read_raw";
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, fn, &st);
    if (!t) return st;
    if (!dst || dst_bytes < t->nbytes)
        return fail(MI_ERR_INVALID_ARG, "%s: destination of %llu bytes < %llu", fn,
                    static_cast<unsigned long long>(dst_bytes), static_cast<unsigned long long>(t->nbytes));
    const uint8_t* p = tensor_bytes(g, *t);
    if (!p) return fail(MI_ERR_IO, "%s: read failed: %s (data past end of file)", fn, t->name.c_str());
    std::memcpy(dst, p, t->nbytes);
    return MI_OK;
}

extern "C" int mi_gguf_read_f32(const mi_gguf* g, uint64_t index, float* dst, uint64_t n) {
    const char* fn = "mi_gguf_read_f32";
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, fn, &st);
    if (!t) return st;
    const uint64_t ne = t->n_elems();
    if (!dst || n < ne) return fail(MI_ERR_INVALID_ARG, "%s: destination of %llu floats < %llu", fn,
                                    static_cast<unsigned long long>(n), static_cast<unsigned long long>(ne));
    if (!decodable(t->type)) return fail(MI_ERR_UNSUPPORTED, "%s: unsupported quant type %u (%s)", fn, t->type, t->name.c_str());
    const uint8_t* p = tensor_bytes(g, *t);
    if (!p) return fail(MI_ERR_IO, "%s: read failed: %s (data past end of file)", fn, t->name.c_str());
    const uint64_t whole = (ne / block_elems(t->type)) * block_elems(t->type);
    decode_range(t->type, p, 0, whole, dst);
    std::fill(dst + whole, dst + ne, 0.0f);  // a partial trailing block decodes to zeros, like readFloat
    return MI_OK;
}

extern "C" int mi_gguf_read_q8_split(const mi_gguf* g, uint64_t index, int8_t* payload, float* scales) {
    const char* fn = "mi_gguf_read_q8_split";
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, fn, &st);
    if (!t) return st;
    if (!payload || !scales) return fail(MI_ERR_INVALID_ARG, "%s: null destination", fn);
    if (t->type != kTQ8_0) return fail(MI_ERR_UNSUPPORTED, "%s: tensor %s is type %u, not Q8_0", fn, t->name.c_str(), t->type);
    const uint8_t* p = tensor_bytes(g, *t);
    if (!p) return fail(MI_ERR_IO, "%s: read failed: %s (data past end of file)", fn, t->name.c_str());
    split_range(p, 0, t->n_elems() / 32, payload, scales);
    return MI_OK;
}

extern "C" int mi_gguf_upload_raw(mi_gguf* g, uint64_t index, void* dst, uint64_t dst_bytes, void* stream) {
    const char* fn = "mi_gguf_upload_raw";
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, fn, &st);
    if (!t) return st;
    if (!dst || dst_bytes < t->nbytes)
        return fail(MI_ERR_INVALID_ARG, "%s: destination of %llu bytes < %llu", fn,
                    static_cast<unsigned long long>(dst_bytes), static_cast<unsigned long long>(t->nbytes));
    const uint8_t* p = tensor_bytes(g, *t);
    if (!p) return fail(MI_ERR_IO, "%s: read failed: %s (data past end of file)", fn, t->name.c_str());
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t* d = static_cast<uint8_t*>(dst);
    int k = 0;
    for (uint64_t off = 0; off < t->nbytes; off += kStageBytes, k ^= 1) {
        const uint64_t n = std::min(kStageBytes, t->nbytes - off);
        void* buf;
        if ((st = acquire_stage(g, k, fn, &buf)) != MI_OK) return st;
        std::memcpy(buf, p + off, n);
        if ((st = enqueue_copy(g, k, d + off, buf, n, s, fn)) != MI_OK) return st;
    }
    return MI_OK;
}

extern "C" int mi_gguf_upload_f32(mi_gguf* g, uint64_t index, float* dst, uint64_t n, void* stream) {
    const char* fn = "mi_gguf_upload_f32";
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, fn, &st);
    if (!t) return st;
    const uint64_t ne = t->n_elems();
    if (!dst || n < ne) return fail(MI_ERR_INVALID_ARG, "%s: destination of %llu floats < %llu", fn,
                                    static_cast<unsigned long long>(n), static_cast<unsigned long long>(ne));
    if (!decodable(t->type)) return fail(MI_ERR_UNSUPPORTED, "%s: unsupported quant type %u (%s)", fn, t->type, t->name.c_str());
    const uint8_t* p = tensor_bytes(g, *t);
    if (!p) return fail(MI_ERR_IO, "%s: read failed: %s (data past end of file)", fn, t->name.c_str());
    const uint64_t be = block_elems(t->type);
    const uint64_t whole = (ne / be) * be;
    const uint64_t chunk = kStageBytes / 4 / 32 * 32;  // elements per chunk, whole blocks
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int k = 0;
    for (uint64_t e0 = 0; e0 < ne; e0 += chunk, k ^= 1) {
        const uint64_t e1 = std::min(ne, e0 + chunk), d1 = std::min(e1, whole);
        void* buf;
        if ((st = acquire_stage(g, k, fn, &buf)) != MI_OK) return st;
        float* f = static_cast<float*>(buf);
        if (d1 > e0) decode_range(t->type, p, e0, d1, f);
        std::fill(f + (std::max(d1, e0) - e0), f + (e1 - e0), 0.0f);  // partial trailing block -> zeros
        if ((st = enqueue_copy(g, k, dst + e0, buf, (e1 - e0) * 4, s, fn)) != MI_OK) return st;
    }
    return MI_OK;
}

extern "C" int mi_gguf_upload_q8_split(mi_gguf* g, uint64_t index, int8_t* payload, float* scales, void* stream) {
    const char* fn = "mi_gguf_upload_q8_split";
    int st = MI_OK;
    const Tensor* t = tensor_at(g, index, fn, &st);
    if (!t) return st;
    if (!payload || !scales) return fail(MI_ERR_INVALID_ARG, "%s: null destination", fn);
    if (t->type != kTQ8_0) return fail(MI_ERR_UNSUPPORTED, "%s: tensor %s is type %u, not Q8_0", fn, t->name.c_str(), t->type);
    const uint8_t* p = tensor_bytes(g, *t);
    if (!p) return fail(MI_ERR_IO, "%s: read failed: %s (data past end of file)", fn, t->name.c_str());
    const uint64_t nb = t->n_elems() / 32;
    const uint64_t chunk = kStageBytes / 36;  // blocks per chunk: 32 payload + 4 scale bytes each
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int k = 0;
    for (uint64_t b0 = 0; b0 < nb; b0 += chunk, k ^= 1) {
        const uint64_t b1 = std::min(nb, b0 + chunk), cnt = b1 - b0;
        void* buf;
        if ((st = acquire_stage(g, k, fn, &buf)) != MI_OK) return st;
        int8_t* q = static_cast<int8_t*>(buf);
        float* sc = reinterpret_cast<float*>(q + cnt * 32);  // cnt * 32 is a multiple of 4
        split_range(p, b0, b1, q, sc);
        if ((st = enqueue_copy(g, k, payload + b0 * 32, q, cnt * 32, s, fn)) != MI_OK) return st;
        if ((st = enqueue_copy(g, k, scales + b0, sc, cnt * 4, s, fn)) != MI_OK) return st;
    }
    return MI_OK;
}
