// status.hip -- status strings, thread-local error detail, version, and the
// process-wide plan overrides of mi_tuning_set.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mi {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return MI_OK;
}

Tuning& tuning() {
    static Tuning t;
    return t;
}

}  // namespace mi

namespace {

// Parses a decimal integer that fills the whole of [p, end); false otherwise.
bool parse_int(const char* p, const char* end, long lo, long hi, long* out) {
    if (p == end) return false;
    char buf[32];
    const size_t n = static_cast<size_t>(end - p);
    if (n >= sizeof(buf)) return false;
    std::memcpy(buf, p, n);
    buf[n] = '\0';
    char* e = nullptr;
    const long v = std::strtol(buf, &e, 10);
    if (*e != '\0' || v < lo || v > hi) return false;
    *out = v;
    return true;
}

// "<a>" or "<a>:<b>" into a (and b, or b_default when absent).
bool parse_pair(const char* v, long lo_a, long hi_a, long lo_b, long hi_b, long b_default, long* a, long* b) {
    const char* c = std::strchr(v, ':');
    const char* end = v + std::strlen(v);
    if (!parse_int(v, c ? c : end, lo_a, hi_a, a)) return false;
    if (!c) {
        *b = b_default;
        return true;
    }
    return parse_int(c + 1, end, lo_b, hi_b, b);
}

}  // namespace

extern "C" int mi_tuning_set(const char* name, const char* value) {
    using mi::fail;
    if (!name) return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: null name");
    mi::Tuning& t = mi::tuning();
    const bool clear = value == nullptr || *value == '\0';
    long a = 0, b = 0;
    if (std::strcmp(name, "gemm_cfg") == 0) {
        if (clear) {
            t.gemm_cfg.store(-1);
            t.gemm_splits.store(1);
            return MI_OK;
        }
        if (!parse_pair(value, 0, mi::kGemmBuilds - 1, 1, 64, 1, &a, &b))
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: gemm_cfg \"%s\" (want <0..%d>[:<1..64>])", value,
                        mi::kGemmBuilds - 1);
        t.gemm_splits.store(static_cast<int>(b));
        t.gemm_cfg.store(static_cast<int>(a));
        return MI_OK;
    }
    if (std::strcmp(name, "nn_kernel") == 0) {
        if (!clear && std::strcmp(value, "general") != 0)
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: nn_kernel \"%s\" (want general)", value);
        t.nn_general.store(clear ? 0 : 1);
        return MI_OK;
    }
    if (std::strcmp(name, "nn_splits") == 0) {
        if (!clear && !parse_int(value, value + std::strlen(value), 1, 64, &a))
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: nn_splits \"%s\" (want 1..64)", value);
        t.nn_splits.store(clear ? 0 : static_cast<int>(a));
        return MI_OK;
    }
    if (std::strcmp(name, "attn_nw") == 0) {
        if (!clear && std::strcmp(value, "2") != 0 && std::strcmp(value, "4") != 0)
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: attn_nw \"%s\" (want 2 or 4)", value);
        t.attn_nw.store(clear ? 0 : std::atoi(value));
        return MI_OK;
    }
    if (std::strcmp(name, "attn_split") == 0) {
        if (clear) {
            t.attn_split_rest.store(-1);
            return MI_OK;
        }
        if (!parse_pair(value, 0, 1L << 30, 1, 64, 2, &a, &b))
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: attn_split \"%s\" (want <rest>[:<pieces>], 0 = off)",
                        value);
        t.attn_split_pieces.store(static_cast<int>(b));
        t.attn_split_rest.store(static_cast<int>(a));
        return MI_OK;
    }
    if (std::strcmp(name, "attn_direct_store") == 0) {
        if (!clear && std::strcmp(value, "1") != 0 && std::strcmp(value, "0") != 0)
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: attn_direct_store \"%s\" (want 0 or 1)", value);
        t.attn_direct_store.store(!clear && value[0] == '1' ? 1 : 0);
        return MI_OK;
    }
    if (std::strcmp(name, "attn_simd_waves") == 0) {
        if (!clear && std::strcmp(value, "2") != 0 && std::strcmp(value, "3") != 0)
            return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: attn_simd_waves \"%s\" (want 2 or 3)", value);
        t.attn_simd_waves.store(clear ? 0 : std::atoi(value));
        return MI_OK;
    }
    return fail(MI_ERR_INVALID_ARG, "mi_tuning_set: unknown name \"%s\"", name);
}

extern "C" void mi_tuning_reset(void) {
    mi::Tuning& t = mi::tuning();
    t.gemm_cfg.store(-1);
    t.gemm_splits.store(1);
    t.nn_general.store(0);
    t.nn_splits.store(0);
    t.attn_nw.store(0);
    t.attn_split_rest.store(-1);
    t.attn_split_pieces.store(2);
    t.attn_direct_store.store(0);
    t.attn_simd_waves.store(0);
}

extern "C" const char* mi_status_string(int status) {
    switch (status) {
        case MI_OK: return "ok";
        case MI_ERR_INVALID_ARG: return "invalid argument";
        case MI_ERR_UNSUPPORTED: return "unsupported shape";
        case MI_ERR_ALIGNMENT: return "alignment requirement not met";
        case MI_ERR_ALIASING: return "output overlaps an input";
        case MI_ERR_HIP: return "HIP runtime error";
        case MI_ERR_IO: return "file or format error";
        case MI_ERR_NOT_FOUND: return "not found";
        default: return "unknown status";
    }
}

extern "C" const char* mi_last_error(void) { return g_last_error; }

extern "C" int mi_version(void) { return 200; /* 0.2.0: mi_attn_args.precision, mi_tuning_set */ }
