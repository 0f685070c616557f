// block.hip -- one SDXL BasicTransformerBlock (diffusers layout) on the
// library's kernels, in the reference's order (src/Modules/Diffusion/
// sdvkgen.cpp:1739-1763, crossAttention :1283-1290, geglu :1709-1720):
//
//   n = LN1(x); x += attn1(n, n)        attn(a, b) = out(attention(q(a), k(b), v(b))) + out_bias
//   n = LN2(x); x += attn2(n, ctx)
//   n = LN3(x); x += ff_down(geglu(ff_up(n) + up_bias)) + down_bias
//
// Rows are batch-stacked ([batch * tokens, C]); self- and cross-attention run
// per batch item through the batched attention entry. All intermediates live
// in a caller-provided workspace (nothing is allocated), every launch is
// ordered on the caller's stream.
//
// mi_block_dims.flags:
//   MI_BLOCK_FUSED_EPILOGUES: the out-projections and FF-down add their product
//     and bias straight into x (GEMM mode 2) and FF-up applies GEGLU in its
//     epilogue (mi_gemm_nt_q8_0_geglu), which removes the three residual-add
//     passes and the [rows, 2 ff_inner] intermediate;
//   MI_BLOCK_JOINT_QKV: attn1 to_q / to_k / to_v are one [3C, C] Q8_0 matrix
//     (the three pointers must be C x C matrices apart), projected by one GEMM;
//   MI_BLOCK_FP16_ACTIVATIONS: LayerNorm, attention and GEGLU outputs stored as
//     fp16 for the GEMMs that read them (the GEMM rounds its A operand to fp16
//     anyway: the same bits);
//   MI_BLOCK_FP16_ATTENTION: the Q / K / V projections (and the cached context
//     K / V) are stored as fp16, the RNE rounding of their fp32 results, and
//     both attentions run on fp16 inputs (the fp16 kernel's pipeline) instead
//     of splitting fp32 inputs into fp16 hi + lo parts. Attention then works at
//     the precision of the library's fp16 attention entries; the block's bits
//     differ from the flag-off block by that rounding.
// Within one setting of MI_BLOCK_FP16_ATTENTION every variant computes the same bits: the GEMMs whose results must agree
// across variants (Q / K / V, context K / V, FF-up) never split K, the
// residual GEMMs split K the same way in both epilogue forms (partials in the
// workspace, summed in a fixed order), and an unsplit GEMM's sums do not
// depend on the tile build.
#include "common.hpp"

namespace mi {
namespace {

struct Workspace {
    float *n, *q, *k, *v, *o, *a, *h, *g;
    float* split;           // K-split partials of the residual GEMMs
    uint64_t split_bytes;
};

uint64_t round256(uint64_t b) { return (b + 255) / 256 * 256; }

// Workspace the residual GEMMs' K splits use (out-projections: K = C,
// FF-down: K = ff_inner; both N = C).
uint64_t split_bytes(const mi_block_dims& d) {
    const uint32_t rows = d.batch * d.tokens;
    const uint64_t a = mi_gemm_nt_q8_workspace_bytes(rows, d.channels, d.channels, 1);
    const uint64_t b = mi_gemm_nt_q8_workspace_bytes(rows, d.channels, d.ff_inner, 1);
    return a > b ? a : b;
}

// Byte layout of the workspace; returns the total. h holds FF-up's
// [rows, 2 ff_inner] output and, before the FF stage, the joint Q/K/V
// projection's [rows, 3C].
uint64_t layout(const mi_block_dims& d, char* base, Workspace* w) {
    const uint64_t rows = static_cast<uint64_t>(d.batch) * d.tokens;
    const uint64_t crow = static_cast<uint64_t>(d.batch) * d.ctx_tokens;
    const uint64_t kvrows = rows > crow ? rows : crow;
    const uint64_t hcols = 2ull * d.ff_inner > 3ull * d.channels ? 2ull * d.ff_inner : 3ull * d.channels;
    const uint64_t sizes[8] = {rows * d.channels, rows * d.channels, kvrows * d.channels, kvrows * d.channels,
                               rows * d.channels, rows * d.channels, rows * hcols, rows * d.ff_inner};
    float** slots[8] = {&w->n, &w->q, &w->k, &w->v, &w->o, &w->a, &w->h, &w->g};
    uint64_t off = 0;
    for (int i = 0; i < 8; ++i) {
        if (base) *slots[i] = reinterpret_cast<float*>(base + off);
        off += round256(sizes[i] * 4);
    }
    w->split_bytes = split_bytes(d);
    w->split = base && w->split_bytes ? reinterpret_cast<float*>(base + off) : nullptr;
    off += round256(w->split_bytes);
    return off;
}

int check_dims(const mi_block_dims& d, const char* fn) {
    if (!d.batch || !d.tokens || !d.channels || !d.heads || !d.ctx_tokens || !d.ctx_channels || !d.ff_inner)
        return fail(MI_ERR_INVALID_ARG, "%s: zero dimension", fn);
    if (!mi_fused_attn_supported(d.channels, d.heads))
        return fail(MI_ERR_UNSUPPORTED, "%s: channels %u / heads %u not served by the fused attention", fn, d.channels,
                    d.heads);
    if (d.channels % 32 || d.ctx_channels % 32 || d.ff_inner % 32)
        return fail(MI_ERR_UNSUPPORTED, "%s: channels, ctx_channels and ff_inner must be multiples of 32 (Q8_0 K)", fn);
    if (d.flags & ~static_cast<uint32_t>(MI_BLOCK_FUSED_EPILOGUES | MI_BLOCK_JOINT_QKV | MI_BLOCK_FP16_ACTIVATIONS |
                                         MI_BLOCK_FP16_ATTENTION))
        return fail(MI_ERR_INVALID_ARG, "%s: unknown flags 0x%x", fn, d.flags);
    return MI_OK;
}

#define MI_TRY(expr)              \
    do {                          \
        const int st_ = (expr);   \
        if (st_ != MI_OK) return st_; \
    } while (0)

// ld: token stride of q, k and v (C, or 3C for the joint Q/K/V projection);
// in_half: q, k, v hold fp16; o_half: the output stored as fp16
int attention(const mi_block_dims& d, const void* q, const void* k, const void* v, uint64_t ld, void* o,
              uint32_t tk, const int32_t* kv_len, bool in_half, bool o_half, hipStream_t s) {
    mi_attn_args x{};
    x.q = q;
    x.k = k;
    x.v = v;
    x.ldq = ld;
    x.ldk = ld;
    x.ldv = ld;
    x.out = o;
    x.batch = d.batch;
    x.Tq = d.tokens;
    x.Tk = tk;
    x.C = d.channels;
    x.heads = d.heads;
    x.in_dtype = in_half ? MI_F16 : MI_F32;
    x.out_dtype = o_half ? MI_F16 : MI_F32;
    x.kv_len = kv_len;
    // the output only feeds the out-projection GEMM, which rounds its A
    // operand to fp16: one fp16 P product (2^-11 per weight) is below that
    x.precision = MI_ATTN_PREC_FP16;
    return mi_fused_attention_ex(&x, s);
}

// MI_BLOCK_JOINT_QKV: Q, K and V weights stored back to back ([Wq; Wk; Wv],
// one 3C x C Q8_0 matrix) take one projection GEMM with N = 3C instead of three
// (a grid three times wider: larger tiles fill the CUs); attention then reads
// Q / K / V from the [rows, 3C] result at token stride 3C.
bool adjacent(const void* a, const void* b, uint64_t bytes) {
    return static_cast<const char*>(a) + bytes == static_cast<const char*>(b);
}

int check_weights(const mi_block_weights& w, const mi_block_dims& d, const char* fn) {
    const void* mats[10] = {w.attn1_q, w.attn1_k, w.attn1_v, w.attn1_out, w.attn2_q,
                            w.attn2_k, w.attn2_v, w.attn2_out, w.ff_up, w.ff_down};
    for (const void* m : mats)
        if (!m) return fail(MI_ERR_INVALID_ARG, "%s: null weight", fn);
    const uint64_t wcc = static_cast<uint64_t>(d.channels) * (d.channels / 32) * 34;  // one C x C Q8_0 matrix
    if ((d.flags & MI_BLOCK_JOINT_QKV) && !(adjacent(w.attn1_q, w.attn1_k, wcc) && adjacent(w.attn1_k, w.attn1_v, wcc)))
        return fail(MI_ERR_INVALID_ARG, "%s: MI_BLOCK_JOINT_QKV needs attn1_k = attn1_q + %llu bytes and attn1_v = "
                    "attn1_k + %llu bytes (one [3C, C] matrix)", fn, static_cast<unsigned long long>(wcc),
                    static_cast<unsigned long long>(wcc));
    return MI_OK;
}

bool fp16_attention(const mi_block_dims& d) { return (d.flags & MI_BLOCK_FP16_ATTENTION) != 0; }

// Bytes of the cached cross-attention K and V: two [batch * ctx_tokens, channels]
// tensors, fp32 (fp16 with MI_BLOCK_FP16_ATTENTION).
uint64_t ctx_kv_bytes(const mi_block_dims& d) {
    return 2 * round256(static_cast<uint64_t>(d.batch) * d.ctx_tokens * d.channels * (fp16_attention(d) ? 2 : 4));
}

// K and V of the context, into k / v (fp32, or fp16 with MI_BLOCK_FP16_ATTENTION).
int ctx_kv(const mi_block_weights& w, const mi_block_dims& d, const float* ctx, void* k, void* v, hipStream_t s) {
    const uint32_t crow = d.batch * d.ctx_tokens;
    if (fp16_attention(d)) {
        MI_TRY(mi_gemm_nt_q8_0_f16o(ctx, MI_F32, w.attn2_k, nullptr, k, crow, d.channels, d.ctx_channels, 0, 0, s));
        return mi_gemm_nt_q8_0_f16o(ctx, MI_F32, w.attn2_v, nullptr, v, crow, d.channels, d.ctx_channels, 0, 0, s);
    }
    MI_TRY(mi_gemm_nt_q8_0(ctx, w.attn2_k, nullptr, static_cast<float*>(k), crow, d.channels, d.ctx_channels, 0, 0, 0,
                           1, 0, 0, s));
    return mi_gemm_nt_q8_0(ctx, w.attn2_v, nullptr, static_cast<float*>(v), crow, d.channels, d.ctx_channels, 0, 0, 0,
                           1, 0, 0, s);
}

// One block. Cross-attention K / V come from `kv` (K then V, ctx_kv_bytes
// layout) when given, else are projected from `ctx` into the workspace.
int forward(const mi_block_weights& w, const mi_block_dims& d, float* x, const float* ctx, const void* kv,
            const int32_t* ctx_len, void* workspace, uint64_t workspace_bytes, hipStream_t s, const char* fn) {
    MI_TRY(check_dims(d, fn));
    MI_TRY(check_weights(w, d, fn));
    Workspace ws;
    const uint64_t need = layout(d, static_cast<char*>(workspace), &ws);
    if (workspace_bytes < need)
        return fail(MI_ERR_INVALID_ARG, "%s: workspace %llu bytes < %llu needed", fn,
                    static_cast<unsigned long long>(workspace_bytes), static_cast<unsigned long long>(need));
    if (!aligned(workspace, 256)) return fail(MI_ERR_ALIGNMENT, "%s: workspace must be 256-byte aligned", fn);

    const uint32_t rows = d.batch * d.tokens, C = d.channels;
    const uint64_t nx = static_cast<uint64_t>(rows) * C;
    const bool fused = (d.flags & MI_BLOCK_FUSED_EPILOGUES) != 0;
    // fp16 activations: n (LayerNorm out), o (attention out) and g (GEGLU out)
    // hold fp16 and feed the fp16-A GEMM (same bits as fp32 + staging)
    const bool half = (d.flags & MI_BLOCK_FP16_ACTIVATIONS) != 0;
    auto gemm = [&](const void* A, const void* W, const float* bias, float* out, uint32_t M, uint32_t N, uint32_t K) {
        if (half) return mi_gemm_nt_q8_0_f16a(A, W, bias, out, M, N, K, 0, 0, 0, 1, 0, 0, nullptr, 0, s);
        return mi_gemm_nt_q8_0(static_cast<const float*>(A), W, bias, out, M, N, K, 0, 0, 0, 1, 0, 0, s);
    };
    auto gemm_ws = [&](const void* A, const void* W, const float* bias, float* out, uint32_t K, uint32_t mode) {
        if (half) return mi_gemm_nt_q8_0_f16a(A, W, bias, out, rows, C, K, mode, 0, 0, 1, 0, 0, ws.split,
                                              ws.split_bytes, s);
        return mi_gemm_nt_q8_0_ws(static_cast<const float*>(A), W, bias, out, rows, C, K, mode, 0, 0, 1, 0, 0,
                                  ws.split, ws.split_bytes, s);
    };
    // MI_BLOCK_FP16_ATTENTION: the Q / K / V projections store fp16 (element
    // offsets below count halves then)
    const bool hattn = fp16_attention(d);
    const uint64_t esz = hattn ? 2 : 4;
    auto proj = [&](const void* A, const void* W, void* out, uint32_t N) {
        if (hattn) return mi_gemm_nt_q8_0_f16o(A, half ? MI_F16 : MI_F32, W, nullptr, out, rows, N, C, 0, 0, s);
        return gemm(A, W, nullptr, static_cast<float*>(out), rows, N, C);
    };
    auto at = [&](const void* base, uint64_t elems) { return static_cast<const char*>(base) + elems * esz; };
    auto layernorm = [&](const float* g, const float* b) {
        return half ? mi_layernorm_f16(x, g, b, ws.n, rows, C, 1e-5f, s) : mi_layernorm(x, g, b, ws.n, rows, C, 1e-5f, s);
    };
    // x += A . W^T + bias: one GEMM with the residual epilogue, or GEMM + add;
    // both split K the same way (the workspace's partials region)
    auto residual = [&](const void* A, const void* W, const float* bias, uint32_t K) {
        if (fused) return gemm_ws(A, W, bias, x, K, 2);
        const int st = gemm_ws(A, W, bias, ws.a, K, 0);
        return st != MI_OK ? st : mi_add_inplace(x, ws.a, nx, s);
    };

    // self-attention
    MI_TRY(layernorm(w.norm1_w, w.norm1_b));
    // the joint result [rows, 3C] goes to the FF-up region, free until the FF stage
    if (d.flags & MI_BLOCK_JOINT_QKV) {
        MI_TRY(proj(ws.n, w.attn1_q, ws.h, 3 * C));
        MI_TRY(attention(d, ws.h, at(ws.h, C), at(ws.h, 2ull * C), 3ull * C, ws.o, d.tokens, nullptr, hattn, half, s));
    } else {
        MI_TRY(proj(ws.n, w.attn1_q, ws.q, C));
        MI_TRY(proj(ws.n, w.attn1_k, ws.k, C));
        MI_TRY(proj(ws.n, w.attn1_v, ws.v, C));
        MI_TRY(attention(d, ws.q, ws.k, ws.v, C, ws.o, d.tokens, nullptr, hattn, half, s));
    }
    MI_TRY(residual(ws.o, w.attn1_out, w.attn1_out_b, C));
    // cross-attention over the context
    MI_TRY(layernorm(w.norm2_w, w.norm2_b));
    MI_TRY(proj(ws.n, w.attn2_q, ws.q, C));
    const void *ck = ws.k, *cv = ws.v;
    if (kv) {
        ck = kv;
        cv = static_cast<const char*>(kv) + ctx_kv_bytes(d) / 2;
    } else {
        MI_TRY(ctx_kv(w, d, ctx, ws.k, ws.v, s));
    }
    MI_TRY(attention(d, ws.q, ck, cv, C, ws.o, d.ctx_tokens, ctx_len, hattn, half, s));
    MI_TRY(residual(ws.o, w.attn2_out, w.attn2_out_b, C));
    // GEGLU feed-forward
    MI_TRY(layernorm(w.norm3_w, w.norm3_b));
    if (fused) {
        if (half) MI_TRY(mi_gemm_nt_q8_0_geglu_f16(ws.n, w.ff_up, w.ff_up_b, ws.g, rows, d.ff_inner, C, 0, 0, s));
        else MI_TRY(mi_gemm_nt_q8_0_geglu(ws.n, w.ff_up, w.ff_up_b, ws.g, rows, d.ff_inner, C, 0, 0, s));
    } else {
        MI_TRY(gemm(ws.n, w.ff_up, w.ff_up_b, ws.h, rows, 2 * d.ff_inner, C));
        if (half) MI_TRY(mi_geglu_f16(ws.h, ws.g, rows, d.ff_inner, s));
        else MI_TRY(mi_geglu(ws.h, ws.g, rows, d.ff_inner, s));
    }
    MI_TRY(residual(ws.g, w.ff_down, w.ff_down_b, d.ff_inner));
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" uint64_t mi_block_workspace_bytes(const mi_block_dims* dims) {
    if (!dims) return 0;
    Workspace w;
    return layout(*dims, nullptr, &w);
}

extern "C" int mi_sdxl_block_forward(const mi_block_weights* wt, const mi_block_dims* dims, float* x, const float* ctx,
                                     const int32_t* ctx_len, void* workspace, uint64_t workspace_bytes, void* stream) {
    const char* fn = "mi_sdxl_block_forward";
    if (!wt || !dims || !x || !ctx || !workspace) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    return forward(*wt, *dims, x, ctx, nullptr, ctx_len, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                   fn);
}

extern "C" uint64_t mi_block_ctx_kv_bytes(const mi_block_dims* dims) { return dims ? ctx_kv_bytes(*dims) : 0; }

extern "C" int mi_block_ctx_kv(const mi_block_weights* wt, const mi_block_dims* dims, const float* ctx, float* kv,
                               uint64_t kv_bytes, void* stream) {
    const char* fn = "mi_block_ctx_kv";
    if (!wt || !dims || !ctx || !kv) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    MI_TRY(check_dims(*dims, fn));
    MI_TRY(check_weights(*wt, *dims, fn));
    if (kv_bytes < ctx_kv_bytes(*dims))
        return fail(MI_ERR_INVALID_ARG, "%s: kv buffer %llu bytes < %llu needed", fn,
                    static_cast<unsigned long long>(kv_bytes), static_cast<unsigned long long>(ctx_kv_bytes(*dims)));
    if (!aligned(kv, 256)) return fail(MI_ERR_ALIGNMENT, "%s: kv buffer must be 256-byte aligned", fn);
    return ctx_kv(*wt, *dims, ctx, kv, reinterpret_cast<char*>(kv) + ctx_kv_bytes(*dims) / 2,
                  static_cast<hipStream_t>(stream));
}

extern "C" int mi_sdxl_block_forward_kv(const mi_block_weights* wt, const mi_block_dims* dims, float* x,
                                        const float* kv, uint64_t kv_bytes, const int32_t* ctx_len, void* workspace,
                                        uint64_t workspace_bytes, void* stream) {
    const char* fn = "mi_sdxl_block_forward_kv";
    if (!wt || !dims || !x || !kv || !workspace) return fail(MI_ERR_INVALID_ARG, "%s: null pointer", fn);
    if (kv_bytes < ctx_kv_bytes(*dims))
        return fail(MI_ERR_INVALID_ARG, "%s: kv buffer %llu bytes < %llu needed", fn,
                    static_cast<unsigned long long>(kv_bytes), static_cast<unsigned long long>(ctx_kv_bytes(*dims)));
    if (!aligned(kv, 256)) return fail(MI_ERR_ALIGNMENT, "%s: kv buffer must be 256-byte aligned", fn);
    return forward(*wt, *dims, x, nullptr, kv, ctx_len, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                   fn);
}
