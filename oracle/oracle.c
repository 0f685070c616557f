/*
 * oracle.c -- CPU restatement of sdvk's Q8_0 GEMM and fused-attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never part of the
 * product. Loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg only.
 *
 * Reference files restated (paths relative to the sdvk source root):
 *   src/Modules/Model/Gguf.cpp:11-35      fp16 decode
 *   src/Modules/Model/Gguf.cpp:83         Q8_0 block = 2 + 32 bytes
 *   src/Modules/Model/Gguf.cpp:514-523    Q8_0 dequant to fp32
 *   src/Modules/Model/Gguf.cpp:559-583    Q8_0 -> split int8 payload + fp32 scale
 *   src/Modules/GPU/shaders/gemm_nt_q8_v.comp:37-43,53-54,115-127   deqB, lda/ldc, epilogue
 *   src/Modules/GPU/shaders/gemm_nn_q8_v.comp:23-28,38-40,54-64,107-108   deqA, ld*, modes
 *   src/Modules/GPU/shaders/fused_attn_tiled.comp, fused_attn.comp   masks, l == 0 guard
 *   tests/fused_attn_test.cpp:25-61       fp64 online-softmax reference
 *   src/Modules/GPU/shaders/layernorm_fwd.comp:15-38, unary_fwd.comp:28-36 (mode 4)
 *   src/Modules/Diffusion/sdvkgen.cpp:533-544 (requant rounding), :1710-1720 (GEGLU)
 *
 * How each function is pinned (tests/test_oracle.py):
 *   or_fp16_to_fp32      exhaustive over all 65536 patterns vs numpy float16
 *   or_fp32_to_fp16      exhaustive-ish sweep vs numpy float16 (RNE, subnormals, inf/nan)
 *   or_q8_0_dequant      known-answer blocks (q in {-128,-127,-1,0,1,127}, d subnormal/
 *                        max/inf/nan) and a numpy restatement on random blocks
 *   or_q8_0_to_split / or_q8_split_dequant   identity with or_q8_0_dequant, byte layout KAT
 *   or_q8_0_quantize     round-trip bound |deq(q(w)) - w| <= d/2 (+fp16 rounding of d), amax -> +-127
 *   or_gemm_nt_q8_*      numpy float64 matmul of the dequantized weight (an independent
 *                        library routine), linearity, mode 1 == C0 + mode 0 without bias,
 *                        bias broadcast, batch with shared W, lda/ldc padding
 *   or_gemm_nn_q8_split  numpy float64 matmul with the flat-index scales, NN(W, B) ==
 *                        NT(B^T, W)^T through the pinned or_gemm_nt_q8_split, mode 1,
 *                        batch offsets of all three operands, lda/ldb/ldc padding, a
 *                        scale block that straddles rows (lda % 32 != 0)
 *   or_fused_attention*  torch/numpy float64 softmax(QK^T s) V (independent library route),
 *                        Tk = 1 -> O = V row, constant scores -> mean of V, causal row 0 = V[0],
 *                        kv_len slicing == unmasked call on the prefix, kv_len = 0 -> O = 0
 *   or_layernorm / or_gelu_erf / or_geglu    numpy float64 closed forms, math.erf
 *   or_fused_attention_f32   vs or_fused_attention (fp64) to 1e-5 relative
 * No function is left "parity unpinned".
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------- fp16 ---- */

/* IEEE binary16 -> binary32 (exact). Same results as Gguf.cpp:11-35: zero,
 * subnormals renormalised, exponent 31 -> inf/nan with the payload shifted. */
float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        /* subnormal: value = m * 2^-24; shift the leading one up to bit 10 */
        int shift = 0;
        while (!(m & 0x400u)) { m <<= 1; ++shift; }
        bits = sign | ((uint32_t)(113 - shift) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u;  /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                        /* below fp16 min normal */
        if (ax < 0x33000000u) return sign;         /* < 2^-25: rounds to zero */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* m * 2^(e-150) in units of 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return sign | (uint16_t)q;
    }
    uint32_t r = ax - 0x38000000u;                 /* rebias exponent 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return sign | (uint16_t)q;
}

/* ------------------------------------------------------------------ rng ---- */

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double u01(uint64_t* s) { return ((double)(splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

void or_fill_normal(uint64_t seed, float mean, float stddev, float* out, uint64_t n) {
    uint64_t s = seed;
    for (uint64_t i = 0; i < n; i += 2) {
        double r = sqrt(-2.0 * log(u01(&s)));
        double t = 6.283185307179586476925 * u01(&s);
        out[i] = (float)(mean + stddev * r * cos(t));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * r * sin(t));
    }
}

void or_fill_uniform_int(uint64_t seed, int32_t lo, int32_t hi, int32_t* out, uint64_t n) {
    uint64_t s = seed;
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)((int64_t)lo + (int64_t)(splitmix64(&s) % span));
}

/* ----------------------------------------------------------------- Q8_0 ---- */

/* Test-input generator. Block scale d = amax/127 stored as fp16 (GGUF Q8_0,
 * Gguf.cpp:83); q = clamp(round-half-away(w * 127/amax), -127, 127), the
 * rounding of the reference's own requantiser (sdvkgen.cpp:533-544). */
void or_q8_0_quantize(const float* w, uint64_t n, uint8_t* blocks) {
    for (uint64_t b = 0; b < n / 32; ++b) {
        const float* x = w + b * 32;
        uint8_t* blk = blocks + b * 34;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
        float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        uint16_t d = or_fp32_to_fp16(amax > 0.0f ? amax / 127.0f : 0.0f);
        blk[0] = (uint8_t)(d & 0xff);
        blk[1] = (uint8_t)(d >> 8);
        for (int i = 0; i < 32; ++i) {
            float t = x[i] * inv;
            int v = (int)(t + (t >= 0.0f ? 0.5f : -0.5f));
            v = v < -127 ? -127 : (v > 127 ? 127 : v);
            blk[2 + i] = (uint8_t)(int8_t)v;
        }
    }
}

static inline float blk_scale(const uint8_t* blk) { return or_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8))); }

/* Gguf.cpp:514-523: out = fp32(d) * q, one fp32 multiply (exact). */
void or_q8_0_dequant(const uint8_t* blocks, uint64_t n, float* out) {
    for (uint64_t b = 0; b < n / 32; ++b) {
        const uint8_t* blk = blocks + b * 34;
        float d = blk_scale(blk);
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* Gguf.cpp:559-583: scales[b] = fp32(d), payload = the 32 int8 in flat order. */
void or_q8_0_to_split(const uint8_t* blocks, uint64_t n, int8_t* payload, float* scales) {
    for (uint64_t b = 0; b < n / 32; ++b) {
        scales[b] = blk_scale(blocks + b * 34);
        memcpy(payload + b * 32, blocks + b * 34 + 2, 32);
    }
}

/* gemm_nt_q8_v.comp:37-43 (deqB): byte fl&3 of word fl>>2, sign-extended, times s[fl>>5]. */
static inline float split_weight(const uint32_t* payload, const float* scales, uint64_t fl) {
    uint32_t w = payload[fl >> 2];
    int v = (int)((w >> ((fl & 3u) * 8u)) & 0xffu);
    if (v > 127) v -= 256;
    return (float)v * scales[fl >> 5];
}

void or_q8_split_dequant(const uint32_t* payload, const float* scales, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = split_weight(payload, scales, i);
}

/* ----------------------------------------------------------------- GEMM ---- */

/* Shared GEMM core over a dequantised fp32 weight Wf[N*K].
 * gemm_nt_q8_v.comp:53-54 (lda/ldc defaults), :115-127 (mode 0 store + bias,
 * mode 1 accumulate without bias), z offsets A and C only (:51-52). */
static void gemm_core(const float* A, const float* Wf, const float* bias, float* C, uint32_t M,
                      uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
                      uint32_t batch, uint64_t sA, uint64_t sC, int acc64, int threads) {
    if (lda == 0) lda = K;
    if (ldc == 0) ldc = N;
    long long total = (long long)batch * M;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads > 0 ? threads : 1)
#endif
    for (long long zm = 0; zm < total; ++zm) {
        uint32_t z = (uint32_t)(zm / M), m = (uint32_t)(zm % M);
        const float* a = A + (uint64_t)z * sA + (uint64_t)m * lda;
        float* c = C + (uint64_t)z * sC + (uint64_t)m * ldc;
        for (uint32_t n = 0; n < N; ++n) {
            const float* w = Wf + (uint64_t)n * K;
            float v;
            if (acc64) {
                double acc = 0.0;
                for (uint32_t k = 0; k < K; ++k) acc += (double)a[k] * (double)w[k];
                v = (float)acc;
            } else {
                /* fp32, eight interleaved partial sums (vectorisable) */
                float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                uint32_t k = 0;
                for (; k + 8 <= K; k += 8)
                    for (int j = 0; j < 8; ++j) p[j] += a[k + j] * w[k + j];
                for (; k < K; ++k) p[k & 7] += a[k] * w[k];
                v = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            }
            if (mode == 0) c[n] = bias ? v + bias[n] : v;
            else c[n] += v;
        }
    }
}

void or_gemm_nt_q8_split(const float* A, const uint32_t* payload, const float* scales,
                         const float* bias, float* C, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch,
                         uint64_t sA, uint64_t sC, int acc64, int threads) {
    float* Wf = (float*)malloc((size_t)N * K * sizeof(float));
    if (!Wf) return;
    or_q8_split_dequant(payload, scales, (uint64_t)N * K, Wf);
    gemm_core(A, Wf, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC, acc64, threads);
    free(Wf);
}

/* Row r's blocks start at byte r*(K/32)*34 (flat GGUF order, K % 32 == 0). */
void or_gemm_nt_q8_0(const float* A, const uint8_t* blocks, const float* bias, float* C,
                     uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda,
                     uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sC, int acc64,
                     int threads) {
    float* Wf = (float*)malloc((size_t)N * K * sizeof(float));
    if (!Wf) return;
    or_q8_0_dequant(blocks, (uint64_t)N * K, Wf);
    gemm_core(A, Wf, bias, C, M, N, K, mode, lda, ldc, batch, sA, sC, acc64, threads);
    free(Wf);
}

void or_gemm_nt_q8_0_rows(const float* A, const uint8_t* blocks, const float* bias, float* C,
                          uint32_t M, uint32_t N, uint32_t K, uint32_t lda, uint32_t ldc,
                          const uint32_t* rows, uint32_t nrows, int threads) {
    (void)M;
    if (lda == 0) lda = K;
    if (ldc == 0) ldc = N;
    float* Wf = (float*)malloc((size_t)N * K * sizeof(float));
    if (!Wf) return;
    or_q8_0_dequant(blocks, (uint64_t)N * K, Wf);
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (long long i = 0; i < (long long)nrows; ++i) {
        const float* a = A + (uint64_t)rows[i] * lda;
        float* c = C + (uint64_t)i * ldc;
        for (uint32_t n = 0; n < N; ++n) {
            const float* w = Wf + (uint64_t)n * K;
            double acc = 0.0;
            for (uint32_t k = 0; k < K; ++k) acc += (double)a[k] * (double)w[k];
            c[n] = (float)acc + (bias ? bias[n] : 0.0f);
        }
    }
    free(Wf);
}

/* gemm_nn_q8_v.comp:30-111 (the weights-left GEMM of the conv / 1x1 paths,
 * sdvkgen.cpp:944-948,1133-1180): C[M,N] (=|+=) A[M,K] . B[K,N] with A the
 * split Q8 layout read at flat index fl = z*sA + m*lda + k, value
 * int8(payload byte fl) * scales[fl >> 5] (:23-28,54-64), B fp32 at
 * z*sB + k*ldb + n, C at z*sC + m*ldc + n; lda = 0 -> K, ldb = 0 -> N,
 * ldc = 0 -> N (:38-40); mode 1 accumulates (:107-108); no bias. The shader's
 * 4-wide staging zero-fills a last partial group when K % 4 or N % 4 != 0
 * (:58,79); this restates the plain product, which the shader equals for
 * K % 4 == 0 and N % 4 == 0 (the only shapes the HIP entry accepts). */
void or_gemm_nn_q8_split(const uint32_t* payload, const float* scales, const float* B, float* C, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb, uint32_t ldc,
                         uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC, int acc64, int threads) {
    if (lda == 0) lda = K;
    if (ldb == 0) ldb = N;
    if (ldc == 0) ldc = N;
    const int8_t* q = (const int8_t*)payload;
    for (uint32_t z = 0; z < batch; ++z) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
#endif
        for (long long mm = 0; mm < (long long)M; ++mm) {
            const uint32_t m = (uint32_t)mm;
            const uint64_t arow = z * sA + (uint64_t)m * lda;
            float* c = C + z * sC + (uint64_t)m * ldc;
            double* acc = (double*)calloc(N, sizeof(double));
            float* accf = (float*)calloc(N, sizeof(float));
            if (!acc || !accf) {
                free(acc);
                free(accf);
                continue;
            }
            for (uint32_t k = 0; k < K; ++k) {
                const uint64_t fl = arow + k;
                const float a = (float)q[fl] * scales[fl >> 5];
                const float* b = B + z * sB + (uint64_t)k * ldb;
                if (acc64) {
                    for (uint32_t n = 0; n < N; ++n) acc[n] += (double)a * (double)b[n];
                } else {
                    for (uint32_t n = 0; n < N; ++n) accf[n] += a * b[n];
                }
            }
            for (uint32_t n = 0; n < N; ++n) {
                const float v = acc64 ? (float)acc[n] : accf[n];
                if (mode == 0) c[n] = v;
                else c[n] += v;
            }
            free(acc);
            free(accf);
        }
    }
}

/* ------------------------------------------------------------ attention ---- */

static inline double load_el(const void* p, uint64_t i, int dt) {
    if (dt == OR_F16) return (double)or_fp16_to_fp32(((const uint16_t*)p)[i]);
    return (double)((const float*)p)[i];
}

static inline void store_el(void* p, uint64_t i, double v, int dt) {
    if (dt == OR_F16) ((uint16_t*)p)[i] = or_fp32_to_fp16((float)v);
    else ((float*)p)[i] = (float)v;
}

/* tests/fused_attn_test.cpp:25-61: fp64 online softmax over the unmasked keys,
 * scale = fp32 1/sqrt(hd) (fused_attn.cpp:55), O = acc / l or 0 when l == 0
 * (fused_attn_tiled.comp:189). Causal masks keys > query
 * (fused_attn.comp:103); kv_len masks keys >= kv_len[b] (batch extension:
 * identical to calling the reference with Tk = kv_len[b] on the prefix). */
void or_fused_attention_ex(const void* q, const void* k, const void* v, void* out,
                           uint32_t batch, uint32_t Tq, uint32_t Tk, uint32_t C,
                           uint32_t heads, int causal, uint64_t ldq, uint64_t ldk,
                           uint64_t ldv, uint64_t ldo, uint64_t sq, uint64_t sk, uint64_t sv,
                           uint64_t so, int in_dtype, int out_dtype, const int32_t* kv_len,
                           const uint32_t* rows, uint32_t nrows, int threads) {
    uint32_t hd = C / heads;
    float scale = 1.0f / sqrtf((float)hd);
    uint32_t nr = rows ? nrows : Tq;
    long long total = (long long)batch * heads * nr;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 8) num_threads(threads > 0 ? threads : 1)
#endif
    for (long long it = 0; it < total; ++it) {
        uint32_t ri = (uint32_t)(it % nr);
        uint32_t h = (uint32_t)((it / nr) % heads);
        uint32_t b = (uint32_t)(it / ((long long)nr * heads));
        uint32_t tq = rows ? rows[ri] : ri;
        uint32_t L = Tk;
        if (kv_len) {
            int32_t l = kv_len[b];
            L = l < 0 ? 0 : ((uint32_t)l < Tk ? (uint32_t)l : Tk);
        }
        double acc[64];
        double qv[64];
        for (uint32_t d = 0; d < hd; ++d) {
            acc[d] = 0.0;
            qv[d] = load_el(q, (uint64_t)b * sq + (uint64_t)tq * ldq + (uint64_t)h * hd + d, in_dtype);
        }
        double m = -INFINITY, l = 0.0;
        for (uint32_t tk = 0; tk < L; ++tk) {
            if (causal && tk > tq) continue;
            uint64_t kb = (uint64_t)b * sk + (uint64_t)tk * ldk + (uint64_t)h * hd;
            uint64_t vb = (uint64_t)b * sv + (uint64_t)tk * ldv + (uint64_t)h * hd;
            double dot = 0.0;
            for (uint32_t d = 0; d < hd; ++d) dot += qv[d] * load_el(k, kb + d, in_dtype);
            double s = dot * (double)scale;
            double mNew = s > m ? s : m;
            double resc = (m == -INFINITY) ? 0.0 : exp(m - mNew);
            l *= resc;
            for (uint32_t d = 0; d < hd; ++d) acc[d] *= resc;
            double p = exp(s - mNew);
            l += p;
            for (uint32_t d = 0; d < hd; ++d) acc[d] += p * load_el(v, vb + d, in_dtype);
            m = mNew;
        }
        double inv = l > 0.0 ? 1.0 / l : 0.0;
        uint64_t ob = (uint64_t)b * so + (uint64_t)(rows ? ri : tq) * ldo + (uint64_t)h * hd;
        for (uint32_t d = 0; d < hd; ++d) store_el(out, ob + d, acc[d] * inv, out_dtype);
    }
}

void or_fused_attention(const float* q, const float* k, const float* v, float* out,
                        uint32_t Tq, uint32_t Tk, uint32_t C, uint32_t heads, int causal) {
    or_fused_attention_ex(q, k, v, out, 1, Tq, Tk, C, heads, causal, C, C, C, C, 0, 0, 0, 0,
                          OR_F32, OR_F32, NULL, NULL, 0, 1);
}

/* fp32 blocked online softmax (fused_attn_tiled.comp structure: 64-key tiles,
 * running max/sum per query, exp2 with log2e folded in). Timing baseline.
 * Processes query rows [0, q_rows) of every batch item and head. */
void or_fused_attention_f32(const float* q, const float* k, const float* v, float* out,
                            uint32_t batch, uint32_t Tq, uint32_t Tk, uint32_t C,
                            uint32_t heads, const int32_t* kv_len, uint32_t q_rows,
                            int threads) {
    const uint32_t hd = C / heads;
    const float c = (1.0f / sqrtf((float)hd)) * 1.4426950408889634f;
    if (q_rows > Tq) q_rows = Tq;
    const uint32_t QB = 16;
    uint32_t nqb = (q_rows + QB - 1) / QB;
    long long total = (long long)batch * heads * nqb;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (long long it = 0; it < total; ++it) {
        uint32_t qb = (uint32_t)(it % nqb);
        uint32_t h = (uint32_t)((it / nqb) % heads);
        uint32_t b = (uint32_t)(it / ((long long)nqb * heads));
        uint32_t L = kv_len ? (uint32_t)kv_len[b] : Tk;
        if (L > Tk) L = Tk;
        uint32_t q0 = qb * QB, nq = q_rows - q0 < QB ? q_rows - q0 : QB;
        float acc[16][64], mrun[16], lrun[16], s[16][64];
        for (uint32_t i = 0; i < nq; ++i) {
            mrun[i] = -1e30f;
            lrun[i] = 0.0f;
            for (uint32_t d = 0; d < hd; ++d) acc[i][d] = 0.0f;
        }
        const float* qbase = q + ((uint64_t)b * Tq) * C + (uint64_t)h * hd;
        const float* kbase = k + ((uint64_t)b * Tk) * C + (uint64_t)h * hd;
        const float* vbase = v + ((uint64_t)b * Tk) * C + (uint64_t)h * hd;
        for (uint32_t kv0 = 0; kv0 < L; kv0 += 64) {
            uint32_t nk = L - kv0 < 64 ? L - kv0 : 64;
            for (uint32_t i = 0; i < nq; ++i) {
                const float* qr = qbase + (uint64_t)(q0 + i) * C;
                float mx = -1e30f;
                for (uint32_t j = 0; j < nk; ++j) {
                    const float* kr = kbase + (uint64_t)(kv0 + j) * C;
                    float dot = 0.0f;
                    for (uint32_t d = 0; d < hd; ++d) dot += qr[d] * kr[d];
                    s[i][j] = dot * c;
                    mx = s[i][j] > mx ? s[i][j] : mx;
                }
                float mnew = mrun[i] > mx ? mrun[i] : mx;
                float resc = exp2f(mrun[i] - mnew);
                lrun[i] *= resc;
                for (uint32_t d = 0; d < hd; ++d) acc[i][d] *= resc;
                for (uint32_t j = 0; j < nk; ++j) {
                    float p = exp2f(s[i][j] - mnew);
                    lrun[i] += p;
                    const float* vr = vbase + (uint64_t)(kv0 + j) * C;
                    for (uint32_t d = 0; d < hd; ++d) acc[i][d] += p * vr[d];
                }
                mrun[i] = mnew;
            }
        }
        for (uint32_t i = 0; i < nq; ++i) {
            float inv = lrun[i] > 0.0f ? 1.0f / lrun[i] : 0.0f;
            float* orow = out + ((uint64_t)b * Tq + q0 + i) * C + (uint64_t)h * hd;
            for (uint32_t d = 0; d < hd; ++d) orow[d] = acc[i][d] * inv;
        }
    }
}

/* ------------------------------------------------------------------ glue ---- */

/* layernorm_fwd.comp:15-38: two-pass mean / variance in fp32, eps inside sqrt. */
void or_layernorm(const float* x, const float* gamma, const float* beta, float* y,
                  uint32_t rows, uint32_t d, float eps) {
    for (uint32_t r = 0; r < rows; ++r) {
        const float* xr = x + (uint64_t)r * d;
        float* yr = y + (uint64_t)r * d;
        double s = 0.0;
        for (uint32_t j = 0; j < d; ++j) s += xr[j];
        float mean = (float)(s / d);
        double ss = 0.0;
        for (uint32_t j = 0; j < d; ++j) { double t = xr[j] - mean; ss += t * t; }
        float var = (float)(ss / d);
        float inv = 1.0f / sqrtf(var + eps);
        for (uint32_t j = 0; j < d; ++j) {
            float t = (xr[j] - mean) * inv;
            yr[j] = gamma ? t * gamma[j] + (beta ? beta[j] : 0.0f) : t;
        }
    }
}

/* unary_fwd.comp:28-36 (mode 4): 0.5 x (1 + erf(x / sqrt 2)), erf from
 * Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7). */
float or_gelu_erf(float v) {
    float xs = v * 0.70710678118654752440f;
    float ax = fabsf(xs);
    float t = 1.0f / (1.0f + 0.3275911f * ax);
    float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
                  0.254829592f) * t;
    float e = 1.0f - poly * expf(-ax * ax);
    float erf = xs >= 0.0f ? e : -e;
    return 0.5f * v * (1.0f + erf);
}

/* sdvkgen.cpp:1710-1720: h = [rows, 2F]; y = h[:, :F] * gelu(h[:, F:]). */
void or_geglu(const float* h, float* y, uint32_t rows, uint32_t F) {
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t j = 0; j < F; ++j)
            y[(uint64_t)r * F + j] = h[(uint64_t)r * 2 * F + j] * or_gelu_erf(h[(uint64_t)r * 2 * F + F + j]);
}

void or_add(const float* a, const float* b, float* c, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) c[i] = a[i] + b[i];
}
