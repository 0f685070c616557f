/*
 * oracle.h -- CPU restatement of sdvk's Q8_0 GEMM / fused-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in
 * sdvk_amd/csrc. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product library (libmi_sdvk.so) never
 * links, loads or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the sdvk source root).
 *
 * Pinning status of each function is listed in the header of oracle.c.
 */
#ifndef SDVK_ORACLE_H
#define SDVK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types used by the attention restatement */
enum { OR_F32 = 0, OR_F16 = 1 };

/* ---- fp16 <-> fp32 ------------------------------------------------------ */
float or_fp16_to_fp32(uint16_t h);           /* Gguf.cpp:11-35 */
uint16_t or_fp32_to_fp16(float f);           /* IEEE round-to-nearest-even */

/* ---- deterministic input generator (splitmix64 + Box-Muller) ------------- */
void or_fill_normal(uint64_t seed, float mean, float stddev, float* out, uint64_t n);
void or_fill_uniform_int(uint64_t seed, int32_t lo, int32_t hi, int32_t* out, uint64_t n);

/* ---- Q8_0 block format --------------------------------------------------- */
/* 34-byte block {fp16 d little-endian, int8 q[32]}; n = element count, n % 32 == 0 */
void or_q8_0_quantize(const float* w, uint64_t n, uint8_t* blocks);
void or_q8_0_dequant(const uint8_t* blocks, uint64_t n, float* out);
void or_q8_0_to_split(const uint8_t* blocks, uint64_t n, int8_t* payload, float* scales);
void or_q8_split_dequant(const uint32_t* payload, const float* scales, uint64_t n, float* out);

/* ---- Q8 NT GEMM:  C[M,N] (=|+=) A[M,K] . deq(W[N,K])^T (+bias) -------------
 * mode 0 stores (adding bias[n] when bias != NULL), mode 1 accumulates into C
 * without bias. lda == 0 -> K, ldc == 0 -> N. Batch z offsets A by z*sA and C
 * by z*sC; W is shared by every batch item.
 * acc64 != 0 accumulates in double (golden values); otherwise fp32 in k order.
 * threads > 1 parallelises over rows with OpenMP (CPU baseline).            */
void or_gemm_nt_q8_split(const float* A, const uint32_t* payload, const float* scales,
                         const float* bias, float* C, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch,
                         uint64_t sA, uint64_t sC, int acc64, int threads);
void or_gemm_nt_q8_0(const float* A, const uint8_t* blocks, const float* bias, float* C,
                     uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda,
                     uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sC, int acc64,
                     int threads);
/* ---- Q8 NN GEMM:  C[M,N] (=|+=) deq(A[M,K]) . B[K,N] (gemm_nn_q8_v.comp) ---
 * A in the split layout read at flat index z*sA + m*lda + k (scale index =
 * flat >> 5), B fp32 row-major with ldb, no bias. 0 leading dims -> K, N, N. */
void or_gemm_nn_q8_split(const uint32_t* payload, const float* scales, const float* B, float* C, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb, uint32_t ldc,
                         uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC, int acc64, int threads);
/* Output rows rows[0..nrows) of batch item `z` only (parity on sampled rows). */
void or_gemm_nt_q8_0_rows(const float* A, const uint8_t* blocks, const float* bias, float* C,
                          uint32_t M, uint32_t N, uint32_t K, uint32_t lda, uint32_t ldc,
                          const uint32_t* rows, uint32_t nrows, int threads);

/* ---- fused attention ------------------------------------------------------
 * softmax(QK^T / sqrt(hd) + mask) V per head, fp64 online softmax.
 * Q/K/V/O are [T, C] row-major with head h in columns [h*hd, h*hd + hd).   */
void or_fused_attention(const float* q, const float* k, const float* v, float* out,
                        uint32_t Tq, uint32_t Tk, uint32_t C, uint32_t heads, int causal);
/* Batched, strided, fp16/fp32, key-padding. Element strides: ld* between
 * tokens, s* between batch items. kv_len (NULL = all Tk keys) masks keys
 * >= kv_len[b]. Only query rows in rows[0..nrows) are computed when rows is
 * non-NULL (the same row indices in every batch item and head).           */
void or_fused_attention_ex(const void* q, const void* k, const void* v, void* out,
                           uint32_t batch, uint32_t Tq, uint32_t Tk, uint32_t C,
                           uint32_t heads, int causal, uint64_t ldq, uint64_t ldk,
                           uint64_t ldv, uint64_t ldo, uint64_t sq, uint64_t sk, uint64_t sv,
                           uint64_t so, int in_dtype, int out_dtype, const int32_t* kv_len,
                           const uint32_t* rows, uint32_t nrows, int threads);

/* ---- transformer-block glue (layernorm, erf-GELU, GEGLU, add) ------------ */
void or_layernorm(const float* x, const float* gamma, const float* beta, float* y,
                  uint32_t rows, uint32_t d, float eps);
float or_gelu_erf(float v);
void or_geglu(const float* h, float* y, uint32_t rows, uint32_t F);
void or_add(const float* a, const float* b, float* c, uint64_t n);

/* ---- fp32 CPU baseline of attention (blocked online softmax) --------------
 * Same math as the reference tiled shader in fp32; used only for timing.   */
void or_fused_attention_f32(const float* q, const float* k, const float* v, float* out,
                            uint32_t batch, uint32_t Tq, uint32_t Tk, uint32_t C,
                            uint32_t heads, const int32_t* kv_len, uint32_t q_rows,
                            int threads);

int or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
