/*
 * mi_sdvk.h -- C-ABI of the MI355X (gfx950) Q8_0 GEMM and fused-attention
 * kernels. Drop-in for the two hot operators of sdvk's SDXL UNet.
 *
 * Contract shared by every entry point:
 *   - Pointers are device pointers (hipMalloc'd or offsets into one); the
 *     caller owns every buffer, the library allocates nothing.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the legacy default
 *     stream) and is asynchronous: results are valid after the stream syncs.
 *   - The return value is an mi_status (0 = MI_OK). Nothing is printed, no
 *     entry point exits the process and no C++ exception crosses the ABI
 *     (the reference's exit(1) paths -- fused_attn.cpp:41-44,
 *     vk_engine.cpp:1147-1150 -- become MI_ERR_UNSUPPORTED / _INVALID_ARG).
 *   - mi_last_error() gives a human-readable reason for the calling thread's
 *     last non-OK status.
 *   - Entry points are reentrant; calls on one stream execute in order, so
 *     the reference's single in-order command buffer needs no barriers here.
 *   - Strides and leading dimensions are in ELEMENTS of the tensor's type.
 *
 * Reference interfaces replaced (paths relative to the sdvk source root):
 *   Engine::dispatch("gemm_nt_q8_v*"/"gemm_nt_q8", {A,Bq,C,S[,bias]}, Pg, ...)
 *       src/Modules/GPU/vk_engine.cpp:1143-1180, KERNELS[] :55-63,
 *       push layout Pg src/Modules/Diffusion/sdvkgen.cpp:901-903
 *   gemmNtQ8 / gemmNtQ8Bias      src/Modules/Diffusion/sdvkgen.cpp:917-936
 *   fusedAttnSupported / fusedAttention / FusedAttnArgs
 *       src/Modules/GPU/fused_attn.hpp:13-28, fused_attn.cpp:34-61
 *   Q8_0 decode (readFloat / readQ8Into) src/Modules/Model/Gguf.cpp:514-583
 *   GgufFile (open / tensors / find / meta / readRaw / readFloat / readQ8Into)
 *       src/Modules/Model/Gguf.hpp:90-140, Gguf.cpp:290-583; weight upload
 *       loadGgufUnet and ggdims src/Modules/Diffusion/sdvkgen.cpp:151-176,549-611
 */
#ifndef MI_SDVK_H
#define MI_SDVK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mi_status {
    MI_OK = 0,
    MI_ERR_INVALID_ARG = 1,  /* null pointer, bad mode / dtype, size overflow */
    MI_ERR_UNSUPPORTED = 2,  /* shape the kernels do not serve (head dim > 64, K % 32 != 0, ...) */
    MI_ERR_ALIGNMENT = 3,    /* pointer or leading-dimension alignment not met */
    MI_ERR_ALIASING = 4,     /* output overlaps an input */
    MI_ERR_HIP = 5,          /* HIP runtime error (launch failure, no device) */
    MI_ERR_IO = 6,           /* file cannot be opened / mapped, or is not a valid GGUF container */
    MI_ERR_NOT_FOUND = 7,    /* no tensor / metadata key of that name, tensor index out of range */
} mi_status;

typedef enum mi_dtype {
    MI_F32 = 0,
    MI_F16 = 1,
} mi_dtype;

/* ---------------------------------------------------------------- misc -- */

/* Text for a status code (static storage). */
const char* mi_status_string(int status);
/* Detail for the calling thread's last non-OK status ("" if none). */
const char* mi_last_error(void);
/* Library version: major * 10000 + minor * 100 + patch. */
int mi_version(void);

/* Plan overrides (extension, no reference counterpart): for tuning sweeps and
 * tests that pin one kernel plan. Process-wide; the library never reads the
 * environment. An override picks tiles, K splits or workgroup sizes only, so
 * results stay within the operators' documented error (a different plan can
 * change the summation order, never the arithmetic). value NULL or "" clears.
 *   "gemm_cfg"          "<build 0..6>[:<K splits>]" (Q8 NT GEMM tile build;
 *                       the splits apply to the workspace entries)
 *   "nn_kernel"         "general": the NN GEMM's untiled kernel for every shape
 *   "nn_splits"         "<1..64>": NN GEMM K splits (workspace entry)
 *   "attn_nw"           "2" | "4": fp16 attention waves per workgroup
 *   "attn_split"        "<rest>[:<pieces>]": key-split plan of
 *                       mi_fused_attention_ws ("0": never split)
 *   "attn_direct_store" "1": attention outputs stored from the MFMA layout
 *                       instead of whole rows through LDS
 *   "attn_simd_waves"   "2" | "3": fp16 attention build of 2 or 3 waves per
 *                       SIMD (fp16-precision, non-causal, 4-wave launches)
 * MI_ERR_INVALID_ARG for an unknown name or a malformed value. Not
 * synchronised with calls in flight on other threads.                      */
int mi_tuning_set(const char* name, const char* value);
/* Clears every override.                                                   */
void mi_tuning_reset(void);

/* ------------------------------------------------------------ Q8_0 format --
 * GGUF Q8_0 block: 34 bytes {fp16 d (little-endian), int8 q[32]}; element i of
 * a tensor lives in block i/32 (flat GGUF order, Gguf.cpp:83, :514-523).
 *
 * mi_q8_0_dequant: out[i] = fp32(d) * q (bit-exact with Gguf.cpp:514-523) when
 *   out_dtype == MI_F32; fp16 round-to-nearest-even of that product when
 *   MI_F16. n % 32 == 0. blocks: 2-byte aligned; out: 16-byte aligned.
 * Replaces GgufFile::readFloat's Q8_0 branch (Gguf.cpp:514-523).          */
int mi_q8_0_dequant(const void* blocks, void* out, int out_dtype, uint64_t n, void* stream);

/* The reference's split device layout (Gguf.cpp:559-583, sdvkgen.cpp:560-586):
 * payload = int8 values packed 4 per uint32 little-endian in flat order,
 * scales = fp32, one per 32 flat elements. out[i] = q[i] * scales[i >> 5]
 * (gemm_nt_q8_v.comp:37-43 deqB). n % 4 == 0; payload and scales 4-byte
 * aligned, out 16-byte aligned.                                            */
int mi_q8_split_dequant(const uint32_t* payload, const float* scales, void* out, int out_dtype,
                        uint64_t n, void* stream);

/* Device-side repack of 34-byte blocks into the split layout (readQ8Into,
 * Gguf.cpp:559-583: scales[b] = fp32(d_b), payload = q in flat order).
 * n % 32 == 0; payload 4-byte aligned, scales 4-byte aligned.             */
int mi_q8_0_to_split(const void* blocks, uint32_t* payload, float* scales, uint64_t n,
                     void* stream);

/* Quantizer with the reference's requantization rule (sdvkgen.cpp:533-544):
 * per block of 32, d = fp16(amax / 127), q = clamp(trunc(w * 127 / amax
 * +- 0.5), -127, 127), all-zero blocks -> d = 0, q = 0. w: fp32, 4-byte
 * aligned, n % 32 == 0; blocks: 34-byte entries, 2-byte aligned.           */
int mi_q8_0_quantize(const float* w, void* blocks, uint64_t n, void* stream);

/* ---------------------------------------------------------------- GEMM -- *
 * C[M,N] (=|+=) A[M,K] . deq(W[N,K])^T (+ bias[N])
 *   A      fp32 row-major, row stride lda (0 -> K), batch stride sA
 *   C      fp32 row-major, row stride ldc (0 -> N), batch stride sC
 *   mode 0 stores acc (+ bias[n] when bias != NULL); mode 1 adds acc to C and
 *          ignores bias (gemm_nt_q8_v.comp:115-127); mode 2 (no reference
 *          counterpart: a residual add fused into the GEMM, replacing the
 *          linear + add2 pair of sdvkgen.cpp:1746,1751,1762) adds acc + bias[n]
 *   batch  grid z: item z reads A + z*sA and writes C + z*sC; W (and bias)
 *          are shared by every item (the reference never offsets B)
 * Arithmetic: A is rounded to fp16, the weight d*q is rounded to fp16, the
 * products are summed in fp32 by the gfx950 MFMA units; accuracy vs the
 * reference's fp32 shader is max|err| <= 2e-3 x RMS(C) at the SDXL shapes.
 * Activations must lie within the fp16 range (|a| < 65504): a larger |a| rounds
 * to an infinite fp16 operand and its output row becomes inf / NaN.
 * Alignment: A 16-byte aligned with lda % 4 == 0 and sA % 4 == 0; C 4-byte
 * aligned. C must not overlap A, W or bias.
 * Returns MI_OK for M == 0 || N == 0 (nothing to do); K == 0 stores bias/0.
 * Determinism: every entry sums in a fixed order, so a call repeats bit for
 * bit. The entries without a workspace never split K, and every such call
 * gives the same bits whatever tile build runs it. The *_ws entries may split
 * K into the caller's workspace (partials summed in split order by a second
 * kernel): bit-identical from run to run, but grouped differently from the
 * unsplit sum (last-bit differences from the entry without a workspace).
 */

/* North-star entry: W is the raw GGUF stream of 34-byte Q8_0 blocks, row n's
 * K/32 blocks starting at byte n*(K/32)*34. K % 32 == 0 (else
 * MI_ERR_UNSUPPORTED). W must be 16-byte aligned; it is read in aligned
 * 16-byte pieces, none of which extends past the 16-byte-aligned end of W.
 * No reference counterpart consumes blocks directly; it replaces the
 * load-time split (Gguf.cpp:559-583) + gemm_nt_q8_v dispatch pair.        */
int mi_gemm_nt_q8_0(const float* A, const void* W, const float* bias, float* C, uint32_t M,
                    uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
                    uint32_t batch, uint64_t sA, uint64_t sC, void* stream);

/* Workspace variants (no reference counterpart: the reference never splits K;
 * the reference caller's step arena, sdvkgen.cpp:1080, is where such scratch
 * lives). Grids too small to fill the GPU split K when `workspace` (device
 * memory, 16-byte aligned, disjoint from every operand, caller-owned, used only
 * in stream order) holds mi_gemm_nt_q8_workspace_bytes(M, N, K, batch) bytes;
 * with less (or NULL) they run exactly as the entries without a workspace.
 * Calls sharing a workspace must be ordered (same stream). */
uint64_t mi_gemm_nt_q8_workspace_bytes(uint32_t M, uint32_t N, uint32_t K, uint32_t batch);
int mi_gemm_nt_q8_0_ws(const float* A, const void* W, const float* bias, float* C, uint32_t M,
                       uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
                       uint32_t batch, uint64_t sA, uint64_t sC, void* workspace,
                       uint64_t workspace_bytes, void* stream);

/* No-allocation variant of mi_gemm_nt_q8_0_ws (no counterpart in the
 * reference). For callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc. Same
 * arguments, semantics and results (bit for bit) as mi_gemm_nt_q8_0_ws given a
 * workspace of mi_gemm_nt_q8_workspace_bytes(M, N, K, batch) bytes, but the
 * K-split partials go to a scratch array inside the library, one per GPU,
 * of MI_GEMM_NOALLOC_SCRATCH_BYTES, held until the process ends. A shape whose
 * plan needs more scratch than that returns MI_ERR_UNSUPPORTED (no shape does
 * under the built-in tile rules: they split only grids of fewer than 256
 * 128 x 128 tiles, into at most 512 / tiles parts, or fewer than 512 64 x 64
 * tiles into about 256 workgroups, at most 32 MiB of partials). Calls on one GPU share
 * the scratch: calls that overlap on one GPU (unordered streams) race, so
 * order them (one stream). Calls no hipMalloc / hipFree. The scratch's device
 * address is looked up once per GPU (hipGetSymbolAddress, which may load the
 * code object there): by mi_gemm_noalloc_init, or else by the first call on
 * that GPU. A caller that captures the entry into a HIP graph calls
 * mi_gemm_noalloc_init on the GPU before capturing; a first call made inside
 * a capture without it returns MI_ERR_UNSUPPORTED and records nothing.      */
#define MI_GEMM_NOALLOC_SCRATCH_BYTES (32ull << 20)
int mi_gemm_nt_q8_0_noalloc(const float* A, const void* W, const float* bias, float* C, uint32_t M,
                            uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
                            uint32_t batch, uint64_t sA, uint64_t sC, void* stream);
/* Looks up the current GPU's scratch address for mi_gemm_nt_q8_0_noalloc
 * (no counterpart in the reference; for the same callers). Idempotent.      */
int mi_gemm_noalloc_init(void);

/* Reference device layout: payload (int8 x4 per uint32, flat [N,K] order) +
 * fp32 scale per 32 flat elements (any fp32 value: LoRA requantisation writes
 * non-fp16 scales, sdvkgen.cpp:536-538). Any K, like the reference's scalar
 * gemm_nt_q8 (gemm_nt_q8.comp:52-80): shapes with K % 4 != 0, lda or sA not a
 * multiple of 4, or A not 16-byte aligned run on an untiled kernel that
 * stages element by element (A 4-byte aligned). (The reference's vectorised
 * gemm_nt_q8_v zero-fills a partial 4-group instead, gemm_nt_q8_v.comp:69,86;
 * that quirk is not reproduced.)
 * Replaces Engine::dispatch("gemm_nt_q8_v[_bm128][_b]" / "gemm_nt_q8",
 * {A, Bq, C, S[, bias]}, Pg{M,N,K,mode,sA,0,sC,batch,lda,0,ldc,0})
 * (vk_engine.cpp:55-63, sdvkgen.cpp:917-936, tests/gemm_q8_bench.cpp:32-38). */
int mi_gemm_nt_q8_split(const float* A, const uint32_t* payload, const float* scales,
                        const float* bias, float* C, uint32_t M, uint32_t N, uint32_t K,
                        uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA,
                        uint64_t sC, void* stream);
/* Workspace variant of mi_gemm_nt_q8_split (as mi_gemm_nt_q8_0_ws). */
int mi_gemm_nt_q8_split_ws(const float* A, const uint32_t* payload, const float* scales,
                           const float* bias, float* C, uint32_t M, uint32_t N, uint32_t K,
                           uint32_t mode, uint32_t lda, uint32_t ldc, uint32_t batch, uint64_t sA,
                           uint64_t sC, void* workspace, uint64_t workspace_bytes, void* stream);

/* GEGLU fused into the FF-up projection: W holds 2F Q8_0 rows (GEGLU's value
 * rows 0..F-1, then its gate rows F..2F-1: the proj layout of diffusers'
 * GEGLU), bias 2F floats or NULL, and
 *   G[m, j] = (A.W[j]^T + bias[j]) * gelu(A.W[F + j]^T + bias[F + j])
 * with the erf GELU of unary_fwd.comp:28-36, for j < F; G row stride ldg
 * (0 -> F). Replaces linear(ff_up) + geglu (sdvkgen.cpp:1709-1720): the
 * [M, 2F] intermediate never reaches memory. K % 32 == 0, K > 0; alignment
 * as mi_gemm_nt_q8_0; G must not overlap A, W or bias.                      */
int mi_gemm_nt_q8_0_geglu(const float* A, const void* W, const float* bias, float* G, uint32_t M,
                          uint32_t F, uint32_t K, uint32_t lda, uint32_t ldg, void* stream);

/* fp16 activations (extension, no reference counterpart: the reference keeps
 * fp32 activations, sdvkgen.cpp:917-936). A holds IEEE binary16 values
 * (uint16_t bits), 16-byte aligned, lda and sA multiples of 8. The GEMM
 * rounds an fp32 A to fp16 when staging it, so a producer that stores fp16
 * (the same RNE rounding of the same fp32 value) gives the fp32 entries'
 * results bit for bit while moving half the bytes -- the config-4 block's
 * LayerNorm, attention and GEGLU outputs, which only feed GEMMs.
 * mi_gemm_nt_q8_0_f16a: mi_gemm_nt_q8_0_ws with fp16 A (workspace NULL: no
 * K split). mi_gemm_nt_q8_0_geglu_f16: mi_gemm_nt_q8_0_geglu with fp16 A and
 * G stored as fp16 (the fp32 result rounded once, RNE; G 8-byte aligned).  */
int mi_gemm_nt_q8_0_f16a(const void* A, const void* W, const float* bias, float* C, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldc,
                         uint32_t batch, uint64_t sA, uint64_t sC, void* workspace,
                         uint64_t workspace_bytes, void* stream);
int mi_gemm_nt_q8_0_geglu_f16(const void* A, const void* W, const float* bias, void* G, uint32_t M,
                              uint32_t F, uint32_t K, uint32_t lda, uint32_t ldg, void* stream);

/* fp16 output (extension, no counterpart in the reference; for the block's
 * MI_BLOCK_FP16_ATTENTION): C[M,N] = fp16(A . deq(W)^T + bias), the fp32
 * result of the unsplit GEMM rounded once (RNE). A is fp32 or fp16
 * (a_dtype MI_F32 / MI_F16, layout as in mi_gemm_nt_q8_0 / _f16a); C is
 * fp16 with row stride ldc (0 -> N) in elements; mode 0, batch 1, no K
 * split. K a positive multiple of 32, W 16-byte aligned, C 2-byte aligned
 * (8-byte aligned with ldc % 4 == 0 for the vector stores).                  */
int mi_gemm_nt_q8_0_f16o(const void* A, uint32_t a_dtype, const void* W, const float* bias, void* C,
                         uint32_t M, uint32_t N, uint32_t K, uint32_t lda, uint32_t ldc, void* stream);

/* Q8 NN GEMM (the conv / 1x1 paths' weights-left product):
 *   C[M,N] (=|+=) deq(A[M,K]) . B[K,N]
 * A in the split layout, read at FLAT index fl = z*sA + m*lda + k: value
 * int8(payload byte fl) * scales[fl >> 5] (gemm_nn_q8_v.comp:23-28,54-64);
 * B fp32 row-major (ldb); mode 0 stores, 1 accumulates, no bias; batch z
 * offsets A by z*sA, B by z*sB, C by z*sC; lda/ldb/ldc == 0 -> K, N, N.
 * K and N must be multiples of 4 (the shader's 4-wide staging zero-fills a
 * partial group, :58,79: rejected, not emulated). payload 4-byte aligned with
 * lda, sA % 4 == 0; B 16-byte aligned with ldb, sB % 4 == 0; each operand
 * below 2 GiB. payload 16-byte aligned with lda, sA % 16 == 0 and
 * K % 64 == 0 (every SDXL conv) take the pipelined tiled kernel; other shapes
 * take the untiled kernel. Sums in a fixed order (results repeat bit for bit).
 * Replaces Engine::dispatch("gemm_nn_q8_v" / "gemm_nn_q8", {Aq, B, C, S}, Pg)
 * (vk_engine.cpp:57,63) behind gemmNnQ8 (sdvkgen.cpp:944-948). */
int mi_gemm_nn_q8_split(const uint32_t* payload, const float* scales, const float* B, float* C,
                        uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb,
                        uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC, void* stream);
/* Workspace variant (no reference counterpart): the tiled kernel splits K when
 * its grid would leave CUs idle and `workspace` holds
 * mi_gemm_nn_q8_workspace_bytes(M, N, K, batch) bytes (16-byte aligned,
 * disjoint from the operands); the partials are summed in split order. */
uint64_t mi_gemm_nn_q8_workspace_bytes(uint32_t M, uint32_t N, uint32_t K, uint32_t batch);
int mi_gemm_nn_q8_split_ws(const uint32_t* payload, const float* scales, const float* B, float* C,
                           uint32_t M, uint32_t N, uint32_t K, uint32_t mode, uint32_t lda, uint32_t ldb,
                           uint32_t ldc, uint32_t batch, uint64_t sA, uint64_t sB, uint64_t sC,
                           void* workspace, uint64_t workspace_bytes, void* stream);

/* ----------------------------------------------------------- attention -- *
 * O = softmax(Q K^T / sqrt(hd) + mask) V per head, hd = C / heads <= 64,
 * never materialising Tq x Tk. Head h occupies columns [h*hd, h*hd + hd) of
 * every token row. Masked keys: key > query when causal (fused_attn.comp:103);
 * key >= kv_len[b] (key padding). A query whose keys are all masked gets
 * O = 0 (fused_attn_tiled.comp:189). Online softmax in fp32; QK^T and PV on
 * fp16 MFMA with fp32 accumulation.                                         */

/* Same predicate as fusedAttnSupported (fused_attn.cpp:34-38): 1 if heads
 * divides C and 1 <= C/heads <= 64, else 0.                                */
int mi_fused_attn_supported(uint32_t C, uint32_t heads);

/* fusedAttention(Engine&, const FusedAttnArgs&) (fused_attn.cpp:40-61):
 * fp32 q/k/v/out [T, C] contiguous, scale 1/sqrt(C/heads).
 * q, k, v, out 16-byte aligned; out must not overlap q, k or v.
 * fp32 output, so MI_ATTN_PREC_AUTO computes P in two fp16 parts (below):
 * max |err| ~1e-5 x RMS, inside the reference test's rel 2e-5.             */
int mi_fused_attention(const float* q, const float* k, const float* v, float* out, uint32_t Tq,
                       uint32_t Tk, uint32_t C, uint32_t heads, int causal, void* stream);

/* Extended form: batch, strides, fp16/fp32 I/O and key-padding lengths.
 * FusedAttnArgs (fused_attn.hpp:13-23) plus the batch / dtype / kv_len
 * extensions the SDXL configs need.                                         */
typedef struct mi_attn_args {
    const void* q;        /* [batch][Tq][ldq] */
    const void* k;        /* [batch][Tk][ldk] */
    const void* v;        /* [batch][Tk][ldv] */
    void* out;            /* [batch][Tq][ldo] */
    uint32_t batch;       /* >= 1 */
    uint32_t Tq, Tk, C, heads;
    int32_t causal;
    int32_t in_dtype;     /* mi_dtype of q, k, v */
    int32_t out_dtype;    /* mi_dtype of out */
    uint64_t ldq, ldk, ldv, ldo;   /* token stride, 0 -> C; ldq, ldk, ldv < 2^22 elements */
    uint64_t sq, sk, sv, so;       /* batch stride, 0 -> T * ld */
    const int32_t* kv_len;         /* device int32[batch] or NULL (all Tk keys) */
    float scale;                   /* 0 -> 1/sqrt(C/heads) (fused_attn.cpp:55) */
    int32_t precision;             /* mi_attn_precision (extension; 0 = MI_ATTN_PREC_AUTO) */
} mi_attn_args;

/* How the softmax weights P enter the PV product (extension; the reference
 * computes in fp32 throughout, fused_attn_tiled.comp:130-182). The MFMA takes
 * fp16 operands, so P = exp2(s - m) is rounded to fp16 (2^-11 relative):
 *   MI_ATTN_PREC_FP16:  one product with fp16 P (plus P's residual on the
 *                       diagonal tiles of a causal launch). Max |err| vs fp32
 *                       math up to ~2e-3 x RMS(out) on rows whose weight sits
 *                       on a few keys; typically 0.5-1.2e-3.
 *   MI_ATTN_PREC_SPLIT: P as fp16 hi + lo (lo = fp16(P - hi)) in two
 *                       products, P exact to ~2^-22: max |err| 1-5e-6 x RMS,
 *                       about +45% time on long key ranges, +6% on short ones.
 *   MI_ATTN_PREC_AUTO:  SPLIT for fp32 outputs (fp32-grade accuracy, as the
 *                       reference's own test asks of its fp32 kernel,
 *                       tests/fused_attn_test.cpp:118-126), FP16 for fp16
 *                       outputs (whose own storage rounding, 2^-12 |out|, is of
 *                       the same order as P's).                             */
enum mi_attn_precision { MI_ATTN_PREC_AUTO = 0, MI_ATTN_PREC_FP16 = 1, MI_ATTN_PREC_SPLIT = 2 };

int mi_fused_attention_ex(const mi_attn_args* args, void* stream);

/* mi_fused_attention_ex with a caller workspace (extension; the reference
 * launches one dispatch per call). When the fp16 kernel's grid ends in a
 * partial round of query blocks (e.g. 2 x 10 heads x 4096 queries: 640 blocks
 * of 128 queries against 512 resident), the blocks of that round run as
 * several workgroups over consecutive key ranges whose partial results are
 * added, in a fixed order, by a second kernel; the last round then fills the
 * GPU. Only unmasked, non-causal fp16 calls split. mi_fused_attention_ws_bytes
 * gives the bytes the call's plan needs (0: no split); a smaller workspace (or
 * NULL) runs mi_fused_attention_ex's plan. The workspace: 16-byte aligned,
 * disjoint from q, k, v and out; calls sharing one must not overlap in time.
 * Results differ from mi_fused_attention_ex's in the last bits (a different
 * summation order) and repeat bit for bit.                                   */
uint64_t mi_fused_attention_ws_bytes(const mi_attn_args* args);
int mi_fused_attention_ws(const mi_attn_args* args, void* workspace, uint64_t workspace_bytes, void* stream);

/* --------------------------------------------------------- block glue -- *
 * The SDXL transformer block's row / elementwise operators, fp32.          */

/* layernorm (sdvkgen.cpp:1094-1103, layernorm_fwd.comp:15-38): per row of d,
 * y = (x - mean) / sqrt(var + eps) [* gamma + beta], mean and var in two
 * passes. gamma and beta both NULL (no affine) or both set. y may equal x. */
int mi_layernorm(const float* x, const float* gamma, const float* beta, float* y, uint32_t rows,
                 uint32_t d, float eps, void* stream);
/* mi_layernorm with y stored as fp16 (extension): each fp32 result rounded
 * once (RNE), the value a following GEMM would stage from an fp32 y.
 * d % 4 == 0, x and y 16-byte / 8-byte aligned; y must not overlap x.      */
int mi_layernorm_f16(const float* x, const float* gamma, const float* beta, void* y, uint32_t rows,
                     uint32_t d, float eps, void* stream);

/* geglu (sdvkgen.cpp:1709-1720, unary_fwd.comp:28-36): h = [rows, 2F],
 * y[r, j] = h[r, j] * gelu_erf(h[r, F + j]), erf by Abramowitz-Stegun 7.1.26. */
int mi_geglu(const float* h, float* y, uint32_t rows, uint32_t F, void* stream);
/* mi_geglu with y stored as fp16 (extension; the fp32 result rounded once, RNE).
 * F % 4 == 0, h 16-byte and y 8-byte aligned.                               */
int mi_geglu_f16(const float* h, void* y, uint32_t rows, uint32_t F, void* stream);

/* add2 in place (sdvkgen.cpp:1746,1751,1762): x[i] += a[i], i < n.         */
int mi_add_inplace(float* x, const float* a, uint64_t n, void* stream);

/* One SDXL BasicTransformerBlock (diffusers parameter names), in the order of
 * spatialTransformer's inner loop (sdvkgen.cpp:1739-1763) with crossAttention
 * (:1283-1290) and geglu (:1709-1720): LayerNorm -> self-attention -> add ->
 * LayerNorm -> cross-attention on ctx -> add -> LayerNorm -> GEGLU FF -> add.
 * Linear weights are Q8_0 blocks [out, in] (K = in, a multiple of 32);
 * LayerNorm eps = 1e-5 with affine. Rows are batch-stacked: x is
 * [batch * tokens, channels] (updated in place), ctx is
 * [batch * ctx_tokens, ctx_channels]; attention runs per batch item.
 * ctx_len: device int32[batch] key-padding lengths for the cross-attention,
 * or NULL. workspace: device memory of mi_block_workspace_bytes() bytes,
 * 256-byte aligned; nothing is allocated. Calls sharing a workspace must be
 * ordered (same stream).
 * dims.flags (0 = the reference's sequence of separate operators):
 *   MI_BLOCK_FUSED_EPILOGUES: the residual adds run in the out-projection /
 *     FF-down GEMM epilogues (mode 2) and GEGLU in the FF-up epilogue;
 *   MI_BLOCK_JOINT_QKV: attn1_q / attn1_k / attn1_v are the three C x C parts
 *     of one [3C, C] Q8_0 matrix (attn1_k = attn1_q + C*(C/32)*34 bytes,
 *     attn1_v = attn1_k + as much; else MI_ERR_INVALID_ARG), projected by one
 *     GEMM;
 *   MI_BLOCK_FP16_ACTIVATIONS: the tensors whose only consumer is a GEMM --
 *     the LayerNorm outputs, the attention outputs and the GEGLU output --
 *     are stored as fp16 (each fp32 value rounded once, RNE, which is what the
 *     GEMM's A staging does to an fp32 tensor) and read by the fp16-A GEMM:
 *     half the bytes, no conversion in the GEMM;
 *   MI_BLOCK_FP16_ATTENTION: the Q / K / V projections and the cached
 *     context K / V are stored as fp16 (mi_gemm_nt_q8_0_f16o: the fp32 result
 *     rounded once) and both attentions take fp16 inputs, i.e. attention at the
 *     precision of the fp16 attention entries (configs 2 and 3) instead of the
 *     fp32 inputs' hi + lo split. A precision choice, not a layout one: the
 *     block's result differs from the flag-off block's by that rounding.
 * Within one setting of MI_BLOCK_FP16_ATTENTION every combination of the other
 * flags computes the same bits (the block sums in a fixed order, and the
 * GEMMs that differ between the variants never split K).                   */
typedef struct mi_block_weights {
    const float *norm1_w, *norm1_b, *norm2_w, *norm2_b, *norm3_w, *norm3_b; /* [channels] */
    const void *attn1_q, *attn1_k, *attn1_v, *attn1_out;    /* [channels, channels] */
    const float* attn1_out_b;                                /* [channels] or NULL */
    const void* attn2_q;                                     /* [channels, channels] */
    const void *attn2_k, *attn2_v;                           /* [channels, ctx_channels] */
    const void* attn2_out;                                   /* [channels, channels] */
    const float* attn2_out_b;                                /* [channels] or NULL */
    const void* ff_up;                                       /* [2 ff_inner, channels] */
    const float* ff_up_b;                                    /* [2 ff_inner] or NULL */
    const void* ff_down;                                     /* [channels, ff_inner] */
    const float* ff_down_b;                                  /* [channels] or NULL */
} mi_block_weights;

enum { MI_BLOCK_FUSED_EPILOGUES = 1, MI_BLOCK_JOINT_QKV = 2, MI_BLOCK_FP16_ACTIVATIONS = 4, MI_BLOCK_FP16_ATTENTION = 8 };

typedef struct mi_block_dims {
    uint32_t batch, tokens, channels, heads, ctx_tokens, ctx_channels, ff_inner;
    uint32_t flags;       /* MI_BLOCK_* bits */
} mi_block_dims;

uint64_t mi_block_workspace_bytes(const mi_block_dims* dims);
int mi_sdxl_block_forward(const mi_block_weights* w, const mi_block_dims* dims, float* x,
                          const float* ctx, const int32_t* ctx_len, void* workspace,
                          uint64_t workspace_bytes, void* stream);

/* Cross-attention K / V caching. The context is fixed for a sampling job, yet
 * crossAttention projects it with to_k / to_v for every block, guidance pass
 * and step (sdvkgen.cpp:1283-1290; ctx uploaded once at :3659-3667).
 * mi_block_ctx_kv computes K = ctx . attn2_k^T and V = ctx . attn2_v^T once
 * into `kv` (K, then V at byte offset mi_block_ctx_kv_bytes / 2; each
 * [batch * ctx_tokens, channels] fp32, or fp16 when dims->flags has
 * MI_BLOCK_FP16_ATTENTION; 256-byte aligned, caller-owned; the cache must be
 * built and read with the same flag);
 * mi_sdxl_block_forward_kv then runs the block exactly like
 * mi_sdxl_block_forward but reads K / V from `kv` instead of projecting ctx;
 * both project with the same unsplit GEMMs, so cached and fresh results are
 * bit-identical.                                                            */
uint64_t mi_block_ctx_kv_bytes(const mi_block_dims* dims);
int mi_block_ctx_kv(const mi_block_weights* w, const mi_block_dims* dims, const float* ctx, float* kv,
                    uint64_t kv_bytes, void* stream);
int mi_sdxl_block_forward_kv(const mi_block_weights* w, const mi_block_dims* dims, float* x,
                             const float* kv, uint64_t kv_bytes, const int32_t* ctx_len, void* workspace,
                             uint64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- GGUF -- *
 * Checkpoint access: the container reader and the upload of its tensors into
 * caller-owned device buffers in the layouts the GEMM entries read.
 * Replaces ofc::GgufFile (Gguf.hpp:90-140) and the Q8_0 branch of loadGgufUnet
 * (sdvkgen.cpp:549-611). Differences from the common contract above:
 *   - mi_gguf_read_* write HOST memory; mi_gguf_upload_* write device memory
 *     and are stream-ordered like the kernels (the host bytes are consumed
 *     before the call returns, so the file may be closed afterwards);
 *   - a handle owns two 8 MiB pinned HOST staging buffers, allocated on its
 *     first upload and freed by mi_gguf_close (no device memory is allocated);
 *   - one handle must not be used by two threads at once; separate handles
 *     are independent.
 * Parse rules, limits and the readFloat decode follow Gguf.cpp:290-416,489-527
 * (v2/v3, prefix filter + strip, general.alignment, 1..4 dims, F32 / F16 /
 * BF16 / Q4_0 / Q8_0 decode, a partial trailing block decodes to zeros).   */
typedef struct mi_gguf mi_gguf;

typedef struct mi_gguf_tensor_info {
    const char* name;     /* NUL-terminated, owned by the handle (prefix stripped) */
    uint32_t type;        /* ggml type id: 0 F32, 1 F16, 2 Q4_0, 8 Q8_0, 30 BF16, ... */
    uint32_t n_dims;      /* 1..4 */
    uint64_t dims[4];     /* dims[0] fastest-varying (ggml ne[0]); unused dims = 1 */
    uint64_t offset;      /* byte offset in the data section */
    uint64_t nbytes;      /* stored bytes (whole blocks) */
    uint64_t n_elems;
    /* logical (rows, cols) of the weight (ggdims, sdvkgen.cpp:151-176):
     * comfy.gguf.orig_shape.<name> if present, else 1-D (n, 1), 2-D
     * (dims[1], dims[0]), N-D (dims[N-1], product of the rest) */
    uint64_t rows, cols;
} mi_gguf_tensor_info;

typedef struct mi_gguf_meta_info {
    uint32_t type;        /* GGUF value type: 0 u8 .. 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64 */
    uint32_t arr_type;    /* element type of an array */
    uint64_t u;           /* integer scalars (signed ones sign-extended) */
    double f;             /* f32 / f64 scalars */
    int32_t b;            /* bool */
    const char* str;      /* string value (owned by the handle, NUL-terminated) */
    uint64_t str_len;
    uint64_t arr_len;     /* array item count */
} mi_gguf_meta_info;

/* Maps and parses `path`; prefix (or NULL) keeps only tensors named
 * prefix* and strips it (GgufFile::open, Gguf.cpp:290-416). */
int mi_gguf_open(const char* path, const char* prefix, mi_gguf** out);
void mi_gguf_close(mi_gguf* g);
int mi_gguf_info(const mi_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* data_offset,
                 uint64_t* file_size);
int mi_gguf_tensor(const mi_gguf* g, uint64_t index, mi_gguf_tensor_info* info);
int mi_gguf_find(const mi_gguf* g, const char* name, uint64_t* index);
int mi_gguf_meta(const mi_gguf* g, const char* key, mi_gguf_meta_info* info);
/* Items [first, first + count) of an array: integer / bool arrays into u64s,
 * float arrays into f64s, string arrays into strs (pointers owned by the
 * handle); the other outputs may be NULL. */
int mi_gguf_meta_array(const mi_gguf* g, const char* key, uint64_t first, uint64_t count, uint64_t* u64s,
                       double* f64s, const char** strs);
/* Host reads: stored bytes (GgufFile::readRaw), fp32 decode (readFloat), and
 * the split Q8_0 layout int8 payload + fp32 scale per block (readQ8Into). */
int mi_gguf_read_raw(const mi_gguf* g, uint64_t index, void* dst, uint64_t dst_bytes);
int mi_gguf_read_f32(const mi_gguf* g, uint64_t index, float* dst, uint64_t n);
int mi_gguf_read_q8_split(const mi_gguf* g, uint64_t index, int8_t* payload, float* scales);
/* Device uploads. upload_raw copies the stored bytes (a Q8_0 weight lands as
 * the 34-byte blocks mi_gemm_nt_q8_0 reads); upload_f32 the readFloat decode;
 * upload_q8_split the reference's device layout for mi_gemm_nt_q8_split
 * (sdvkgen.cpp:560-582: payload n bytes, scales n / 32 floats). */
int mi_gguf_upload_raw(mi_gguf* g, uint64_t index, void* dst, uint64_t dst_bytes, void* stream);
int mi_gguf_upload_f32(mi_gguf* g, uint64_t index, float* dst, uint64_t n, void* stream);
int mi_gguf_upload_q8_split(mi_gguf* g, uint64_t index, int8_t* payload, float* scales, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MI_SDVK_H */
