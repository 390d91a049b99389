/*
 * libw8a8 -- W8A8 linear engine for MI355X (gfx950): the C ABI.
 *
 * Every entry point takes plain device pointers, element counts / leading dimensions (in
 * elements) and a hipStream_t, enqueues its kernels on that stream and returns a status:
 * 0 (W8A8_OK) or one of W8A8_E*.  On failure nothing was launched and w8a8_last_error()
 * (thread-local) describes why.  The library never allocates device memory, never frees
 * caller memory and never synchronises; results are ready when the stream reaches them.
 * Matrices are row-major.  bf16 data is passed as uint16_t bit patterns.
 *
 * Reference interfaces replaced (AyaSakura-comp/gemma-npu, file:line):
 *   npu_kernels.mm_i8 / matmul_i8_k ........ npu_kernels.py:40-64      -> w8a8_gemm_i32
 *   resident.to_npu(w, static=True) ........ gemma_npu.py:70-75        -> w8a8_pack_weight_kn / _nk
 *   _quant / _quant_rows ................... pipeline.py:49-52, gemma_npu.py:37-42 -> w8a8_quant_rows_*
 *   per-channel weight quant ............... gemma_npu.py:68-69        -> w8a8_quant_rows_f32 / _bf16 on W[N,K]
 *   _deq / _dequant ........................ pipeline.py:55-57, gemma_npu.py:45-47 -> w8a8_dequant_bf16,
 *                                                                         w8a8_gemm_bf16 (epilogue 0)
 *   k_gelu ................................. pipeline.py:102-107       -> w8a8_gemm_bf16 (epilogue 1)
 *   k_post_ff / _rms ....................... pipeline.py:43-46,110-114 -> w8a8_rms_residual_bf16, w8a8_k_post_ff
 *   k_in ................................... pipeline.py:66-69         -> w8a8_k_in
 *   k_qkv (+ _rope) ........................ pipeline.py:60-63, 72-85  -> w8a8_k_qkv
 *   k_attn_out ............................. pipeline.py:88-92         -> w8a8_k_attn_out
 *   k_post_attn ............................ pipeline.py:95-99         -> w8a8_k_post_attn
 *   k_gelu on an int32 result .............. pipeline.py:102-107       -> w8a8_k_gelu
 *   k_ple_gate / k_ple_out ................. pipeline.py:117-127       -> w8a8_k_ple_gate / w8a8_k_ple_out
 *   NPUGemm.matmul (quant->GEMM->dequant) .. gemma_npu.py:117-152      -> w8a8_linear_bf16
 *   cpu_int8_linear / Int8Head ............. gemma_npu.py:155-172      -> w8a8_gemv_bf16,
 *     (torch._weight_int8pack_mm semantics)                               w8a8_gemv_packed_bf16
 *   resident decode weight w_cpu ........... gemma_npu.py:81           -> w8a8_pack_gemv_weight
 *   full_attention / sliding_attention ..... pipeline.py:140-180,      -> w8a8_attention_bf16
 *     (prefill sdpa of local_sdpa)             local_attn.py:71-107
 *   _split_kv_decode / local_sdpa decode ... local_attn.py:44-83       -> w8a8_attention_decode_bf16
 */
#ifndef W8A8_H
#define W8A8_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W8A8_OK 0
#define W8A8_EINVAL 1  /* bad shape, pointer, leading dimension or option */
#define W8A8_EALIGN 2  /* pointer or leading dimension not aligned as required */
#define W8A8_EHIP 3    /* a HIP launch failed */
#define W8A8_ENOTSUP 4 /* valid but unsupported (K % 16 != 0, offsets beyond 32 bits, ...) */

/* Message for the last failing call on this thread ("" if none). */
const char *w8a8_last_error(void);

/* ABI revision of this header (1). */
int w8a8_abi_version(void);

/* ---- resident weights ------------------------------------------------------------------ */

/* Bytes of the packed (MFMA-fragment) weight for N output channels x K inputs.  With
 * interleave = I > 0 the weight is a [gate; up] pair (N == 2*I, I % 32 == 0) whose channels
 * are interleaved in 32-channel tiles for the fused GELU epilogue.  -1 if invalid.
 * Replaces the zero-padded [K, N_pad] resident copy of gemma_npu.py:67-75. */
int64_t w8a8_packed_weight_bytes(int64_t N, int64_t K, int64_t interleave);

/* Pack an int8 weight given in the reference GEMM's B layout, b_kn[K, N] (ld = ldb)
 * (npu_kernels.py:46 B[K,N]; gemma_npu.py:70-71 wt[K, N_pad]).  `packed` is 16-byte aligned,
 * w8a8_packed_weight_bytes(N, K, interleave) long. */
int w8a8_pack_weight_kn(const int8_t *b_kn, int64_t ldb, int64_t K, int64_t N, int64_t interleave,
                        int8_t *packed, hipStream_t stream);

/* Same, from the [N, K] layout (gemma_npu.py:69 q, :81 w_cpu). */
int w8a8_pack_weight_nk(const int8_t *w_nk, int64_t ldw, int64_t N, int64_t K, int64_t interleave,
                        int8_t *packed, hipStream_t stream);

/* ---- prologue: per-row int8 quantisation (pipeline.py:49-52) ---------------------------- */

/* scale[m] = max(amax_k |x[m,k]|, 1e-8) / 127;  q[m,k] = clamp(rint(x[m,k] / scale[m]), +-127)
 * with IEEE fp32 division and round-half-even.  x bf16 [M, K]. */
int w8a8_quant_rows_bf16(const uint16_t *x, int64_t ldx, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                         float *scale, hipStream_t stream);

/* Same for fp32 rows; applied to a weight W[N, K] it is the per-output-channel weight quant
 * of gemma_npu.py:68-69. */
int w8a8_quant_rows_f32(const float *x, int64_t ldx, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                        float *scale, hipStream_t stream);

/* ---- GEMM (npu_kernels.py:40-64) --------------------------------------------------------- */

/* C[M, N] int32 = A[M, K] int8 @ W, W packed by w8a8_pack_weight_* (interleave 0).
 * Exact integer arithmetic.  K % 16 == 0; A rows 16-byte aligned (lda % 16 == 0); C 4-byte
 * aligned (rows 16-byte aligned use vector stores).  Any M >= 0 and N >= 1: no padding to 512 is needed
 * (the reference's mm_i8 floors M and N to multiples of 512, npu_kernels.py:63). */
int w8a8_gemm_i32(const int8_t *a, int64_t lda, const int8_t *w_packed, int64_t M, int64_t N, int64_t K,
                  int32_t *c, int64_t ldc, hipStream_t stream);

/* Self-check of the division-free quant step the bf16 quant kernels use (no counterpart in the
 * reference; for callers and tests that want to confirm the device's arithmetic): for every
 * positive finite bf16 absmax a and every bf16 v with |v| <= a, compares
 * clamp(rint(v / s), +-127) (IEEE division, s = max(a, 1e-8) / 127) with the kernels' form
 * q0 = v * (1/s), q1 = fma(fma(-q0, s, v), 1/s, q0), clamp(rint(q1), +-127).  Adds the number of
 * differing pairs to counts[0] and the number of pairs compared (1,065,402,240) to counts[1];
 * counts is device memory, 8-byte aligned, zeroed by the caller. */
int w8a8_selfcheck_quant_step(unsigned long long *counts, hipStream_t stream);

/* Engine-clock probe (no counterpart in the reference; for benchmarks that state the clock a
 * kernel ran at): launches one wave on `stream` that reads the core-clock counter and the
 * constant-rate real-time counter at the start and the end of a window of `ticks` real-time ticks
 * (ticks in 1 .. 1e8) and writes out[0] = core cycles and out[1] = real-time ticks elapsed (device
 * memory, 8-byte aligned).  *wall_clock_khz (host) receives the real-time counter's rate, so the
 * clock over the window is out[0] / out[1] * wall_clock_khz kHz.  Launched on a second stream while
 * other kernels run, it measures the clock they run at. */
int w8a8_clock_probe(unsigned long long *out, unsigned ticks, int *wall_clock_khz, hipStream_t stream);

/* ---- packed activations ----------------------------------------------------------------- */

/* The GEMM streams A fastest when it is laid out like the packed weight: 1 KiB fragments of
 * 32 rows x 32 k (fragment (mt, j) at (mt * KF + j) * 1024, KF = 2 * ceil(K/64); byte 16*l + b
 * = row 32*mt + l%32, k 32*j + 16*(l/32) + b), zero past M (to a multiple of 32) and past K (to
 * a multiple of 64).  Bytes of that layout for M rows of K; -1 if invalid. */
int64_t w8a8_packed_act_bytes(int64_t M, int64_t K);

/* Row-major int8 A[M, K] (lda % 16 == 0) -> packed activations. */
int w8a8_pack_act(const int8_t *a, int64_t lda, int64_t M, int64_t K, int8_t *packed, hipStream_t stream);

/* Per-row quantisation of bf16 rows (as w8a8_quant_rows_bf16) written straight into the packed
 * activation layout; scale[m] fp32 per row. */
int w8a8_quant_rows_packed_bf16(const uint16_t *x, int64_t ldx, int64_t M, int64_t K, int8_t *packed, float *scale,
                                hipStream_t stream);

/* Number of explicit tile configurations the _ex GEMMs accept (tile_cfg 0 .. n-1). */
int w8a8_gemm_tile_configs(void);

/* The tile configuration the automatic choice (tile_cfg = -1) takes for [M, N, K] with int32
 * output (epilogue -1) or the bf16 epilogue 0 (dequant), 1 (GELU) or 2 (residual); -1 for an
 * invalid shape or epilogue.  No
 * counterpart in the reference (its single Triton kernel has one schedule, npu_kernels.py:29-37);
 * for tests and benchmarks that report which kernel ran. */
int w8a8_gemm_pick_tile_config(int64_t M, int64_t N, int64_t K, int epilogue);

/* Workspace bytes the _ex GEMMs need for [M, N, K] with tile_cfg (-1 = automatic) and split_k:
 * always 0, since no tile configuration splits K across blocks (the long-K configurations split
 * a tile's k-steps among the waves of one block and add the partials in LDS); -1 for a tile_cfg out
 * of range or split_k > 1.  Kept so that callers written against a split-K workspace still work. */
int64_t w8a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int tile_cfg, int split_k);

/* As w8a8_gemm_i32 with A given either row-major (a_packed = 0, lda used) or packed
 * (a_packed = 1, lda ignored) and an explicit tile configuration (0 .. w8a8_gemm_tile_configs()-1,
 * -1 = automatic).  split_k must be 0 (automatic) or 1; larger values fail with W8A8_ENOTSUP.
 * workspace / workspace_bytes are not used (may be NULL / 0). */
int w8a8_gemm_i32_ex(const int8_t *a, int64_t lda, int a_packed, const int8_t *w_packed, int64_t M, int64_t N,
                     int64_t K, int32_t *c, int64_t ldc, int tile_cfg, int split_k, void *workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/* GEMM with the dequantising epilogue, bf16 out:
 *   y[m, n] = bf16((float(acc[m, n]) * sx[m]) * sw[n])                 (pipeline.py:55-57)
 * epilogue 0: out = y                                                  [M, N]
 *          1: out = bf16(bf16(gelu_tanh(y[:, :I])) * y[:, I:])          [M, I] (pipeline.py:106);
 *             needs the weight packed with interleave = I = N / 2
 *          2: out = bf16(res + y)                                      [M, N]
 * sx fp32 [M] (per token), sw fp32 [N] (per channel, [gate; up] order for epilogue 1). */
int w8a8_gemm_bf16(const int8_t *a, int64_t lda, const float *sx, const int8_t *w_packed, const float *sw,
                   int64_t M, int64_t N, int64_t K, int epilogue, int64_t interleave, const uint16_t *res,
                   int64_t ldr, uint16_t *out, int64_t ldo, hipStream_t stream);

/* As w8a8_gemm_bf16 with packed or row-major A and an explicit tile configuration; split_k and
 * the workspace as w8a8_gemm_i32_ex. */
int w8a8_gemm_bf16_ex(const int8_t *a, int64_t lda, int a_packed, const float *sx, const int8_t *w_packed,
                      const float *sw, int64_t M, int64_t N, int64_t K, int epilogue, int64_t interleave,
                      const uint16_t *res, int64_t ldr, uint16_t *out, int64_t ldo, int tile_cfg, int split_k,
                      void *workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---- element-wise neighbours ------------------------------------------------------------- */

/* out = bf16((float(acc) * sx[m]) * sw[n])  (pipeline.py:55-57 on an int32 result). */
int w8a8_dequant_bf16(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, int64_t M, int64_t N,
                      uint16_t *out, int64_t ldo, hipStream_t stream);

/* h = bf16(res + bf16(y * (mean(y^2) + eps)^-0.5 * w))  (k_post_ff, pipeline.py:110-114) on a
 * bf16 y; w may be NULL (no weight, pipeline.py:46).  res may be NULL: then h = bf16(y *
 * (mean(y^2) + eps)^-0.5 * w), the RMSNorm module of HF's Gemma 4 text model on bf16 rows (the
 * norms around every decoder layer of the reference's HF-driven decode, gemma_npu.py:278-300).
 * If q / sq are given, also the int8 rows (row-major, ld = ldq) and scales of h (the `_quant(h)` of
 * k_post_ff).  h may alias y or res.  N % 8 == 0, N <= 12288, 16-byte aligned rows and w. */
int w8a8_rms_residual_bf16(const uint16_t *y, int64_t ldy, const uint16_t *res, int64_t ldr, const uint16_t *w,
                           float eps, int64_t M, int64_t N, uint16_t *h, int64_t ldh, int8_t *q, int64_t ldq,
                           float *sq, hipStream_t stream);

/* ---- the fused kernels between the GEMMs (pipeline.py:66-127) ---------------------------------
 *
 * Each takes the int32 GEMM result acc [M, N] (ld = ldacc) with its per-token scales sx fp32 [M]
 * and per-channel scales sw fp32 [N], exactly as the reference's k_* functions do, and applies
 *   y = bf16((float(acc) * sx[m]) * sw[n])                              (_deq, pipeline.py:55-57)
 *   rms(x, w) = x * (mean(x^2) + eps)^-0.5 * w in fp32, w NULL: no weight (_rms, pipeline.py:43-46)
 *   quant(x): s = max(amax|x|, 1e-8) / 127, q = clamp(rint(x / s), +-127)  (_quant, pipeline.py:49-52)
 * with every bf16 rounding the eager torch expressions perform.  Where an int8 output q is
 * produced, q_packed = 0 writes it row-major (ld = ldq, 8-byte aligned rows) and q_packed = 1 in
 * the packed activation layout (w8a8_packed_act_bytes(M, N) bytes, 16-byte aligned; ldq ignored),
 * ready as the next GEMM's A operand; sq fp32 [M] receives the scales.  Row lengths N are
 * multiples of 8 up to 12288; bf16 / int32 rows and the sw / weight vectors are 16-byte aligned
 * (ld % 8 == 0 for bf16, ldacc % 4 == 0).  Outputs may alias the residual they replace. */

/* k_in (pipeline.py:66-69): q, sq = quant(bf16(rms(x, w))), x bf16 [M, N]. */
int w8a8_k_in(const uint16_t *x, int64_t ldx, const uint16_t *w, float eps, int64_t M, int64_t N, int8_t *q,
              int64_t ldq, int q_packed, float *sq, hipStream_t stream);

/* k_qkv (pipeline.py:72-85): y = dequant(acc) [T, slots * D] with columns [q heads; k heads; v heads];
 * per token and head: q = rope(bf16(rms(q_h, qw))), k = rope(bf16(rms(k_h, kw))),
 * v = bf16(rms(v_h, NULL)), rope(x) = bf16(bf16(x * cos) + bf16(cat(-x[D/2:], x[:D/2]) * sin))
 * (pipeline.py:60-63) with cos / sin bf16 [T, D] (ld = ldcs).  Outputs are head-major and
 * contiguous: q [H, T, D], k and v [KV, T, D] (the reference's .transpose(0, 1) views, stored).
 * shared != 0 (a KV-shared layer): only the H query heads exist; k, v, kw are not used.
 * D in {128, 256, 512}. */
int w8a8_k_qkv(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, const uint16_t *cos_,
               const uint16_t *sin_, int64_t ldcs, const uint16_t *qw, const uint16_t *kw, float eps, int64_t T,
               int64_t H, int64_t KV, int64_t D, int shared, uint16_t *q, uint16_t *k, uint16_t *v,
               hipStream_t stream);

/* k_attn_out (pipeline.py:88-92): the attention output o [H, T, D] bf16, element (h, t, d) at
 * o + h * head_stride + t * row_stride + d, read as rows [T, H * D] and quantised. */
int w8a8_k_attn_out(const uint16_t *o, int64_t head_stride, int64_t row_stride, int64_t H, int64_t T, int64_t D,
                    int8_t *q, int64_t ldq, int q_packed, float *sq, hipStream_t stream);

/* k_post_attn (pipeline.py:95-99): h = bf16(res + bf16(rms(y, w_post)));
 * q, sq = quant(bf16(rms(h, w_pre_ff))). */
int w8a8_k_post_attn(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, const uint16_t *res,
                     int64_t ldr, const uint16_t *w_post, const uint16_t *w_pre_ff, float eps, int64_t M, int64_t N,
                     uint16_t *h, int64_t ldh, int8_t *q, int64_t ldq, int q_packed, float *sq, hipStream_t stream);

/* k_gelu (pipeline.py:102-107) on an int32 result acc [M, 2I] in [gate; up] column order:
 * q, sq = quant(bf16(bf16(gelu_tanh(y[:, :I])) * y[:, I:])).  (The fused GEMM epilogue 1 computes
 * the same activation without the int32 round trip.) */
int w8a8_k_gelu(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, int64_t M, int64_t I, int8_t *q,
                int64_t ldq, int q_packed, float *sq, hipStream_t stream);

/* k_post_ff (pipeline.py:110-114): h = bf16(res + bf16(rms(y, w_post_ff))); q, sq = quant(h). */
int w8a8_k_post_ff(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, const uint16_t *res,
                   int64_t ldr, const uint16_t *w_post_ff, float eps, int64_t M, int64_t N, uint16_t *h, int64_t ldh,
                   int8_t *q, int64_t ldq, int q_packed, float *sq, hipStream_t stream);

/* k_ple_gate (pipeline.py:117-121): q, sq = quant(bf16(bf16(gelu_tanh(y)) * ple)), ple bf16 [M, N]
 * (ld = ldp; the reference passes a strided per-layer slice). */
int w8a8_k_ple_gate(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, const uint16_t *ple,
                    int64_t ldp, int64_t M, int64_t N, int8_t *q, int64_t ldq, int q_packed, float *sq,
                    hipStream_t stream);

/* k_ple_out (pipeline.py:124-127): out = bf16(bf16(h + bf16(rms(y, w_post_ple))) * scalar), scalar
 * one bf16 value in device memory (the layer scalar). */
int w8a8_k_ple_out(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, const uint16_t *h,
                   int64_t ldh, const uint16_t *w_post_ple, const uint16_t *scalar, float eps, int64_t M, int64_t N,
                   uint16_t *out, int64_t ldo, hipStream_t stream);

/* h = bf16(bf16(res + bf16(rms(y, w1))) * scalar) (scalar one bf16 value in device memory, or NULL: no
 * product) and x = bf16(rms(h, w2)), both stored as bf16 rows [M, N]: k_post_attn's two norms
 * (pipeline.py:95-99) and k_ple_out followed by the next layer's input norm (pipeline.py:124-127,
 * 66-69), with bf16 outputs instead of the quant, for the decode step.  w1 / w2 may be NULL (no
 * weight).  N % 8 == 0, N <= 12288, 16-byte aligned rows and weights. */
int w8a8_rms_residual_norm_bf16(const uint16_t *y, int64_t ldy, const uint16_t *res, int64_t ldr, const uint16_t *w1,
                                const uint16_t *scalar, const uint16_t *w2, float eps, int64_t M, int64_t N,
                                uint16_t *h, int64_t ldh, uint16_t *x, int64_t ldx, hipStream_t stream);

/* bf16(bf16(gelu_tanh(y[:, :N])) * m) as bf16 rows out [M, N] (ld = ldo), m = mul [M, N] (ld = ldm) or,
 * with mul NULL, y[:, N:2N] (y then holds 2N columns): k_gelu's and k_ple_gate's activation
 * (pipeline.py:102-107, 117-121) for the decode step, whose next linear is the bf16-activation
 * int8 GEMV (gemma_npu.py:117-121, 155-156) rather than a quantised GEMM.  The same kernel and
 * arithmetic as those two; N % 8 == 0, N <= 12288, 16-byte aligned rows. */
int w8a8_gelu_mul_bf16(const uint16_t *y, int64_t ldy, const uint16_t *mul, int64_t ldm, int64_t M, int64_t N,
                       uint16_t *out, int64_t ldo, hipStream_t stream);

/* The same five kernels fed the dequantised bf16 rows y [rows, N] (ld = ldy, 16-byte aligned rows)
 * instead of an int32 result with its scales: y is what the GEMM's dequant epilogue
 * (w8a8_gemm_bf16 epilogue 0) writes, bf16((acc * sx) * sw), the values the int32 entries compute
 * first, so the results are bit-identical while the GEMM writes, and the kernel reads, half the
 * bytes.  Same reference functions as their int32 twins (pipeline.py:72-85, 95-99, 110-127). */
int w8a8_k_qkv_y(const uint16_t *y, int64_t ldy, const uint16_t *cos_, const uint16_t *sin_, int64_t ldcs,
                 const uint16_t *qw, const uint16_t *kw, float eps, int64_t T, int64_t H, int64_t KV, int64_t D,
                 int shared, uint16_t *q, uint16_t *k, uint16_t *v, hipStream_t stream);
/* k_qkv_y for a decode step that writes its keys and values into the cache: k_cache / v_cache are
 * [KV, kv_rows, D] bf16 (rows contiguous, heads kv_rows * D apart) and token t's key and value go to
 * row *pos + t (pos: one int32 in device memory, so a step captured in a HIP graph writes at each new
 * position); rows at or past kv_rows (or negative) are not written.  q as in k_qkv_y.  Not for
 * KV-shared layers (they write no keys). */
int w8a8_k_qkv_cache_y(const uint16_t *y, int64_t ldy, const uint16_t *cos_, const uint16_t *sin_, int64_t ldcs,
                       const uint16_t *qw, const uint16_t *kw, float eps, int64_t T, int64_t H, int64_t KV, int64_t D,
                       uint16_t *q, uint16_t *k_cache, uint16_t *v_cache, int64_t kv_rows, const int32_t *pos,
                       hipStream_t stream);
int w8a8_k_post_attn_y(const uint16_t *y, int64_t ldy, const uint16_t *res, int64_t ldr, const uint16_t *w_post,
                       const uint16_t *w_pre_ff, float eps, int64_t M, int64_t N, uint16_t *h, int64_t ldh, int8_t *q,
                       int64_t ldq, int q_packed, float *sq, hipStream_t stream);
int w8a8_k_post_ff_y(const uint16_t *y, int64_t ldy, const uint16_t *res, int64_t ldr, const uint16_t *w_post_ff,
                     float eps, int64_t M, int64_t N, uint16_t *h, int64_t ldh, int8_t *q, int64_t ldq, int q_packed,
                     float *sq, hipStream_t stream);
int w8a8_k_ple_gate_y(const uint16_t *y, int64_t ldy, const uint16_t *ple, int64_t ldp, int64_t M, int64_t N,
                      int8_t *q, int64_t ldq, int q_packed, float *sq, hipStream_t stream);
int w8a8_k_ple_out_y(const uint16_t *y, int64_t ldy, const uint16_t *h, int64_t ldh, const uint16_t *w_post_ple,
                     const uint16_t *scalar, float eps, int64_t M, int64_t N, uint16_t *out, int64_t ldo,
                     hipStream_t stream);

/* w8a8_k_ple_out / _y followed by the next layer's w8a8_k_in on the rows it writes, in one launch:
 * out as w8a8_k_ple_out writes it, and q / sq = quant(bf16(rms(out) * w_in_next)) as w8a8_k_in
 * (pipeline.py:124-127 then 66-69; row-major or packed q).  Bit for bit the two launches. */
int w8a8_k_ple_out_k_in(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw, const uint16_t *h,
                        int64_t ldh, const uint16_t *w_post_ple, const uint16_t *scalar, const uint16_t *w_in_next,
                        float eps, int64_t M, int64_t N, uint16_t *out, int64_t ldo, int8_t *q, int64_t ldq,
                        int q_packed, float *sq, hipStream_t stream);
int w8a8_k_ple_out_k_in_y(const uint16_t *y, int64_t ldy, const uint16_t *h, int64_t ldh, const uint16_t *w_post_ple,
                          const uint16_t *scalar, const uint16_t *w_in_next, float eps, int64_t M, int64_t N,
                          uint16_t *out, int64_t ldo, int8_t *q, int64_t ldq, int q_packed, float *sq,
                          hipStream_t stream);

/* ---- whole linear: bf16 in -> bf16 out (NPUGemm.matmul, gemma_npu.py:117-152) ------------ */

/* Workspace for w8a8_linear_bf16: the packed int8 rows and the per-row scales, 256-byte aligned
 * parts (scratch: nothing is kept between calls, no clearing is needed).  Calls that overlap in
 * time need separate workspaces. */
int64_t w8a8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* quant_rows(x) -> GEMM -> epilogue.  epilogue 0-2 as w8a8_gemm_bf16; 3: residual with RMSNorm,
 * out = bf16(res + bf16(rms(y) * rms_w)) (pipeline.py:113).  workspace: 256-byte aligned,
 * w8a8_linear_workspace_bytes(M, N, K) long. */
int w8a8_linear_bf16(const uint16_t *x, int64_t ldx, const int8_t *w_packed, const float *sw, int64_t M, int64_t N,
                     int64_t K, int epilogue, int64_t interleave, const uint16_t *res, int64_t ldr,
                     const uint16_t *rms_w, float eps, uint16_t *out, int64_t ldo, void *workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/* w8a8_linear_bf16 without a workspace and without allocating anything.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The packed int8 rows and the
 * per-row scales go to a 64 MiB scratch array that the library holds on each GPU it runs on
 * until the process ends, so align256(w8a8_packed_act_bytes(M, K)) + align256(4 * M) must not
 * exceed 64 MiB (e.g. M = 8192 at K = 6144, M = 16384 at K = 2048): larger calls fail with
 * W8A8_ENOTSUP before launching.  The same kernels and the same results as w8a8_linear_bf16.
 * Every call on one GPU shares that scratch: calls that overlap in time on one GPU (two streams,
 * two threads) race; calls ordered on one stream do not.  Nothing needs clearing between calls. */
int w8a8_linear_bf16_noalloc(const uint16_t *x, int64_t ldx, const int8_t *w_packed, const float *sw, int64_t M,
                             int64_t N, int64_t K, int epilogue, int64_t interleave, const uint16_t *res,
                             int64_t ldr, const uint16_t *rms_w, float eps, uint16_t *out, int64_t ldo,
                             hipStream_t stream);

/* ---- decode GEMV (gemma_npu.py:155-172, torch._weight_int8pack_mm) ---------------------- */

/* y[m, n] = bf16((sum_k x[m, k] * w[n, k]) * s[n]),  x bf16 [M, K] with 1 <= M <= 16,
 * w int8 [N, K] (ld = ldw), s bf16 (scale_is_f32 = 0, as gemma_npu.py:82) or fp32 [N].
 * K % 16 == 0; x and w rows 16-byte aligned.  fp32 accumulation; deterministic. */
int w8a8_gemv_bf16(const uint16_t *x, int64_t ldx, int64_t M, const int8_t *w, int64_t ldw, int64_t N, int64_t K,
                   const void *scales, int scale_is_f32, uint16_t *y, int64_t ldy, hipStream_t stream);

/* Bytes of the GEMV fragment layout of an int8 W [N, K]: ceil(N/16) * ceil(K/64) KiB; -1 if invalid.
 * Fragment (t, kb) (n-tile t of 16 rows, k-block kb of 64) is 1 KiB at (t * ceil(K/64) + kb) * 1024
 * whose byte 16*l + b is W[16t + l%16][64kb + 16(l/16) + b]; rows past N and k past K are zero.
 * The resident decode copy of a weight (the reference's w_cpu [N, K], gemma_npu.py:81) can be
 * kept in this layout: the GEMV then reads it in whole contiguous KiB with the streaming cache
 * policy. */
int64_t w8a8_gemv_packed_bytes(int64_t N, int64_t K);

/* Row-major int8 W [N, K] (ld = ldw, 16-byte aligned rows, K % 16 == 0) -> GEMV fragment layout. */
int w8a8_pack_gemv_weight(const int8_t *w, int64_t ldw, int64_t N, int64_t K, int8_t *packed, hipStream_t stream);

/* As w8a8_gemv_bf16 with the weight in the GEMV fragment layout (w8a8_pack_gemv_weight); same
 * results bit for bit (the same products are added in the same order). */
int w8a8_gemv_packed_bf16(const uint16_t *x, int64_t ldx, int64_t M, const int8_t *packed, int64_t N, int64_t K,
                          const void *scales, int scale_is_f32, uint16_t *y, int64_t ldy, hipStream_t stream);

/* w8a8_gemv_packed_bf16 with the activation that follows it on the decode path, in its epilogue:
 *   act 1 (GELU pair): the packed weight holds [gate; up] stacked (N = 2I, I % 16 == 0); y [M, I] =
 *     bf16(bf16(gelu_tanh(g)) * u) with g, u the bf16 GEMV outputs of gate row n and up row I + n
 *     (the MLP's act(gate) * up on the decode rows, pipeline.py:102-107 without the quant);
 *   act 2 (GELU times a multiplier): y [M, N] = bf16(bf16(gelu_tanh(g)) * mul[m, n]), mul bf16 [M, N]
 *     (ld = ldm; the per-layer-input gate, pipeline.py:117-121 without the quant).
 * Bit for bit the GEMV followed by w8a8_gelu_mul_bf16; one launch instead of two.  Shapes with
 * fewer than 4096 n-tiles of 16 rows (the per-layer decode shapes). */
int w8a8_gemv_packed_act_bf16(const uint16_t *x, int64_t ldx, int64_t M, const int8_t *packed, int64_t N, int64_t K,
                              const void *scales, int scale_is_f32, int act, const uint16_t *mul, int64_t ldm,
                              uint16_t *y, int64_t ldy, hipStream_t stream);

/* One decode row (M = 1) whose GEMV input is the residual stream's norm, made in the same launch:
 *   h = bf16(res + bf16(rms(y) * w1)), then h = bf16(h * scalar[0]) when scalar is given
 *   (no res: h = bf16(rms(y) * w1); no w1: no weight), x = norm2 ? bf16(rms(h) * w2) : h,
 *   out = the GEMV of x (act 0), or with act 1 / 2 as w8a8_gemv_packed_act_bf16 (mul [N]).
 * h and x are what w8a8_rms_residual_norm_bf16 (norm2 = 1) or w8a8_rms_residual_bf16 (norm2 = 0)
 * write, bit for bit, and out is then the GEMV's result on that x: the post-attention / post-MLP /
 * per-layer-input norms of the decode step (pipeline.py:95-99, 110-114, 124-127 on one row) each
 * become the prologue of the next linear instead of a launch of their own.  Every workgroup makes
 * x from y and res; workgroup 0 stores h when h is non-null, so h must not overlap y, res or out,
 * and out must not overlap y, res or mul.  y, res, h: bf16 [K], K % 16 == 0, K <= 1536; w1, w2
 * bf16 [K]; 16-byte aligned.  Shapes with fewer than 4096 n-tiles (the per-layer decode shapes). */
int w8a8_gemv_packed_norm_bf16(const uint16_t *y, const uint16_t *res, const uint16_t *w1, const uint16_t *scalar,
                               int norm2, const uint16_t *w2, float eps, uint16_t *h, const int8_t *packed, int64_t N,
                               int64_t K, const void *scales, int scale_is_f32, int act, const uint16_t *mul,
                               uint16_t *out, hipStream_t stream);

/* The decode step's o projection (gemma_npu.py:120-121 on the attention output) with the decode
 * attention's chunk merge (local_attn.py:60-68) as its prologue: out [1, N] = the GEMV of the
 * token's attention output [H * D], which every workgroup merges from the chunk partials that
 * w8a8_attention_decode_qkv_dev_bf16 left in `workspace` when called with o = NULL (same H, KV, Tk,
 * D, window, scale and q_pos).  Bit for bit that attention's merge followed by
 * w8a8_gemv_packed_bf16; the merge launch is saved.  At most 16 key chunks (a sliding window of 512
 * keys: 8 at head_dim 256, 16 at 512), H * D <= 4096, the few-tile GEMV shapes. */
int w8a8_gemv_packed_attn_merge_bf16(const void *workspace, const int32_t *q_pos, int64_t H, int64_t KV, int64_t Tk,
                                     int64_t D, int64_t window, float scale, const int8_t *packed, int64_t N,
                                     const void *scales, int scale_is_f32, uint16_t *out, hipStream_t stream);

/* The decode step's end (the reference's decode loop, gemma_npu.py:292-295), two launches: y bf16 [V]
 * (the LM head's output) softcapped as the model's bf16 ops do it when cap > 0 (t = bf16(y * (1/cap)),
 * u = bf16(tanh(t)), bf16(u * cap); cap 0: none) into fp32 logits [V]; the first index of their
 * maximum (NaN counting as the largest, as torch.argmax) is written to *tok and to emitted[*n_emitted]
 * (when below max_emitted); *n_emitted, *pos and *pos64 advance by one.  Everything it reads and
 * writes is in device memory, so a captured decode step replays it at each new position.  Workspace
 * bytes from w8a8_decode_tail_workspace_bytes(V). */
int64_t w8a8_decode_tail_workspace_bytes(int64_t V);
int w8a8_decode_tail(const uint16_t *y, int64_t V, float cap, float *logits, int32_t *pos, int64_t *pos64,
                     int64_t *tok, int64_t *emitted, int64_t *n_emitted, int64_t max_emitted, void *workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/* ---- prefill attention ------------------------------------------------------------------ */

/* o[h, i, :] = sum_j softmax_j(scale * q[h, i] . k[g, j]) v[g, j] with g = h / (H / KV), over the
 * keys the query at position p = q_start + i may see: j <= p and, if window > 0, p - j < window.
 * Replaces full_attention (window 0: causal over k_all[:, :q_start + Tq], pipeline.py:140-155,
 * merging the prefix and the micro-batch's own keys in one pass) and sliding_attention
 * (pipeline.py:158-180, local_attn.py:91-107), both with scale 1.0, and the prefill branches of
 * local_sdpa (local_attn.py:84-107) for any positive scale.
 *   q  bf16 [H, Tq, D]  (element strides q_head_stride, q_row_stride; last dim contiguous)
 *   k  bf16 [KV, Tk, D] (k_head_stride, k_row_stride), v likewise; Tk >= q_start + Tq
 *   o  bf16 [H, Tq, D]  (o_head_stride, o_row_stride): e.g. D, H*D writes HF's [T, H, D] layout
 *   lse fp32 [H, Tq] natural-log logsumexp of the scaled scores per query, or NULL
 * D in {128, 256, 512}; H % KV == 0 and H / KV <= 128; strides multiples of 8 elements; pointers
 * 16-byte aligned.  Scores, softmax and sums in fp32, the softmax weights rounded to bf16 for the
 * second product (as the CPU flash kernel does). */
int w8a8_attention_bf16(const uint16_t *q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t *k,
                        int64_t k_head_stride, int64_t k_row_stride, const uint16_t *v, int64_t v_head_stride,
                        int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                        int64_t q_start, int64_t window, float scale, uint16_t *o, int64_t o_head_stride,
                        int64_t o_row_stride, float *lse, hipStream_t stream);

/* Bytes of the workspace w8a8_attention_ws_bf16 uses for these arguments (0: it splits no query
 * tile and needs none; -1: invalid arguments).  For causal calls the host plans the work list: long
 * query tiles' keys are split over several workgroups (the last to finish merging the parts by their
 * logsumexp) when a model of the chip's workgroup dispatch says the split finishes sooner (at
 * T = 3658, head_dim 512: 229 tiles of 1 to 115 blocks of 32 keys become 520 items of at most 33
 * blocks), and the items are launched longest first.  The plan depends on the arguments and the
 * device's CU count only, so this size is stable for a shape. */
int64_t w8a8_attention_workspace_bytes(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start,
                                       int64_t window);

/* Diagnostic, no counterpart in the reference (for tests that must reach every form of the work
 * list): the items per KV group w8a8_attention_ws_bf16 plans for these arguments (query tiles,
 * each counted once per part its keys are split into), with *launch_order (if not NULL) set to 1
 * when the items launch through the longest-first order table and 0 when they run in plain item
 * order (plans of more than 1536 items per group, or one item per tile), and *merge_kernel (if not
 * NULL) set to 1 when split tiles are merged by a second kernel after the parts, 0 when the last
 * part of each tile merges them (or nothing is split); -1 if invalid. */
int64_t w8a8_attention_plan_items(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start,
                                  int64_t window, int *launch_order, int *merge_kernel);

/* w8a8_attention_bf16 with a workspace for splitting long causal tiles: device memory of at least
 * w8a8_attention_workspace_bytes(...) bytes, 16-byte aligned, ZERO-FILLED BEFORE ITS FIRST USE (its
 * first 64 KiB are arrival counters that every call leaves zero, at the same offsets for every
 * shape, so one workspace serves calls of any shapes; the rest is scratch for the parked parts).  Calls that
 * share a workspace must be ordered (one stream).  NULL behaves as w8a8_attention_bf16.  The parts
 * are merged in a fixed order, so results are deterministic; they may differ from the unsplit
 * call's in the last bits. */
int w8a8_attention_ws_bf16(const uint16_t *q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t *k,
                           int64_t k_head_stride, int64_t k_row_stride, const uint16_t *v, int64_t v_head_stride,
                           int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                           int64_t q_start, int64_t window, float scale, uint16_t *o, int64_t o_head_stride,
                           int64_t o_row_stride, float *lse, void *workspace, int64_t workspace_bytes,
                           hipStream_t stream);

/* 1 when w8a8_attention_quant_bf16 runs these arguments in one launch (one KV group of at most 16
 * query heads, a power of two, and a plan that merges split key parts in the attention kernel
 * itself), else 0. */
int w8a8_attention_quant_supported(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start,
                                   int64_t window);

/* Attention with k_attn_out (pipeline.py:88-92; attention as pipeline.py:140-180) in its epilogue:
 * instead of o, the per-token int8 rows of the [Tq, H*D] output (row t = [head 0 | head 1 | ...] of
 * position t) in the packed activation layout (w8a8_packed_act_bytes(Tq, H*D) bytes, 16-byte aligned,
 * rows Tq.. of the padding written as zeros) and their fp32 scales sx [Tq], the same bits as
 * w8a8_attention_ws_bf16 followed by w8a8_k_attn_out on its output.  The bf16 output is never
 * written.  W8A8_ENOTSUP where w8a8_attention_quant_supported is 0; the workspace as
 * w8a8_attention_ws_bf16's. */
int w8a8_attention_quant_bf16(const uint16_t *q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t *k,
                              int64_t k_head_stride, int64_t k_row_stride, const uint16_t *v, int64_t v_head_stride,
                              int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                              int64_t q_start, int64_t window, float scale, int8_t *packed, float *sx,
                              void *workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---- decode attention ------------------------------------------------------------------- */

/* Bytes of the workspace w8a8_attention_decode_bf16 needs: KV * ceil-chunks * (H/KV) * (D + 2) * 4,
 * chunks of 64 keys (32 at head_dim 512) over the visible range; -1 if the arguments are invalid. */
int64_t w8a8_attention_decode_workspace_bytes(int64_t H, int64_t KV, int64_t Tk, int64_t D, int64_t q_pos,
                                              int64_t window);

/* One query per head at position q_pos against keys 0..q_pos (the last `window` of them if window > 0):
 * o[h, :] = sum_j softmax_j(scale * q[h] . k[g, j]) v[g, j], g = h / (H / KV).  Replaces
 * _split_kv_decode (local_attn.py:44-68) and the decode branch of local_sdpa (local_attn.py:74-83):
 * the keys are split into chunks of 64 (32 at head_dim 512) whose partial results are merged by their
 * logsumexp (two launches; the merge runs in chunk order, so results are deterministic).
 *   q bf16 [H, D] (q_head_stride), k / v bf16 [KV, Tk, D], o bf16 [H, D] (o_head_stride), lse fp32 [H]
 *   or NULL; workspace: device memory of w8a8_attention_decode_workspace_bytes(...) bytes or more,
 *   16-byte aligned, scratch (no contents are kept between calls).
 * D in {128, 256, 512}; H / KV <= 16; strides multiples of 8 elements. */
int w8a8_attention_decode_bf16(const uint16_t *q, int64_t q_head_stride, const uint16_t *k, int64_t k_head_stride,
                               int64_t k_row_stride, const uint16_t *v, int64_t v_head_stride, int64_t v_row_stride,
                               int64_t H, int64_t KV, int64_t Tk, int64_t D, int64_t q_pos, int64_t window,
                               float scale, uint16_t *o, int64_t o_head_stride, float *lse, void *workspace,
                               int64_t workspace_bytes, hipStream_t stream);

/* The same attention with the query position read from device memory, *q_pos (int32), so that a
 * decode step captured in a HIP graph replays at each new position (the reference's decode loop,
 * gemma_npu.py:278-300, with local_attn.py:44-83 per layer).  Tk is the key cache's capacity: the
 * launch covers every position 0 <= *q_pos < Tk (chunks past the live ones return at once).  A
 * position outside that range is the caller's error: it yields meaningless values, never an access
 * outside k, v or the workspace.  Workspace bytes from w8a8_attention_decode_dev_workspace_bytes
 * (-1 for invalid arguments); no lse output. */
int64_t w8a8_attention_decode_dev_workspace_bytes(int64_t H, int64_t KV, int64_t Tk, int64_t D, int64_t window);
int w8a8_attention_decode_dev_bf16(const uint16_t *q, int64_t q_head_stride, const uint16_t *k, int64_t k_head_stride,
                                   int64_t k_row_stride, const uint16_t *v, int64_t v_head_stride,
                                   int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tk, int64_t D,
                                   const int32_t *q_pos, int64_t window, float scale, uint16_t *o,
                                   int64_t o_head_stride, void *workspace, int64_t workspace_bytes,
                                   hipStream_t stream);

/* w8a8_k_qkv_cache_y (or w8a8_k_qkv_y for q alone) and w8a8_attention_decode_dev_bf16 in one
 * launch (the decode step's k_qkv and attention, pipeline.py:72-86 and local_attn.py:44-83): y is
 * the token's qkv row, bf16 [H*D q | KV*D k | KV*D v] (kv_write = 1) or [H*D] (kv_write = 0, a layer
 * that reads another layer's keys); per q head RMS norm with qw (null: no weight) and RoPE with the
 * cos / sin rows [D] at the position: cos_ / sin_ are tables of rope_rows rows of D (row r for
 * position r) read at row *q_pos (a position past them reads zeros), or with rope_rows = 1 the one
 * row to use.  With kv_write the workgroup holding the position also makes
 * each KV head's key (norm with kw, RoPE) and value (norm without weight), writes them into k / v at
 * row *q_pos (when it is below Tk) and attends to them there.  Bit for bit the two-launch form.  At
 * most 8 query heads per KV head; 16-byte aligned pointers; workspace as
 * w8a8_attention_decode_dev_bf16's.  o = NULL: the chunks are not merged; their partials stay in
 * the workspace for w8a8_gemv_packed_attn_merge_bf16 (at most 16 chunks). */
int w8a8_attention_decode_qkv_dev_bf16(const uint16_t *y, const uint16_t *cos_, const uint16_t *sin_,
                                       int64_t rope_rows, const uint16_t *qw, const uint16_t *kw, float eps, uint16_t *k,
                                       int64_t k_head_stride, int64_t k_row_stride, uint16_t *v,
                                       int64_t v_head_stride, int64_t v_row_stride, int64_t H, int64_t KV,
                                       int64_t Tk, int64_t D, int kv_write, const int32_t *q_pos, int64_t window,
                                       float scale, uint16_t *o, int64_t o_head_stride, void *workspace,
                                       int64_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_H */
