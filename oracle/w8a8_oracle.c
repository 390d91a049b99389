/*
 * CPU oracle for the W8A8 linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic the reference runs on its
 * prefill/decode linear path, so that the GPU kernels can be checked against
 * it on the same seeded inputs.  It is never linked into the product library
 * and only the test suite, the smoke check and the benchmark's CPU-baseline
 * leg load it.
 *
 * Sources restated (reference repository, file:line):
 *   int_mm        npu_kernels.py:40-56  (matmul_i8_k: C = A @ B, int32 acc)
 *                 pipeline.py:237       (torch._int_mm(xq, w_kn), the cpu-int8 backend)
 *   quant_rows    pipeline.py:49-52     (_quant: absmax/127, round-half-even, clamp +-127)
 *                 gemma_npu.py:37-42    (_quant_rows, same formula)
 *                 gemma_npu.py:68-69    (per-output-channel weight quant, same formula)
 *   dequant       pipeline.py:55-57     (_deq: ((acc.float()*sx)*sw).to(bf16))
 *   gelu_mul      pipeline.py:102-107   (k_gelu: gelu_tanh(y[:, :I]) * y[:, I:])
 *   rms_residual  pipeline.py:43-46, 110-114 (k_post_ff: res + rms(y, w).to(bf16))
 *   gemv          gemma_npu.py:155-156  (torch._weight_int8pack_mm(x, w[N,K], s))
 *   rms_bf16      pipeline.py:43-46     (_rms(x, w, eps).to(bfloat16), the norms of k_in,
 *                                        k_qkv, k_post_attn)
 *   rope_rows     pipeline.py:60-63     (_rope on bf16 tensors)
 *   attention     pipeline.py:141-180, local_attn.py:71-107 (causal / sliding-window GQA
 *                                        attention, scale 1, the math of torch's sdpa / flash)
 * The fused k_* functions of pipeline.py:66-127 are compositions of these; oracle.py composes
 * them in the reference's order.
 *
 * bf16 values travel as uint16_t bit patterns.  All float arithmetic is
 * IEEE binary32 with round-to-nearest-even, matching torch's eager CPU ops
 * for the integer-exact parts; the fp32 reductions (rms mean, gemv dot) are
 * sequential and so agree with torch only to rounding.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fp32 -> bf16, round to nearest even; NaN stays a quiet NaN. */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }
float oracle_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }

/* C[M,N] int32 = A[M,K] int8 @ B[K,N] int8, all row-major (npu_kernels.py:40-56). */
void oracle_int_mm(const int8_t *a, int64_t lda, const int8_t *b, int64_t ldb,
                   int32_t *c, int64_t ldc, int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; ++m) {
        int32_t *crow = c + m * ldc;
        for (int64_t n = 0; n < N; ++n) crow[n] = 0;
        for (int64_t k = 0; k < K; ++k) {
            int32_t av = a[m * lda + k];
            if (av == 0) continue;
            const int8_t *brow = b + k * ldb;
            for (int64_t n = 0; n < N; ++n) crow[n] += av * (int32_t)brow[n];
        }
    }
}

/* Same product with the weight given as W[N,K] (the decode / packed-source layout,
 * gemma_npu.py:69 q and :81 w_cpu): C[m,n] = sum_k A[m,k] * W[n,k]. */
void oracle_int_mm_nk(const int8_t *a, int64_t lda, const int8_t *w, int64_t ldw,
                      int32_t *c, int64_t ldc, int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            int32_t s = 0;
            const int8_t *ar = a + m * lda, *wr = w + n * ldw;
            for (int64_t k = 0; k < K; ++k) s += (int32_t)ar[k] * (int32_t)wr[k];
            c[m * ldc + n] = s;
        }
}

/* Per-row symmetric int8 quantisation (pipeline.py:49-52):
 *   s = max(amax(|x|), 1e-8) / 127          (fp32 division)
 *   q = clamp(round_half_even(x / s), -127, 127)
 * dtype 0: x is bf16, dtype 1: x is fp32. */
void oracle_quant_rows(const void *x, int dtype, int64_t ldx, int64_t M, int64_t K,
                       int8_t *q, int64_t ldq, float *scale) {
    const float floor_v = 1e-8f;
    for (int64_t m = 0; m < M; ++m) {
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float v = dtype == 0 ? bf16_to_f32(((const uint16_t *)x)[m * ldx + k])
                                 : ((const float *)x)[m * ldx + k];
            float a = fabsf(v);
            if (a > amax || isnan(a)) amax = a;
        }
        if (!(amax >= floor_v)) amax = isnan(amax) ? amax : floor_v;
        float s = amax / 127.0f;
        scale[m] = s;
        for (int64_t k = 0; k < K; ++k) {
            float v = dtype == 0 ? bf16_to_f32(((const uint16_t *)x)[m * ldx + k])
                                 : ((const float *)x)[m * ldx + k];
            float r = nearbyintf(v / s);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            /* A NaN quotient (a row holding NaN: s is NaN; a row holding +-Inf: Inf / Inf) is
             * what torch's float -> int8 conversion turns into 0 on the host. */
            q[m * ldq + k] = isnan(r) ? 0 : (int8_t)r;
        }
    }
}

/* out[m,n] = bf16( (float(acc[m,n]) * sx[m]) * sw[n] )   (pipeline.py:55-57) */
void oracle_dequant(const int32_t *acc, int64_t ldacc, const float *sx, const float *sw,
                    int64_t M, int64_t N, uint16_t *out, int64_t ldo) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float v = (float)acc[m * ldacc + n];
            v = v * sx[m];
            v = v * sw[n];
            out[m * ldo + n] = f32_to_bf16(v);
        }
}

/* GELU, tanh form, on one bf16 value; result rounded to bf16 (F.gelu on a bf16 tensor). */
static inline uint16_t gelu_tanh_bf16(uint16_t h) {
    const float x = bf16_to_f32(h);
    const float kBeta = 0.7978845608028654f;   /* sqrt(2/pi) */
    const float kKappa = 0.044715f;
    float inner = kBeta * (x + kKappa * x * x * x);
    return f32_to_bf16(0.5f * x * (1.0f + tanhf(inner)));
}

/* k_gelu's activation (pipeline.py:106): a = bf16(gelu_tanh(y[:, :I]) * y[:, I:]),
 * y bf16 [M, 2I] in [gate ; up] column order (gemma_npu.py:219). */
void oracle_gelu_mul(const uint16_t *y, int64_t ldy, int64_t M, int64_t I,
                     uint16_t *out, int64_t ldo) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t i = 0; i < I; ++i) {
            float g = bf16_to_f32(gelu_tanh_bf16(y[m * ldy + i]));
            float u = bf16_to_f32(y[m * ldy + I + i]);
            out[m * ldo + i] = f32_to_bf16(g * u);
        }
}

/* h = bf16(res + bf16(rms(y) * w))  with rms(y) = y * (mean(y^2) + eps)^-0.5 in fp32
 * (pipeline.py:43-46 _rms, :113 k_post_ff).  w == NULL means no weight (pipeline.py:46). */
void oracle_rms_residual(const uint16_t *y, int64_t ldy, const uint16_t *res, int64_t ldr,
                         const uint16_t *w, float eps, int64_t M, int64_t N,
                         uint16_t *h, int64_t ldh) {
    for (int64_t m = 0; m < M; ++m) {
        float ss = 0.0f;
        for (int64_t n = 0; n < N; ++n) {
            float v = bf16_to_f32(y[m * ldy + n]);
            ss += v * v;
        }
        float r = 1.0f / sqrtf(ss / (float)N + eps);
        for (int64_t n = 0; n < N; ++n) {
            float v = bf16_to_f32(y[m * ldy + n]) * r;
            if (w) v = v * bf16_to_f32(w[n]);
            uint16_t nb = f32_to_bf16(v);
            h[m * ldh + n] = f32_to_bf16(bf16_to_f32(res[m * ldr + n]) + bf16_to_f32(nb));
        }
    }
}

/* h = bf16(res + y), the plain residual-add epilogue. */
void oracle_add_residual(const uint16_t *y, int64_t ldy, const uint16_t *res, int64_t ldr,
                         int64_t M, int64_t N, uint16_t *h, int64_t ldh) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            h[m * ldh + n] = f32_to_bf16(bf16_to_f32(res[m * ldr + n]) + bf16_to_f32(y[m * ldy + n]));
}

/* Weight-only int8 GEMV/GEMM (gemma_npu.py:155-156, torch._weight_int8pack_mm):
 *   y[m,n] = bf16( (sum_k float(x[m,k]) * float(w[n,k])) * s[n] )
 * x bf16 [M,K], w int8 [N,K], s bf16 (sdtype 0) or fp32 (sdtype 1) [N]. */
void oracle_gemv(const uint16_t *x, int64_t ldx, int64_t M, const int8_t *w, int64_t ldw,
                 int64_t N, int64_t K, const void *s, int sdtype, uint16_t *y, int64_t ldy) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            const uint16_t *xr = x + m * ldx;
            const int8_t *wr = w + n * ldw;
            for (int64_t k = 0; k < K; ++k) acc += bf16_to_f32(xr[k]) * (float)wr[k];
            float sc = sdtype == 0 ? bf16_to_f32(((const uint16_t *)s)[n]) : ((const float *)s)[n];
            y[m * ldy + n] = f32_to_bf16(acc * sc);
        }
}

/* ---- the reference's other fused element-wise kernels (pipeline.py:43-127) ---------------- */

/* out = bf16(rms(x) * w), rms(x) = x * (mean(x^2) + eps)^-0.5 in fp32, w == NULL: no weight
 * (pipeline.py:43-46 _rms followed by .to(bfloat16)).  x bf16 [M, N]. */
void oracle_rms_bf16(const uint16_t *x, int64_t ldx, const uint16_t *w, float eps, int64_t M, int64_t N,
                     uint16_t *out, int64_t ldo) {
    for (int64_t m = 0; m < M; ++m) {
        float ss = 0.0f;
        for (int64_t n = 0; n < N; ++n) {
            float v = bf16_to_f32(x[m * ldx + n]);
            ss += v * v;
        }
        float r = 1.0f / sqrtf(ss / (float)N + eps);
        for (int64_t n = 0; n < N; ++n) {
            float v = bf16_to_f32(x[m * ldx + n]) * r;
            if (w) v = v * bf16_to_f32(w[n]);
            out[m * ldo + n] = f32_to_bf16(v);
        }
    }
}

/* Rotary embedding of bf16 rows x[R, D] (D even), row r with cos / sin row r (pipeline.py:60-63):
 * rot = cat(-x[D/2:], x[:D/2]);  out = bf16(bf16(x * cos) + bf16(rot * sin)), all bf16 tensors. */
void oracle_rope_rows(const uint16_t *x, int64_t ldx, const uint16_t *cs, const uint16_t *sn, int64_t ldcs,
                      int64_t R, int64_t D, uint16_t *out, int64_t ldo) {
    const int64_t h = D / 2;
    for (int64_t r = 0; r < R; ++r) {
        const uint16_t *xr = x + r * ldx, *cr = cs + r * ldcs, *sr = sn + r * ldcs;
        for (int64_t d = 0; d < D; ++d) {
            float xv = bf16_to_f32(xr[d]);
            float rv = d < h ? -bf16_to_f32(xr[d + h]) : bf16_to_f32(xr[d - h]);
            float a = bf16_to_f32(f32_to_bf16(xv * bf16_to_f32(cr[d])));
            float b = bf16_to_f32(f32_to_bf16(rv * bf16_to_f32(sr[d])));
            out[r * ldo + d] = f32_to_bf16(a + b);
        }
    }
}

/* ---- prefill attention (pipeline.py:141-180, local_attn.py:71-107) -------------------------
 * o[h, i, :] = sum_j softmax_j(scale * q[h, i] . k[g, j]) v[g, j]  over the keys j the query at
 * position p = q_start + i may see: j <= p and, for a sliding layer (window W > 0), p - j < W;
 * g = h / (H / KV) (grouped-query heads).  q [H, Tq, D], k / v [KV, Tk, D] bf16, row-major with
 * the given strides (elements).  Scores, softmax and the weighted sum are computed in double; out
 * receives the bf16 result, budget (optional) sum_j p_j |v[g, j, d]| per output element (the scale
 * of the error a bf16 rounding of the weights p can make), lse (optional) the natural-log
 * logsumexp of the scaled scores per query [H, Tq] (what sdpa's flash kernels return and _merge,
 * pipeline.py:133-137, weighs partial results by). */
void oracle_attention(const uint16_t *q, int64_t qhs, int64_t qrs, const uint16_t *k, const uint16_t *v,
                      int64_t khs, int64_t krs, int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                      int64_t q_start, int64_t window, double scale, uint16_t *out, int64_t ohs, int64_t ors,
                      float *budget, double *lse) {
    double *s = (double *)malloc((size_t)Tk * sizeof(double));
    double *acc = (double *)malloc((size_t)D * sizeof(double));
    double *bud = (double *)malloc((size_t)D * sizeof(double));
    const int64_t G = H / KV;
    for (int64_t h = 0; h < H; ++h) {
        const int64_t g = h / G;
        for (int64_t i = 0; i < Tq; ++i) {
            const int64_t p = q_start + i;
            int64_t lo = 0, hi = p < Tk - 1 ? p : Tk - 1;
            if (window > 0 && p - window + 1 > lo) lo = p - window + 1;
            double mx = -INFINITY;
            for (int64_t j = lo; j <= hi; ++j) {
                double d = 0.0;
                for (int64_t e = 0; e < D; ++e)
                    d += (double)bf16_to_f32(q[h * qhs + i * qrs + e]) * (double)bf16_to_f32(k[g * khs + j * krs + e]);
                s[j] = d * scale;
                if (s[j] > mx) mx = s[j];
            }
            double sum = 0.0;
            for (int64_t j = lo; j <= hi; ++j) {
                s[j] = exp(s[j] - mx);
                sum += s[j];
            }
            for (int64_t e = 0; e < D; ++e) acc[e] = bud[e] = 0.0;
            for (int64_t j = lo; j <= hi; ++j) {
                const double w = s[j] / sum;
                for (int64_t e = 0; e < D; ++e) {
                    const double ve = (double)bf16_to_f32(v[g * khs + j * krs + e]);
                    acc[e] += w * ve;
                    bud[e] += w * fabs(ve);
                }
            }
            if (lse) lse[h * Tq + i] = mx + log(sum);
            for (int64_t e = 0; e < D; ++e) {
                out[h * ohs + i * ors + e] = f32_to_bf16((float)acc[e]);
                if (budget) budget[(h * Tq + i) * D + e] = (float)bud[e];
            }
        }
    }
    free(s);
    free(acc);
    free(bud);
}
