// C ABI of libw8a8: validation, error reporting and the GEMM / linear entry points.
//
// Every entry point takes plain device pointers, sizes and a hipStream_t, launches on that
// stream and returns 0 or a W8A8_E* status; w8a8_last_error() gives the message for the
// calling thread.  Nothing here allocates device memory or synchronises the stream.
#include <stdarg.h>
#include <stdio.h>

#include "gemm.h"
#include "w8a8_common.h"

namespace w8a8 {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(W8A8_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return W8A8_OK;
}

// Shared validation of the int8 A operand and packed weight for every GEMM entry point.
static int check_gemm_operands(const char* fn, const int8_t* a, int64_t lda, const int8_t* wp, int64_t M, int64_t N,
                               int64_t K, int64_t interleave, GemmParams& p) {
  if ((M > 0 && !a) || !wp) return fail(W8A8_EINVAL, "%s: null pointer", fn);
  if (M < 0 || N <= 0 || K <= 0) return fail(W8A8_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld", fn, (long long)M,
                                           (long long)N, (long long)K);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "%s: K=%lld must be a multiple of 16", fn, (long long)K);
  if (lda < K) return fail(W8A8_EINVAL, "%s: lda=%lld < K=%lld", fn, (long long)lda, (long long)K);
  if (lda % 16 != 0 || (uintptr_t)a % 16 != 0)
    return fail(W8A8_EALIGN, "%s: A rows must be 16-byte aligned (lda=%lld)", fn, (long long)lda);
  if ((uintptr_t)wp % 16 != 0) return fail(W8A8_EALIGN, "%s: packed weight not 16-byte aligned", fn);
  const int64_t wbytes = w8a8_packed_weight_bytes_internal(N, K, interleave);
  if (wbytes < 0) return fail(W8A8_EINVAL, "%s: interleave %lld does not fit N=%lld", fn, (long long)interleave,
                              (long long)N);
  // Buffer offsets are 32-bit: rows up to a full tile past M, and n-tiles up to a full tile
  // past N, must still be representable.
  const int64_t kt = (K + 63) / 64;
  if ((M + 257) * lda >= (int64_t(1) << 32) || wbytes + 17 * kt * 1024 >= (int64_t(1) << 32) || M > INT32_MAX ||
      N > INT32_MAX)
    return fail(W8A8_ENOTSUP, "%s: operands too large for 32-bit buffer offsets", fn);
  p = GemmParams{};
  p.a = a;
  p.wp = wp;
  p.lda = lda;
  p.M = int(M);
  p.N = int(N);
  p.KT = int((K + 63) / 64);
  p.NT = int(wbytes / (int64_t(p.KT) * 1024));
  p.a_bytes = M > 0 ? uint32_t((M - 1) * lda + K) : 0;
  p.w_bytes = uint32_t(wbytes);
  p.I = interleave > 0 ? int(interleave) : 0;
  return W8A8_OK;
}

int64_t w8a8_packed_weight_bytes_internal(int64_t N, int64_t K, int64_t interleave) {
  if (N <= 0 || K <= 0) return -1;
  int64_t nt;
  if (interleave > 0) {
    if (interleave % 16 != 0 || N != 2 * interleave) return -1;
    nt = 2 * (interleave / 16);
  } else {
    nt = (N + 15) / 16;
  }
  return nt * ((K + 63) / 64) * 1024;
}

}  // namespace w8a8

using namespace w8a8;

extern "C" {

const char* w8a8_last_error(void) { return g_err; }

int w8a8_abi_version(void) { return 1; }

int w8a8_gemm_i32_cfg(const int8_t* a, int64_t lda, const int8_t* w_packed, int64_t M, int64_t N, int64_t K,
                      int32_t* c, int64_t ldc, int tile_cfg, hipStream_t stream) {
  GemmParams p;
  int rc = check_gemm_operands("gemm_i32", a, lda, w_packed, M, N, K, 0, p);
  if (rc) return rc;
  if (!c && M > 0) return fail(W8A8_EINVAL, "gemm_i32: null C");
  if (ldc < N) return fail(W8A8_EINVAL, "gemm_i32: ldc=%lld < N=%lld", (long long)ldc, (long long)N);
  if ((uintptr_t)c % 4 != 0) return fail(W8A8_EALIGN, "gemm_i32: C must be 4-byte aligned");
  if (tile_cfg >= gemm_config_count()) return fail(W8A8_EINVAL, "gemm_i32: tile config %d out of range", tile_cfg);
  if (M == 0) return W8A8_OK;
  p.c = c;
  p.ldc = ldc;
  p.vec_store = (ldc % 4 == 0) && ((uintptr_t)c % 16 == 0);
  return gemm_launch(p, EPI_I32, tile_cfg, stream);
}

int w8a8_gemm_i32(const int8_t* a, int64_t lda, const int8_t* w_packed, int64_t M, int64_t N, int64_t K, int32_t* c,
                  int64_t ldc, hipStream_t stream) {
  return w8a8_gemm_i32_cfg(a, lda, w_packed, M, N, K, c, ldc, -1, stream);
}

int w8a8_gemm_bf16_cfg(const int8_t* a, int64_t lda, const float* sx, const int8_t* w_packed, const float* sw,
                       int64_t M, int64_t N, int64_t K, int epilogue, int64_t interleave, const uint16_t* res,
                       int64_t ldr, uint16_t* out, int64_t ldo, int tile_cfg, hipStream_t stream) {
  GemmParams p;
  int rc = check_gemm_operands("gemm_bf16", a, lda, w_packed, M, N, K, interleave, p);
  if (rc) return rc;
  if (M > 0 && (!sx || !out)) return fail(W8A8_EINVAL, "gemm_bf16: null scale or output pointer");
  if (!sw) return fail(W8A8_EINVAL, "gemm_bf16: null per-channel scales");
  int epi;
  int64_t out_cols = N;
  switch (epilogue) {
    case 0: epi = EPI_BF16; break;
    case 1:
      epi = EPI_GELU;
      if (interleave <= 0 || N != 2 * interleave)
        return fail(W8A8_EINVAL, "gemm_bf16: the GELU epilogue needs a weight packed with interleave = N/2");
      out_cols = interleave;
      break;
    case 2:
      epi = EPI_RESID;
      if (!res) return fail(W8A8_EINVAL, "gemm_bf16: residual epilogue without a residual");
      if (ldr < N) return fail(W8A8_EINVAL, "gemm_bf16: ldr < N");
      break;
    default: return fail(W8A8_EINVAL, "gemm_bf16: unknown epilogue %d", epilogue);
  }
  if (epi != EPI_GELU && interleave > 0)
    return fail(W8A8_EINVAL, "gemm_bf16: a gate/up-interleaved weight only goes with the GELU epilogue");
  if (ldo < out_cols) return fail(W8A8_EINVAL, "gemm_bf16: ldo=%lld too small", (long long)ldo);
  if ((uintptr_t)out % 2 != 0) return fail(W8A8_EALIGN, "gemm_bf16: output must be 2-byte aligned");
  if (tile_cfg >= gemm_config_count()) return fail(W8A8_EINVAL, "gemm_bf16: tile config %d out of range", tile_cfg);
  if (M == 0) return W8A8_OK;
  p.sx = sx;
  p.sw = sw;
  p.out = out;
  p.ldo = ldo;
  p.vec_store = (ldo % 4 == 0) && ((uintptr_t)out % 8 == 0);
  p.res = res;
  p.ldr = ldr;
  return gemm_launch(p, epi, tile_cfg, stream);
}

int w8a8_gemm_bf16(const int8_t* a, int64_t lda, const float* sx, const int8_t* w_packed, const float* sw, int64_t M,
                   int64_t N, int64_t K, int epilogue, int64_t interleave, const uint16_t* res, int64_t ldr,
                   uint16_t* out, int64_t ldo, hipStream_t stream) {
  return w8a8_gemm_bf16_cfg(a, lda, sx, w_packed, sw, M, N, K, epilogue, interleave, res, ldr, out, ldo, -1, stream);
}

int64_t w8a8_linear_workspace_bytes(int64_t M, int64_t K) {
  if (M < 0 || K <= 0) return -1;
  const int64_t kq = (K + 15) / 16 * 16;
  return (M * kq + 255) / 256 * 256 + M * 4;
}

int w8a8_quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq, float* scale,
                         hipStream_t stream);
int w8a8_rms_residual_bf16(const uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldr, const uint16_t* w,
                           float eps, int64_t M, int64_t N, uint16_t* h, int64_t ldh, int8_t* q, int64_t ldq,
                           float* sq, hipStream_t stream);

int w8a8_linear_bf16(const uint16_t* x, int64_t ldx, const int8_t* w_packed, const float* sw, int64_t M, int64_t N,
                     int64_t K, int epilogue, int64_t interleave, const uint16_t* res, int64_t ldr,
                     const uint16_t* rms_w, float eps, uint16_t* out, int64_t ldo, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream) {
  if (!x) return fail(W8A8_EINVAL, "linear_bf16: null x");
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "linear_bf16: K=%lld must be a multiple of 16", (long long)K);
  if (epilogue < 0 || epilogue > 3) return fail(W8A8_EINVAL, "linear_bf16: unknown epilogue %d", epilogue);
  const int64_t need = w8a8_linear_workspace_bytes(M, K);
  if (need < 0) return fail(W8A8_EINVAL, "linear_bf16: bad shape");
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256 != 0)
    return fail(W8A8_EINVAL, "linear_bf16: workspace needs %lld bytes, 256-byte aligned", (long long)need);
  if (M == 0) return W8A8_OK;
  const int64_t kq = (K + 15) / 16 * 16;
  int8_t* q = static_cast<int8_t*>(workspace);
  float* sx = reinterpret_cast<float*>(static_cast<char*>(workspace) + (M * kq + 255) / 256 * 256);
  int rc = w8a8_quant_rows_bf16(x, ldx, M, K, q, kq, sx, stream);
  if (rc) return rc;
  if (epilogue == 3) {
    // Reference order (pipeline.py:113): y = dequant (bf16) first, then res + rms(y) * w.
    if (!res) return fail(W8A8_EINVAL, "linear_bf16: residual_rms epilogue without a residual");
    rc = w8a8_gemm_bf16(q, kq, sx, w_packed, sw, M, N, K, 0, 0, nullptr, 0, out, ldo, stream);
    if (rc) return rc;
    return w8a8_rms_residual_bf16(out, ldo, res, ldr, rms_w, eps, M, N, out, ldo, nullptr, 0, nullptr, stream);
  }
  return w8a8_gemm_bf16(q, kq, sx, w_packed, sw, M, N, K, epilogue, interleave, res, ldr, out, ldo, stream);
}

}  // extern "C"
