// C ABI of libw8a8: validation, error reporting and the GEMM / linear entry points.
//
// Every entry point takes plain device pointers, sizes and a hipStream_t, launches on that
// stream and returns 0 or a W8A8_E* status; w8a8_last_error() gives the message for the
// calling thread.  Nothing here allocates device memory or synchronises the stream; the one
// file-scope device array (the scratch of w8a8_linear_bf16_noalloc) is part of the code object.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

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
static int check_gemm_operands(const char* fn, const int8_t* a, int64_t lda, int a_packed, const int8_t* wp,
                               int64_t M, int64_t N, int64_t K, int64_t interleave, GemmParams& p) {
  if ((M > 0 && !a) || !wp) return fail(W8A8_EINVAL, "%s: null pointer", fn);
  if (M < 0 || N <= 0 || K <= 0) return fail(W8A8_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld", fn, (long long)M,
                                           (long long)N, (long long)K);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "%s: K=%lld must be a multiple of 16", fn, (long long)K);
  if (!a_packed) {
    if (lda < K) return fail(W8A8_EINVAL, "%s: lda=%lld < K=%lld", fn, (long long)lda, (long long)K);
    if (lda % 16 != 0 || (uintptr_t)a % 16 != 0)
      return fail(W8A8_EALIGN, "%s: A rows must be 16-byte aligned (lda=%lld)", fn, (long long)lda);
  } else if ((uintptr_t)a % 16 != 0) {
    return fail(W8A8_EALIGN, "%s: packed A not 16-byte aligned", fn);
  }
  if ((uintptr_t)wp % 16 != 0) return fail(W8A8_EALIGN, "%s: packed weight not 16-byte aligned", fn);
  const int64_t wbytes = w8a8_packed_weight_bytes_internal(N, K, interleave);
  if (wbytes < 0) return fail(W8A8_EINVAL, "%s: interleave %lld does not fit N=%lld", fn, (long long)interleave,
                              (long long)N);
  // Buffer offsets are 32-bit: rows up to a full tile past M, and tiles up to a full block
  // past N, must still be representable.
  const int64_t kf = 2 * ((K + 63) / 64);
  const int64_t abytes = a_packed ? (M + 31) / 32 * kf * 1024 : (M > 0 ? (M - 1) * lda + K : 0);
  const int64_t aspan = a_packed ? abytes + 9 * kf * 1024 : (M + 257) * lda;
  if (aspan >= (int64_t(1) << 32) || wbytes + 9 * kf * 1024 >= (int64_t(1) << 32) || M > INT32_MAX ||
      N > INT32_MAX)
    return fail(W8A8_ENOTSUP, "%s: operands too large for 32-bit buffer offsets", fn);
  p = GemmParams{};
  p.a = a;
  p.wp = wp;
  p.lda = lda;
  p.M = int(M);
  p.N = int(N);
  p.KF = int(kf);
  p.NT = int(wbytes / (kf * 1024));
  p.a_bytes = uint32_t(abytes);
  p.w_bytes = uint32_t(wbytes);
  p.I = interleave > 0 ? int(interleave) : 0;
  return W8A8_OK;
}

int64_t w8a8_packed_weight_bytes_internal(int64_t N, int64_t K, int64_t interleave) {
  if (N <= 0 || K <= 0) return -1;
  int64_t nt;
  if (interleave > 0) {
    if (interleave % 32 != 0 || N != 2 * interleave) return -1;
    nt = 2 * (interleave / 32);
  } else {
    nt = (N + 31) / 32;
  }
  return nt * 2 * ((K + 63) / 64) * 1024;
}

// Shader-clock probe: one wave reads the core-clock counter (s_memtime) and the constant-rate
// real-time counter (s_memrealtime) at the start and at the end of a window of `ticks` real-time
// ticks, sleeping between reads; the ratio is the engine clock over the window, whatever else
// runs on the device meanwhile.  The loop also ends after 2^22 reads, so it always terminates.
__global__ __launch_bounds__(64) void clock_probe_kernel(unsigned long long* out, unsigned ticks) {
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  unsigned long long r = r0;
  for (int n = 0; r - r0 < ticks && n < (1 << 22); ++n) {
    __builtin_amdgcn_s_sleep(8);
    r = __builtin_amdgcn_s_memrealtime();
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r - r0;
  }
}

}  // namespace w8a8

using namespace w8a8;

extern "C" {

const char* w8a8_last_error(void) { return g_err; }

int w8a8_clock_probe(unsigned long long* out, unsigned ticks, int* wall_clock_khz, hipStream_t stream) {
  if (!out || !wall_clock_khz) return fail(W8A8_EINVAL, "clock_probe: null pointer");
  if (ticks == 0 || ticks > 100000000u) return fail(W8A8_EINVAL, "clock_probe: ticks %u out of range", ticks);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return fail(W8A8_EHIP, "clock_probe: %s", hipGetErrorString(e));
  clock_probe_kernel<<<1, 64, 0, stream>>>(out, ticks);
  return check_launch("clock_probe");
}

int w8a8_abi_version(void) { return 1; }

int w8a8_gemm_tile_configs(void) { return gemm_config_count(); }

int w8a8_gemm_pick_tile_config(int64_t M, int64_t N, int64_t K, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return -1;
  if (epilogue < -1 || epilogue > 2) return -1;
  const int epi = epilogue == 1 ? EPI_GELU : (epilogue == 2 ? EPI_RESID : (epilogue == 0 ? EPI_BF16 : EPI_I32));
  return gemm_pick_config(int(M), int((N + 31) / 32 * 32), int(2 * ((K + 63) / 64)) * 32, epi);
}

int64_t w8a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int tile_cfg, int split_k) {
  if (tile_cfg >= gemm_config_count() || split_k > 1) return -1;
  (void)M, (void)N, (void)K;
  return 0;  // no configuration splits K across blocks: the GEMMs need no workspace
}

int w8a8_gemm_i32_ex(const int8_t* a, int64_t lda, int a_packed, const int8_t* w_packed, int64_t M, int64_t N,
                     int64_t K, int32_t* c, int64_t ldc, int tile_cfg, int split_k, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream) {
  GemmParams p;
  int rc = check_gemm_operands("gemm_i32", a, lda, a_packed, w_packed, M, N, K, 0, p);
  if (rc) return rc;
  if (!c && M > 0) return fail(W8A8_EINVAL, "gemm_i32: null C");
  if (ldc < N) return fail(W8A8_EINVAL, "gemm_i32: ldc=%lld < N=%lld", (long long)ldc, (long long)N);
  if ((uintptr_t)c % 4 != 0) return fail(W8A8_EALIGN, "gemm_i32: C must be 4-byte aligned");
  if (tile_cfg >= gemm_config_count()) return fail(W8A8_EINVAL, "gemm_i32: tile config %d out of range", tile_cfg);
  if (split_k > 1) return fail(W8A8_ENOTSUP, "gemm_i32: split_k=%d: K is never split across blocks", split_k);
  (void)workspace, (void)workspace_bytes;
  if (M == 0) return W8A8_OK;
  p.c = c;
  p.ldc = ldc;
  p.vec_store = (ldc % 4 == 0) && ((uintptr_t)c % 16 == 0);
  return gemm_launch(p, EPI_I32, tile_cfg, a_packed != 0, stream);
}

int w8a8_gemm_i32(const int8_t* a, int64_t lda, const int8_t* w_packed, int64_t M, int64_t N, int64_t K, int32_t* c,
                  int64_t ldc, hipStream_t stream) {
  return w8a8_gemm_i32_ex(a, lda, 0, w_packed, M, N, K, c, ldc, -1, 0, nullptr, 0, stream);
}

int w8a8_gemm_bf16_ex(const int8_t* a, int64_t lda, int a_packed, const float* sx, const int8_t* w_packed,
                      const float* sw, int64_t M, int64_t N, int64_t K, int epilogue, int64_t interleave,
                      const uint16_t* res, int64_t ldr, uint16_t* out, int64_t ldo, int tile_cfg, int split_k,
                      void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  GemmParams p;
  int rc = check_gemm_operands("gemm_bf16", a, lda, a_packed, w_packed, M, N, K, interleave, p);
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
  if (split_k > 1) return fail(W8A8_ENOTSUP, "gemm_bf16: split_k=%d: K is never split across blocks", split_k);
  (void)workspace, (void)workspace_bytes;
  if (M == 0) return W8A8_OK;
  p.sx = sx;
  p.sw = sw;
  p.out = out;
  p.ldo = ldo;
  p.vec_store = (ldo % 4 == 0) && ((uintptr_t)out % 8 == 0);
  p.res = res;
  p.ldr = ldr;
  p.res_vec = res && (ldr % 4 == 0) && ((uintptr_t)res % 8 == 0);
  return gemm_launch(p, epi, tile_cfg, a_packed != 0, stream);
}

int w8a8_gemm_bf16(const int8_t* a, int64_t lda, const float* sx, const int8_t* w_packed, const float* sw, int64_t M,
                   int64_t N, int64_t K, int epilogue, int64_t interleave, const uint16_t* res, int64_t ldr,
                   uint16_t* out, int64_t ldo, hipStream_t stream) {
  return w8a8_gemm_bf16_ex(a, lda, 0, sx, w_packed, sw, M, N, K, epilogue, interleave, res, ldr, out, ldo, -1, 0,
                           nullptr, 0, stream);
}

// Workspace of w8a8_linear_bf16: [packed int8 rows | per-row scales], each part 256-byte aligned.
static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

int64_t w8a8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int64_t a = w8a8_packed_act_bytes(M, K);
  if (a < 0 || N <= 0) return -1;
  return align256(a) + align256(M * 4);
}

}  // extern "C"

namespace w8a8 {

// Argument checks shared by the two whole-linear entry points (everything but the workspace).
static int check_linear(const char* fn, const uint16_t* x, int64_t M, int64_t N, int64_t K, int epilogue,
                        const uint16_t* res, int64_t ldr, const uint16_t* rms_w, const uint16_t* out, int64_t ldo) {
  if (!x && M > 0) return fail(W8A8_EINVAL, "%s: null x", fn);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "%s: K=%lld must be a multiple of 16", fn, (long long)K);
  if (epilogue < 0 || epilogue > 3) return fail(W8A8_EINVAL, "%s: unknown epilogue %d", fn, epilogue);
  if (w8a8_packed_act_bytes(M, K) < 0 || N <= 0) return fail(W8A8_EINVAL, "%s: bad shape", fn);
  if (M > 0 && epilogue == 3) {
    if (!res) return fail(W8A8_EINVAL, "%s: residual_rms epilogue without a residual", fn);
    if (N % 8 != 0 || N > 12288)
      return fail(W8A8_ENOTSUP, "%s: the RMSNorm residual needs N %% 8 == 0 and N <= 12288 (N=%lld)", fn,
                  (long long)N);
    if ((uintptr_t)out % 16 || ldo % 8 || (uintptr_t)res % 16 || ldr % 8 || (uintptr_t)rms_w % 16)
      return fail(W8A8_EALIGN, "%s: the RMSNorm residual needs 16-byte aligned out / res rows and rms_w", fn);
  }
  return W8A8_OK;
}

// quant_rows(x) into the packed rows q and scales sx, then the GEMM with its epilogue.
static int run_linear(const uint16_t* x, int64_t ldx, const int8_t* w_packed, const float* sw, int64_t M, int64_t N,
                      int64_t K, int epilogue, int64_t interleave, const uint16_t* res, int64_t ldr,
                      const uint16_t* rms_w, float eps, uint16_t* out, int64_t ldo, int8_t* q, float* sx,
                      hipStream_t stream) {
  int rc = w8a8_quant_rows_packed_bf16(x, ldx, M, K, q, sx, stream);
  if (rc) return rc;
  if (epilogue == 3) {
    // Reference order (pipeline.py:113): y = dequant (bf16) first, then res + rms(y) * w.
    rc = w8a8_gemm_bf16_ex(q, 0, 1, sx, w_packed, sw, M, N, K, 0, 0, nullptr, 0, out, ldo, -1, 0, nullptr, 0,
                           stream);
    if (rc) return rc;
    return w8a8_rms_residual_bf16(out, ldo, res, ldr, rms_w, eps, M, N, out, ldo, nullptr, 0, nullptr, stream);
  }
  return w8a8_gemm_bf16_ex(q, 0, 1, sx, w_packed, sw, M, N, K, epilogue, interleave, res, ldr, out, ldo, -1, 0,
                           nullptr, 0, stream);
}

// ---- scratch of the linear that allocates nothing -----------------------------------------------
// Packed int8 rows, then per-row scales, for w8a8_linear_bf16_noalloc.  The array lives in the
// code object's zero-initialised data: each GPU the library runs on holds its own copy until the
// process ends.  In host code `scratch` only names the symbol; its device address (one per GPU)
// comes from hipGetSymbolAddress with that GPU current, and only that address is ever passed to
// a kernel.
static constexpr int64_t kNoAllocScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

static int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(W8A8_EHIP, "linear_bf16_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(W8A8_ENOTSUP, "linear_bf16_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(W8A8_EHIP, "linear_bf16_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  e != hipSuccess ? hipGetErrorString(e) : "null address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return W8A8_OK;
}

}  // namespace w8a8

extern "C" {

int w8a8_linear_bf16(const uint16_t* x, int64_t ldx, const int8_t* w_packed, const float* sw, int64_t M, int64_t N,
                     int64_t K, int epilogue, int64_t interleave, const uint16_t* res, int64_t ldr,
                     const uint16_t* rms_w, float eps, uint16_t* out, int64_t ldo, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream) {
  int rc = check_linear("linear_bf16", x, M, N, K, epilogue, res, ldr, rms_w, out, ldo);
  if (rc) return rc;
  const int64_t need = w8a8_linear_workspace_bytes(M, N, K);
  if (need < 0) return fail(W8A8_EINVAL, "linear_bf16: bad shape");
  if (M == 0) return W8A8_OK;
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256 != 0)
    return fail(W8A8_EINVAL, "linear_bf16: workspace needs %lld bytes, 256-byte aligned", (long long)need);
  char* base = static_cast<char*>(workspace);
  int8_t* q = reinterpret_cast<int8_t*>(base);
  float* sx = reinterpret_cast<float*>(base + align256(w8a8_packed_act_bytes(M, K)));
  return run_linear(x, ldx, w_packed, sw, M, N, K, epilogue, interleave, res, ldr, rms_w, eps, out, ldo, q, sx,
                    stream);
}

int w8a8_linear_bf16_noalloc(const uint16_t* x, int64_t ldx, const int8_t* w_packed, const float* sw, int64_t M,
                             int64_t N, int64_t K, int epilogue, int64_t interleave, const uint16_t* res, int64_t ldr,
                             const uint16_t* rms_w, float eps, uint16_t* out, int64_t ldo, hipStream_t stream) {
  int rc = check_linear("linear_bf16_noalloc", x, M, N, K, epilogue, res, ldr, rms_w, out, ldo);
  if (rc) return rc;
  if (M == 0) return W8A8_OK;
  const int64_t abytes = align256(w8a8_packed_act_bytes(M, K));
  const int64_t need = abytes + align256(M * 4);
  if (need > kNoAllocScratchBytes)
    return fail(W8A8_ENOTSUP,
                "linear_bf16_noalloc: M=%lld rows of K=%lld need %lld bytes of scratch, more than the library's "
                "%lld (%lld MiB); split the rows or call w8a8_linear_bf16 with a workspace",
                (long long)M, (long long)K, (long long)need, (long long)kNoAllocScratchBytes,
                (long long)(kNoAllocScratchBytes >> 20));
  void* base = nullptr;
  rc = scratch_of_current_device(&base);
  if (rc) return rc;
  int8_t* q = static_cast<int8_t*>(base);
  float* sx = reinterpret_cast<float*>(static_cast<char*>(base) + abytes);
  return run_linear(x, ldx, w_packed, sw, M, N, K, epilogue, interleave, res, ldr, rms_w, eps, out, ldo, q, sx,
                    stream);
}

}  // extern "C"
