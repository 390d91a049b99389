// Row-wise element-wise kernels around the GEMM.
//
// dequant_bf16:   out = bf16((float(acc) * sx[m]) * sw[n])          (_deq, pipeline.py:55-57;
//                                                                    _dequant, gemma_npu.py:45-47)
// rms_residual:   h = bf16(res + bf16(y * (mean(y^2) + eps)^-0.5 * w)) and, optionally, the int8
//                 rows + scale of h for the next GEMM                (k_post_ff, pipeline.py:110-114;
//                                                                    _rms, pipeline.py:43-46)
// One wave per row for rms_residual (the row statistic is a wave reduction); the reduction
// order differs from torch's, so h agrees to fp32 rounding, not bit for bit.
#include "w8a8_common.h"

namespace w8a8 {

__global__ __launch_bounds__(256) void dequant_kernel(const int32_t* __restrict__ acc, int64_t ldacc,
                                                      const float* __restrict__ sx, const float* __restrict__ sw,
                                                      int M, int N, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= int64_t(M) * N) return;
  const int m = int(i / N), n = int(i % N);
  const float v = (float(acc[int64_t(m) * ldacc + n]) * sx[m]) * sw[n];
  out[int64_t(m) * ldo + n] = f32_to_bf16(v);
}

__global__ __launch_bounds__(256) void rms_residual_kernel(const uint16_t* y, int64_t ldy,
                                                           const uint16_t* __restrict__ res, int64_t ldr,
                                                           const uint16_t* __restrict__ w, float eps, int M, int N,
                                                           uint16_t* h, int64_t ldh, int8_t* __restrict__ q,
                                                           int64_t ldq, float* __restrict__ sq) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* yr = y + int64_t(row) * ldy;
  const uint16_t* rr = res + int64_t(row) * ldr;
  uint16_t* hr = h + int64_t(row) * ldh;
  float ss = 0.0f;
  for (int n = lane; n < N; n += 64) {
    const float v = bf16_to_f32(yr[n]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float rs = 1.0f / sqrtf(ss / float(N) + eps);
  float amax = 0.0f;
  // h may alias y: every y value of the row has been read above; each element is read
  // before its own h is written below.
  for (int n = lane; n < N; n += 64) {
    float v = bf16_to_f32(yr[n]) * rs;
    if (w) v = v * bf16_to_f32(w[n]);
    const float nb = bf16_to_f32(f32_to_bf16(v));
    const uint16_t hb = f32_to_bf16(bf16_to_f32(rr[n]) + nb);
    hr[n] = hb;
    amax = fmaxf(amax, fabsf(bf16_to_f32(hb)));
  }
  if (!q) return;
  amax = wave_max(amax);
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
  if (lane == 0) sq[row] = s;
  int8_t* qr = q + int64_t(row) * ldq;
  for (int n = lane; n < N; n += 64) {
    float r = __builtin_rintf(bf16_to_f32(hr[n]) / s);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    qr[n] = int8_t(int(r));
  }
}

}  // namespace w8a8

using namespace w8a8;

extern "C" {

int w8a8_dequant_bf16(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, int64_t M, int64_t N,
                      uint16_t* out, int64_t ldo, hipStream_t stream) {
  if (!acc || !sx || !sw || !out) return fail(W8A8_EINVAL, "dequant: null pointer");
  if (M < 0 || N <= 0 || ldacc < N || ldo < N) return fail(W8A8_EINVAL, "dequant: bad shape");
  if (M == 0) return W8A8_OK;
  const int64_t total = M * N;
  if (total > INT32_MAX || M > INT32_MAX || N > INT32_MAX) return fail(W8A8_ENOTSUP, "dequant: too large");
  dequant_kernel<<<unsigned((total + 255) / 256), 256, 0, stream>>>(acc, ldacc, sx, sw, int(M), int(N), out, ldo);
  return check_launch("dequant_bf16");
}

int w8a8_rms_residual_bf16(const uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldr, const uint16_t* w,
                           float eps, int64_t M, int64_t N, uint16_t* h, int64_t ldh, int8_t* q, int64_t ldq,
                           float* sq, hipStream_t stream) {
  if (!y || !res || !h) return fail(W8A8_EINVAL, "rms_residual: null pointer");
  if ((q == nullptr) != (sq == nullptr)) return fail(W8A8_EINVAL, "rms_residual: q and its scale go together");
  if (M < 0 || N <= 0 || ldy < N || ldr < N || ldh < N || (q && ldq < N))
    return fail(W8A8_EINVAL, "rms_residual: bad shape");
  if (M == 0) return W8A8_OK;
  if (M > INT32_MAX / 4 || N > INT32_MAX) return fail(W8A8_ENOTSUP, "rms_residual: too large");
  rms_residual_kernel<<<unsigned((M + 3) / 4), 256, 0, stream>>>(y, ldy, res, ldr, w, eps, int(M), int(N), h, ldh, q,
                                                                 ldq, sq);
  return check_launch("rms_residual_bf16");
}

}  // extern "C"
