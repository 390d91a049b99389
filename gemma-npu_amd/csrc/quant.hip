// Per-row int8 quantisation and weight packing.
//
// quant_rows: one wave per row.  s = max(amax(|x|), 1e-8) / 127 and
// q = clamp(rint(x / s), -127, 127) with an IEEE (correctly rounded) fp32 divide and
// round-half-even, the arithmetic of pipeline.py:49-52 / gemma_npu.py:37-42 and, applied to
// weight rows, of the per-output-channel weight quant at gemma_npu.py:68-69.
//
// pack_weight: rewrites an int8 weight into the GEMM's resident layout of 1 KiB MFMA
// fragments.  Fragment (t, j) holds output channels [32t, 32t+32) x inputs [32j, 32j+32);
// byte 16*l + b of it is channel 32t + l%32, input 32j + 16*(l/32) + b, i.e. exactly the
// 16 bytes lane l feeds to v_mfma_i32_32x32x32_i8.  Fragments are stored tile-major
// ((t * KF + j) * 1024) with K zero-padded to a multiple of 64 (KF = 2 * ceil(K/64)) and N to
// a multiple of 32.  With `interleave` = I > 0 the tiles alternate gate / up: tile 2u is
// channels [32u, 32u+32) and tile 2u+1 is channels [I+32u, I+32u+32), so a lane holds
// matching gate and up accumulators for the fused GELU epilogue.
#include "w8a8_common.h"

namespace w8a8 {

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float (&v)[8]) {
  v4u d = *reinterpret_cast<const v4u*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(d[i] << 16);
    v[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
  v4f a = *reinterpret_cast<const v4f*>(p);
  v4f b = *reinterpret_cast<const v4f*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[4 + i] = b[i];
  }
}

template <typename T>
__device__ __forceinline__ float load1(const T* p);
template <>
__device__ __forceinline__ float load1<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }
template <>
__device__ __forceinline__ float load1<float>(const float* p) { return *p; }

// VEC: rows are 16-byte aligned and K % 8 == 0, so 8 elements move per access.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void quant_rows_kernel(const T* __restrict__ x, int64_t ldx, int M, int K,
                                                         int8_t* __restrict__ q, int64_t ldq,
                                                         float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* xr = x + int64_t(row) * ldx;
  int8_t* qr = q + int64_t(row) * ldq;
  float amax = 0.0f;
  if (VEC) {
    for (int k = lane * 8; k < K; k += 512) {
      float v[8];
      load8<T>(xr + k, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = absmax2(amax, fabsf(v[i]));
    }
  } else {
    for (int k = lane; k < K; k += 64) amax = absmax2(amax, fabsf(load1<T>(xr + k)));
  }
  amax = wave_absmax(amax);
  const float s = quant_scale(amax);
  const float rs = 1.0f / s;
  if (lane == 0) scale[row] = s;
  // bf16 rows take the division-free step (exact for bf16 values); fp32 rows divide.
  auto qt = [&](float v) { return sizeof(T) == 2 ? quant1_bf16(v, s, rs) : quant1(v, s); };
  if (VEC) {
    for (int k = lane * 8; k < K; k += 512) {
      float v[8];
      load8<T>(xr + k, v);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo |= uint32_t(uint8_t(qt(v[i]))) << (8 * i);
        hi |= uint32_t(uint8_t(qt(v[4 + i]))) << (8 * i);
      }
      *reinterpret_cast<v2u*>(qr + k) = v2u{lo, hi};
    }
  } else {
    for (int k = lane; k < K; k += 64) qr[k] = qt(load1<T>(xr + k));
  }
}

// One thread per 16-byte chunk of the packed output.  src_kn: the source is [K, N] (ld = ldw,
// the reference's B layout, npu_kernels.py:46); otherwise it is [N, K] (gemma_npu.py:69).
__global__ __launch_bounds__(256) void pack_weight_kernel(const int8_t* __restrict__ w, int64_t ldw, int N, int K,
                                                          int src_kn, int interleave, int KF, int64_t nchunks,
                                                          int8_t* __restrict__ out) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const int lane = int(c & 63);
  const int64_t f = c >> 6;
  const int t = int(f / KF);
  const int j = int(f % KF);
  int n;
  int limit;
  if (interleave > 0) {
    const int u = t >> 1;
    n = (t & 1 ? interleave : 0) + 32 * u + (lane & 31);
    limit = (t & 1 ? N : interleave);
  } else {
    n = 32 * t + (lane & 31);
    limit = N;
  }
  const int k0 = 32 * j + 16 * (lane >> 5);
  uint32_t word[4] = {0, 0, 0, 0};
  if (n < limit) {
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int k = k0 + b;
      if (k < K) {
        const int8_t v = src_kn ? w[int64_t(k) * ldw + n] : w[int64_t(n) * ldw + k];
        word[b >> 2] |= uint32_t(uint8_t(v)) << (8 * (b & 3));
      }
    }
  }
  *reinterpret_cast<v4u*>(out + c * 16) = v4u{word[0], word[1], word[2], word[3]};
}

// One wave per row (padding rows included): absmax, then 16-element chunks quantised and
// stored as 16-byte vectors at their packed position.
template <bool VEC>
__global__ __launch_bounds__(256) void quant_rows_packed_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                                int Mp, int K, int KF, int8_t* __restrict__ q,
                                                                float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  // Blocks in XCD order, so the 8 rows sharing each 128-byte line of q are written in one L2.
  const int row = xcd_remap(int(blockIdx.x), int(gridDim.x)) * 4 + (threadIdx.x >> 6);
  if (row >= Mp) return;
  const int KP = KF * 32;
  if (row >= M) {
    for (int k = lane * 16; k < KP; k += 1024)
      *reinterpret_cast<v4u*>(q + packed_act_offset(row, k, KF)) = v4u{0, 0, 0, 0};
    return;
  }
  const uint16_t* xr = x + int64_t(row) * ldx;
  float amax = 0.0f;
  for (int k = lane * 16; k < K; k += 1024) {
    float v[16];
    if (VEC) {
      load8<uint16_t>(xr + k, *reinterpret_cast<float(*)[8]>(&v[0]));
      load8<uint16_t>(xr + k + 8, *reinterpret_cast<float(*)[8]>(&v[8]));
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = bf16_to_f32(xr[k + i]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = absmax2(amax, fabsf(v[i]));
  }
  amax = wave_absmax(amax);
  const float s = quant_scale(amax);
  const float rs = 1.0f / s;
  if (lane == 0) scale[row] = s;
  for (int k = lane * 16; k < KP; k += 1024) {
    uint32_t w[4] = {0, 0, 0, 0};
    if (k < K) {
      float v[16];
      if (VEC) {
        load8<uint16_t>(xr + k, *reinterpret_cast<float(*)[8]>(&v[0]));
        load8<uint16_t>(xr + k + 8, *reinterpret_cast<float(*)[8]>(&v[8]));
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = bf16_to_f32(xr[k + i]);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i >> 2] |= uint32_t(uint8_t(quant1_bf16(v[i], s, rs))) << (8 * (i & 3));
    }
    *reinterpret_cast<v4u*>(q + packed_act_offset(row, k, KF)) = v4u{w[0], w[1], w[2], w[3]};
  }
}

// Single-pass quantisation of bf16 rows held in registers: one 256-thread block per row; thread
// t holds chunks c = 0 .. CH-1 of 8 consecutive elements at k = 8 * (256c + t), all loaded in one
// burst, so the row costs one memory round trip and its quant steps are spread over four waves.
// The absmax is a DPP wave reduction plus one LDS exchange between the waves.  The int8 bytes
// leave as 8-byte stores, row-major or into the packed fragment layout (half of the 16-byte
// piece holding k: fragment (row/32, k/32), lane slot row%32 + 32 * ((k/16) % 2), byte k % 16).
// PACKED also zero-fills rows M .. Mp-1 and k K .. 32*KF-1.
template <int CH, bool PACKED>
__global__ __launch_bounds__(256) void quant_rows_blk_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                             int K, int KF, int8_t* __restrict__ q, int64_t ldq,
                                                             float* __restrict__ scale) {
  __shared__ float wave_amax[4];
  const int t = threadIdx.x;
  // Packed output: the 16-byte pieces of 8 consecutive rows share each 128-byte line, so rows
  // are dealt out XCD by XCD and every line is assembled in one L2 (round-robin rows would leave
  // a dirty eighth of every line in each of the 8 L2s).
  const int row = PACKED ? xcd_remap(int(blockIdx.x), int(gridDim.x)) : int(blockIdx.x);
  const int KP = PACKED ? KF * 32 : K;
  auto dst = [&](int k) -> int8_t* {
    if constexpr (PACKED)
      return q + packed_act_offset(row, k & ~15, KF) + (k & 15);
    else
      return q + int64_t(row) * ldq + k;
  };
  if (row >= M) {  // PACKED only: padding rows are zero
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = 8 * (256 * c + t);
      if (k < KP) *reinterpret_cast<v2u*>(dst(k)) = v2u{0u, 0u};
    }
    return;
  }
  const uint16_t* xr = x + int64_t(row) * ldx;
  v4u v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int k = 8 * (256 * c + t);
    v[c] = k < K ? *reinterpret_cast<const v4u*>(xr + k) : v4u{0u, 0u, 0u, 0u};
  }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      amax = absmax2(amax, absmax2(fabsf(__uint_as_float(v[c][i] << 16)), fabsf(__uint_as_float(v[c][i] & 0xffff0000u))));
  amax = wave_absmax_dpp(amax);
  if ((t & 63) == 0) wave_amax[t >> 6] = amax;
  __syncthreads();
  amax = absmax2(absmax2(wave_amax[0], wave_amax[1]), absmax2(wave_amax[2], wave_amax[3]));
  const float s = quant_scale(amax);
  const float rs = 1.0f / s;
  if (t == 0) scale[row] = s;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int k = 8 * (256 * c + t);
    if (k >= KP) continue;
    uint32_t w[2] = {0u, 0u};
    if (k < K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = uint8_t(quant1_bf16(__uint_as_float(v[c][i] << 16), s, rs));
        const uint32_t hi = uint8_t(quant1_bf16(__uint_as_float(v[c][i] & 0xffff0000u), s, rs));
        w[i >> 1] |= (lo | (hi << 8)) << (16 * (i & 1));
      }
    }
    *reinterpret_cast<v2u*>(dst(k)) = v2u{w[0], w[1]};
  }
}

// Launch the block-per-row kernel for K <= 8 * 256 * 6 = 12288; false if K is beyond it.
template <bool PACKED>
static bool launch_quant_reg(const uint16_t* x, int64_t ldx, int M, int Mp, int K, int KF, int8_t* q, int64_t ldq,
                             float* scale, hipStream_t stream) {
  const int ch = (K + 2047) / 2048;
  const dim3 grid{static_cast<unsigned>(Mp)};
#define W8A8_QBLK(N) quant_rows_blk_kernel<N, PACKED><<<grid, 256, 0, stream>>>(x, ldx, M, K, KF, q, ldq, scale)
  if (ch <= 1) W8A8_QBLK(1);
  else if (ch <= 2) W8A8_QBLK(2);
  else if (ch <= 3) W8A8_QBLK(3);
  else if (ch <= 4) W8A8_QBLK(4);
  else if (ch <= 6) W8A8_QBLK(6);
  else return false;
#undef W8A8_QBLK
  return true;
}

// Row-major int8 A -> packed activations; one thread per 16-byte chunk of the output.
__global__ __launch_bounds__(256) void pack_act_kernel(const int8_t* __restrict__ a, int64_t lda, int M, int K, int KF,
                                                       int64_t nchunks, int8_t* __restrict__ out) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const int l = int(c & 63);
  const int64_t f = c >> 6;
  const int mt = int(f / KF), j = int(f % KF);
  const int row = 32 * mt + (l & 31);
  const int k = 32 * j + 16 * (l >> 5);
  v4u v = {0, 0, 0, 0};
  if (row < M && k < K) v = *reinterpret_cast<const v4u*>(a + int64_t(row) * lda + k);
  *reinterpret_cast<v4u*>(out + c * 16) = v;
}

// Self-check of quant1_bf16 against the IEEE-division form: one block per positive finite bf16
// absmax a, its threads walking every bf16 v with |v| <= a.  counts[0] += pairs whose int8 codes
// differ, counts[1] += pairs compared (1,065,402,240 in all).
__global__ __launch_bounds__(256) void selfcheck_quant_step_kernel(unsigned long long* counts) {
  const float a = bf16_to_f32(uint16_t(blockIdx.x));
  const float s = fmaxf(a, 1e-8f) / 127.0f;
  const float rs = 1.0f / s;
  int bad = 0, n = 0;
  for (int vh = int(threadIdx.x); vh < 65536; vh += 256) {
    const float v = bf16_to_f32(uint16_t(vh));
    if (!(fabsf(v) <= a)) continue;
    ++n;
    bad += quant1_bf16(v, s, rs) != quant1(v, s);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    bad += __shfl_xor(bad, o, 64);
    n += __shfl_xor(n, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(counts, (unsigned long long)bad);
    atomicAdd(counts + 1, (unsigned long long)n);
  }
}

}  // namespace w8a8

using namespace w8a8;

extern "C" {

int w8a8_quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq,
                         float* scale, hipStream_t stream) {
  if (M < 0 || K <= 0 || ldx < K || ldq < K) return fail(W8A8_EINVAL, "quant_rows: bad shape M=%lld K=%lld ldx=%lld ldq=%lld",
                                                         (long long)M, (long long)K, (long long)ldx, (long long)ldq);
  if (!x || !q || !scale) return fail(W8A8_EINVAL, "quant_rows: null pointer");
  if (M == 0) return W8A8_OK;
  if (M > INT32_MAX / 4 || K > INT32_MAX) return fail(W8A8_ENOTSUP, "quant_rows: too large");
  const bool vec = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                   ((uintptr_t)q % 8 == 0);
  if (vec && launch_quant_reg<false>(x, ldx, int(M), int(M), int(K), 0, q, ldq, scale, stream))
    return check_launch("quant_rows_bf16");
  dim3 grid((unsigned)((M + 3) / 4));
  if (vec)
    quant_rows_kernel<uint16_t, true><<<grid, 256, 0, stream>>>(x, ldx, (int)M, (int)K, q, ldq, scale);
  else
    quant_rows_kernel<uint16_t, false><<<grid, 256, 0, stream>>>(x, ldx, (int)M, (int)K, q, ldq, scale);
  return check_launch("quant_rows_bf16");
}

int w8a8_quant_rows_f32(const float* x, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq, float* scale,
                        hipStream_t stream) {
  if (M < 0 || K <= 0 || ldx < K || ldq < K) return fail(W8A8_EINVAL, "quant_rows_f32: bad shape");
  if (!x || !q || !scale) return fail(W8A8_EINVAL, "quant_rows_f32: null pointer");
  if (M == 0) return W8A8_OK;
  if (M > INT32_MAX / 4 || K > INT32_MAX) return fail(W8A8_ENOTSUP, "quant_rows_f32: too large");
  const bool vec = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                   ((uintptr_t)q % 8 == 0);
  dim3 grid((unsigned)((M + 3) / 4));
  if (vec)
    quant_rows_kernel<float, true><<<grid, 256, 0, stream>>>(x, ldx, (int)M, (int)K, q, ldq, scale);
  else
    quant_rows_kernel<float, false><<<grid, 256, 0, stream>>>(x, ldx, (int)M, (int)K, q, ldq, scale);
  return check_launch("quant_rows_f32");
}

int64_t w8a8_packed_weight_bytes(int64_t N, int64_t K, int64_t interleave) {
  return w8a8_packed_weight_bytes_internal(N, K, interleave);
}

static int pack_common(const int8_t* w, int64_t ldw, int64_t N, int64_t K, int src_kn, int64_t interleave,
                       int8_t* packed, hipStream_t stream) {
  if (!w || !packed) return fail(W8A8_EINVAL, "pack_weight: null pointer");
  if (N <= 0 || K <= 0) return fail(W8A8_EINVAL, "pack_weight: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  if (src_kn ? ldw < N : ldw < K) return fail(W8A8_EINVAL, "pack_weight: leading dimension %lld too small", (long long)ldw);
  if (interleave > 0 && (interleave % 32 != 0 || N != 2 * interleave))
    return fail(W8A8_EINVAL, "pack_weight: interleave %lld needs N == 2*I and I %% 32 == 0 (N=%lld)",
                (long long)interleave, (long long)N);
  if ((uintptr_t)packed % 16 != 0) return fail(W8A8_EALIGN, "pack_weight: packed buffer not 16-byte aligned");
  const int64_t bytes = w8a8_packed_weight_bytes_internal(N, K, interleave);
  if (bytes > INT32_MAX) return fail(W8A8_ENOTSUP, "pack_weight: packed weight of %lld bytes exceeds 2 GiB", (long long)bytes);
  const int KF = int(2 * ((K + 63) / 64));
  const int64_t nchunks = bytes / 16;
  dim3 grid((unsigned)((nchunks + 255) / 256));
  pack_weight_kernel<<<grid, 256, 0, stream>>>(w, ldw, (int)N, (int)K, src_kn, (int)interleave, KF, nchunks, packed);
  return check_launch("pack_weight");
}

int w8a8_pack_weight_nk(const int8_t* w_nk, int64_t ldw, int64_t N, int64_t K, int64_t interleave, int8_t* packed,
                        hipStream_t stream) {
  return pack_common(w_nk, ldw, N, K, 0, interleave, packed, stream);
}

int w8a8_pack_weight_kn(const int8_t* b_kn, int64_t ldb, int64_t K, int64_t N, int64_t interleave, int8_t* packed,
                        hipStream_t stream) {
  return pack_common(b_kn, ldb, N, K, 1, interleave, packed, stream);
}

int64_t w8a8_packed_act_bytes(int64_t M, int64_t K) {
  if (M < 0 || K <= 0) return -1;
  return (M + 31) / 32 * 2 * ((K + 63) / 64) * 1024;
}

int w8a8_pack_act(const int8_t* a, int64_t lda, int64_t M, int64_t K, int8_t* packed, hipStream_t stream) {
  if (M < 0 || K <= 0 || lda < K) return fail(W8A8_EINVAL, "pack_act: bad shape M=%lld K=%lld lda=%lld", (long long)M,
                                               (long long)K, (long long)lda);
  if (M == 0) return W8A8_OK;
  if (!a || !packed) return fail(W8A8_EINVAL, "pack_act: null pointer");
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "pack_act: K=%lld must be a multiple of 16", (long long)K);
  if (lda % 16 != 0 || (uintptr_t)a % 16 != 0 || (uintptr_t)packed % 16 != 0)
    return fail(W8A8_EALIGN, "pack_act: rows and the packed buffer must be 16-byte aligned");
  const int64_t bytes = w8a8_packed_act_bytes(M, K);
  if (bytes > INT32_MAX || M > INT32_MAX) return fail(W8A8_ENOTSUP, "pack_act: too large");
  const int KF = int(2 * ((K + 63) / 64));
  const int64_t nchunks = bytes / 16;
  pack_act_kernel<<<unsigned((nchunks + 255) / 256), 256, 0, stream>>>(a, lda, int(M), int(K), KF, nchunks, packed);
  return check_launch("pack_act");
}

int w8a8_quant_rows_packed_bf16(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* packed, float* scale,
                                hipStream_t stream) {
  if (M < 0 || K <= 0 || ldx < K) return fail(W8A8_EINVAL, "quant_rows_packed: bad shape M=%lld K=%lld ldx=%lld",
                                               (long long)M, (long long)K, (long long)ldx);
  if (M == 0) return W8A8_OK;
  if (!x || !packed || !scale) return fail(W8A8_EINVAL, "quant_rows_packed: null pointer");
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "quant_rows_packed: K=%lld must be a multiple of 16", (long long)K);
  if ((uintptr_t)packed % 16 != 0) return fail(W8A8_EALIGN, "quant_rows_packed: packed buffer not 16-byte aligned");
  const int64_t bytes = w8a8_packed_act_bytes(M, K);
  if (bytes > INT32_MAX || M > INT32_MAX / 4) return fail(W8A8_ENOTSUP, "quant_rows_packed: too large");
  const int KF = int(2 * ((K + 63) / 64));
  const int Mp = int((M + 31) / 32 * 32);
  const bool vec = (ldx % 8 == 0) && ((uintptr_t)x % 16 == 0);
  if (vec && launch_quant_reg<true>(x, ldx, int(M), Mp, int(K), KF, packed, 0, scale, stream))
    return check_launch("quant_rows_packed_bf16");
  dim3 grid(unsigned((Mp + 3) / 4));
  if (vec)
    quant_rows_packed_kernel<true><<<grid, 256, 0, stream>>>(x, ldx, int(M), Mp, int(K), KF, packed, scale);
  else
    quant_rows_packed_kernel<false><<<grid, 256, 0, stream>>>(x, ldx, int(M), Mp, int(K), KF, packed, scale);
  return check_launch("quant_rows_packed_bf16");
}

int w8a8_selfcheck_quant_step(unsigned long long* counts, hipStream_t stream) {
  if (!counts) return fail(W8A8_EINVAL, "selfcheck_quant_step: null counts");
  if ((uintptr_t)counts % 8 != 0) return fail(W8A8_EALIGN, "selfcheck_quant_step: counts must be 8-byte aligned");
  selfcheck_quant_step_kernel<<<0x7f80, 256, 0, stream>>>(counts);
  return check_launch("selfcheck_quant_step");
}

}  // extern "C"
