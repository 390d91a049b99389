// Shared device/host helpers for the W8A8 engine (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// ---- bf16 <-> fp32 --------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// Round to nearest even; NaN stays NaN (torch's .to(torch.bfloat16)).  One v_cvt_pk_bf16_f32 on
// gfx950; checked against the bit-level round-half-even form over all 2^32 fp32 inputs.
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const v2bf v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// bf16(x) as fp32: the value x rounds to.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---- raw buffer loads -----------------------------------------------------------------------
// A raw buffer resource over [base, base + bytes).  Loads whose byte offset is at or past
// `bytes` return zero instead of touching memory, which is how the kernels read ragged M / N
// edges without a branch.  Word 3 (0x00020000) is the gfx9-family raw-buffer format word.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// ---- wave reductions (wave64) --------------------------------------------------------------
// Row absmax as torch.amax(|x|) computes it (pipeline.py:51): NaN propagates.  For sign-cleared
// fp32 bit patterns the unsigned order is the numeric order with every NaN above +Inf, so an
// unsigned max of |x| keeps a NaN where fmaxf would drop it.  Every input is an |x| (or 0).
__device__ __forceinline__ float absmax2(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

__device__ __forceinline__ float wave_absmax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = absmax2(v, __shfl_xor(v, o, 64));
  return v;
}
// Wave absmax (as absmax2) of v broadcast to every lane, through DPP lane moves (no LDS round
// trips): butterflies inside each row of 16 lanes, then row_bcast:15 / row_bcast:31 carry the row
// maxima up to lane 63, which is read back as a scalar.
__device__ __forceinline__ float wave_absmax_dpp(float v) {
  auto dpp = [](float x, int ctrl) {
    const int xi = __builtin_bit_cast(int, x);
    switch (ctrl) {
      case 0xB1: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0xB1, 0xF, 0xF, false));
      case 0x4E: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x4E, 0xF, 0xF, false));
      case 0x141: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x141, 0xF, 0xF, false));
      case 0x140: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x140, 0xF, 0xF, false));
      case 0x142: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x142, 0xA, 0xF, false));
      default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x143, 0xC, 0xF, false));
    }
  };
  v = absmax2(v, dpp(v, 0xB1));   // quad_perm [1,0,3,2]
  v = absmax2(v, dpp(v, 0x4E));   // quad_perm [2,3,0,1]
  v = absmax2(v, dpp(v, 0x141));  // row_half_mirror: 8 lanes
  v = absmax2(v, dpp(v, 0x140));  // row_mirror: 16 lanes
  v = absmax2(v, dpp(v, 0x142));  // row_bcast:15 into rows 1, 3
  v = absmax2(v, dpp(v, 0x143));  // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Wave sum broadcast to every lane: butterflies inside each row of 16 lanes, then row_bcast:15 /
// row_bcast:31 carry the row sums up to lane 63.  Rows a broadcast step leaves out add 0.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  auto dpp = [](float x, int ctrl) {
    const int xi = __builtin_bit_cast(int, x);
    switch (ctrl) {
      case 0xB1: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0xB1, 0xF, 0xF, false));
      case 0x4E: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x4E, 0xF, 0xF, false));
      case 0x141: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x141, 0xF, 0xF, false));
      case 0x140: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x140, 0xF, 0xF, false));
      case 0x142: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x142, 0xA, 0xF, false));
      default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x143, 0xC, 0xF, false));
    }
  };
  v += dpp(v, 0xB1);   // quad_perm [1,0,3,2]
  v += dpp(v, 0x4E);   // quad_perm [2,3,0,1]
  v += dpp(v, 0x141);  // row_half_mirror: 8 lanes
  v += dpp(v, 0x140);  // row_mirror: 16 lanes
  v += dpp(v, 0x142);  // row_bcast:15 into rows 1, 3
  v += dpp(v, 0x143);  // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ void unpack8(v4u u, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(u[i] << 16);
    v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ v4u pack8(const float (&v)[8]) {
  return v4u{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}

template <int E>
__device__ __forceinline__ void load_bf16(const uint16_t* p, float (&o)[E]) {
  if constexpr (E == 4) {
    const v2u a = *reinterpret_cast<const v2u*>(p);
    o[0] = __uint_as_float(a[0] << 16); o[1] = __uint_as_float(a[0] & 0xffff0000u);
    o[2] = __uint_as_float(a[1] << 16); o[3] = __uint_as_float(a[1] & 0xffff0000u);
  } else if constexpr (E == 2) {
    const uint32_t a = *reinterpret_cast<const uint32_t*>(p);
    o[0] = __uint_as_float(a << 16); o[1] = __uint_as_float(a & 0xffff0000u);
  } else {
    o[0] = bf16_to_f32(*p);
  }
}
template <int E>
__device__ __forceinline__ void store_bf16(uint16_t* p, const float (&o)[E]) {
  if constexpr (E == 4) {
    *reinterpret_cast<v2u*>(p) = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  } else if constexpr (E == 2) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(o[0], o[1]);
  } else {
    *p = f32_to_bf16(o[0]);
  }
}

// One head of k_qkv (pipeline.py:72-86) on one wave, in place: the lane holds E = D/128 values of
// each half of the head, at p0 .. p0+E-1 (y1) and p0+D/2 .. (y2).  RMS norm over the head with the
// weight halves w1 / w2 (has_w false: no weight), each value rounded to bf16; then, with rope, RoPE
// with the cos / sin halves c1, c2 / s1, s2 on the bf16 values: x * cos + cat(-x[D/2:], x[:D/2]) * sin
// with every product and the sum rounded (pipeline.py:60-63).  The rotation pairs element d with
// d + D/2, so it needs no lane exchange.  The operands come in registers, so a caller can fetch them
// early.
template <int E>
__device__ __forceinline__ void qkv_head_regs(float (&y1)[E], float (&y2)[E], float eps, bool has_w,
                                              const float (&w1)[E], const float (&w2)[E], bool rope,
                                              const float (&c1)[E], const float (&c2)[E], const float (&s1)[E],
                                              const float (&s2)[E]) {
  constexpr int D = 128 * E;
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += y1[e] * y1[e] + y2[e] * y2[e];
  ss = wave_sum_dpp(ss);
  const float r = 1.0f / sqrtf(ss / float(D) + eps);
  if (has_w) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      y1[e] = round_bf16((y1[e] * r) * w1[e]);
      y2[e] = round_bf16((y2[e] * r) * w2[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      y1[e] = round_bf16(y1[e] * r);
      y2[e] = round_bf16(y2[e] * r);
    }
  }
  if (rope) {
    float o1[E], o2[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      o1[e] = round_bf16(round_bf16(y1[e] * c1[e]) + round_bf16(-y2[e] * s1[e]));
      o2[e] = round_bf16(round_bf16(y2[e] * c2[e]) + round_bf16(y1[e] * s2[e]));
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      y1[e] = o1[e];
      y2[e] = o2[e];
    }
  }
}

// qkv_head_regs with its operands fetched here: the norm weight w (null: none) and, with cr / sr
// non-null, the RoPE cos / sin rows.
template <int E>
__device__ __forceinline__ void qkv_head(float (&y1)[E], float (&y2)[E], float eps, const uint16_t* w,
                                         const uint16_t* cr, const uint16_t* sr, int p0) {
  constexpr int HALF = 64 * E;
  float w1[E], w2[E], c1[E], c2[E], s1[E], s2[E];
#pragma unroll
  for (int e = 0; e < E; ++e) w1[e] = w2[e] = c1[e] = c2[e] = s1[e] = s2[e] = 0.0f;
  if (w) {
    load_bf16<E>(w + p0, w1);
    load_bf16<E>(w + p0 + HALF, w2);
  }
  if (cr) {
    load_bf16<E>(cr + p0, c1);
    load_bf16<E>(cr + p0 + HALF, c2);
    load_bf16<E>(sr + p0, s1);
    load_bf16<E>(sr + p0 + HALF, s2);
  }
  qkv_head_regs<E>(y1, y2, eps, w != nullptr, w1, w2, cr != nullptr, c1, c2, s1, s2);
}

// ---- per-row int8 quantisation step (pipeline.py:51) -----------------------------------------
// s = amax.clamp(min=1e-8) / 127 from a row absmax (pipeline.py:51); a NaN absmax stays NaN, as
// torch's clamp keeps it.
__device__ __forceinline__ float quant_scale(float amax) {
  return (amax != amax ? amax : fmaxf(amax, 1e-8f)) / 127.0f;
}

// clamp(r, +-127) -> int8, with NaN -> 0: torch's float -> int8 conversion on the host gives 0
// for NaN, which is what a row holding NaN (scale NaN) or +-Inf (scale Inf, Inf / Inf) quantises
// to in the reference (fminf / fmaxf alone would turn NaN into -127).
__device__ __forceinline__ int8_t clamp_q(float r) {
  return r != r ? int8_t(0) : int8_t(int(fminf(fmaxf(r, -127.0f), 127.0f)));
}

// q = clamp(rint(v / s), +-127): IEEE fp32 division, round half to even.
__device__ __forceinline__ int8_t quant1(float v, float s) { return clamp_q(__builtin_rintf(v / s)); }

// The same q for a bf16-valued v with |v| <= 127 s (every element of the row the scale was taken
// from), without a division per element: rs = 1 / s (IEEE, once per row), q0 = v * rs,
// r = fma(-q0, s, v) (exact), q1 = fma(r, rs, q0).  q1 may differ from the IEEE quotient v / s in
// its last bit, but rint(q1) == rint(v / s) for every bf16 absmax a (s = max(a, 1e-8) / 127) and
// every bf16 v with |v| <= a: all 1.07e9 such pairs were compared, and the library's self-check
// (w8a8_selfcheck_quant_step) repeats that comparison on the GPU.
__device__ __forceinline__ int8_t quant1_bf16(float v, float s, float rs) {
  const float q0 = v * rs;
  const float r = __builtin_fmaf(-q0, s, v);
  const float q1 = __builtin_fmaf(r, rs, q0);
  return clamp_q(__builtin_rintf(q1));
}

// ---- XCD-aware block order ---------------------------------------------------------------------
// Workgroups are dealt to the 8 XCDs round-robin (block b runs on XCD b % 8), each XCD with its
// own L2.  xcd_remap(b) gives each XCD a contiguous run of logical indices (the last nblocks % 8
// blocks keep their own index).
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
  const int full = nblocks & ~7;
  if (b >= full) return b;
  const int per = full >> 3;
  return (b & 7) * per + (b >> 3);
}

// ---- packed activations ----------------------------------------------------------------------
// The GEMM reads A fastest when it is laid out like the packed weight: 1 KiB fragments of 32
// rows x 32 k, fragment (mt, j) at (mt * KF + j) * 1024 with KF = 2 * ceil(K/64), byte 16*l + b
// of it = row 32*mt + l%32, k 32*j + 16*(l/32) + b.  Rows up to the next multiple of 32 and k up
// to the next multiple of 64 are zero.

__device__ __forceinline__ uint32_t packed_act_offset(int row, int k, int KF) {
  const int lane = (row & 31) + 32 * ((k >> 4) & 1);
  return (uint32_t(row >> 5) * uint32_t(KF) + uint32_t(k >> 5)) * 1024u + uint32_t(lane) * 16u;
}

// ---- GELU ------------------------------------------------------------------------------------
// tanh(u) in fp32 as 1 - 2 / (1 + e^(2|u|)) with the sign of u.  What matters downstream is
// 1 + tanh(u) (gelu below): for u << 0 that is the cancellation 1 - fl(1 - d), d = 2 / (1 + e^(2|u|)),
// which lands on the fp32 grid just below 1 exactly where a correctly rounded tanhf does, as long as
// d carries a small *relative* error.  Here d has ~1e-6 relative error (hardware exp2 / rcp), so
// 1 + tanh(u) matches the correctly rounded form except within ~1e-6 of a rounding tie; for
// |u| > 9.01 fl(1 - d) is exactly 1 and tanh saturates to +-1 as tanhf does.
__device__ __forceinline__ float tanh_f32(float u) {
  const float a = fabsf(u);
  const float e = __builtin_amdgcn_exp2f(a * 2.8853900817779268f);  // e^(2a) = 2^(2a log2 e)
  const float d = 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
  return copysignf(1.0f - d, u);
}

// GELU, tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), evaluated in the operation
// order of torch's gelu(approximate="tanh") on float: x^3 = (x * x) * x, inner = beta * (x +
// kappa * x^3), result = (0.5 * x) * (1 + tanh(inner)).
__device__ __forceinline__ float gelu_tanh_f32(float x) {
  const float kBeta = 0.7978845608028654f;
  const float kKappa = 0.044715f;
  const float inner = kBeta * (x + kKappa * (x * x * x));
  return 0.5f * x * (1.0f + tanh_f32(inner));
}

// Decode attention chunks: keys per chunk (32 at head_dim 512, so that two workgroups fit in a CU's
// LDS), and the chunks a launch covers per KV head for a cache of Tk rows (the last `window` of
// them with a window).  Both the attention and the GEMV that merges its chunks use these.
__host__ __device__ constexpr int dec_chunk(int D) { return D >= 512 ? 32 : 64; }
inline int decode_grid_chunks(int64_t D, int64_t Tk, int64_t window) {
  const int64_t span = window > 0 && window < Tk ? window : Tk;
  return int((span - 1) / dec_chunk(int(D)) + 1);
}
// At most this many chunks are merged inside the o GEMV (w8a8_gemv_packed_attn_merge_bf16).
constexpr int DEC_MERGE_IN_GEMV_CHUNKS = 16;

// Status codes and the extern "C" declarations every source implements.
#include "w8a8.h"

namespace w8a8 {
// Host side: record a message for w8a8_last_error() (thread-local) and return `code`.
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
// Packed weight size in bytes, or -1 for an invalid shape / interleave.
int64_t w8a8_packed_weight_bytes_internal(int64_t N, int64_t K, int64_t interleave);
}  // namespace w8a8
