// Row-wise kernels between the GEMMs: the reference's fused CPU kernels (pipeline.py:43-127) on
// the GPU.
//
// dequant_bf16    out = bf16((float(acc) * sx[m]) * sw[n])            (_deq, pipeline.py:55-57;
//                                                                      _dequant, gemma_npu.py:45-47)
// row chain       one block per row runs, on the row held in registers:
//                   load    y = the bf16 row, or bf16((acc * sx) * sw) from an int32 GEMM result
//                   op      GELU_MUL  y = bf16(bf16(gelu_tanh(y)) * up)
//                           NORM_RES  y = bf16(res + bf16(rms(y) * w1))
//                   scale   y = bf16(y * scalar)
//                   store   h = y
//                   norm2   u = bf16(rms(y) * w2), else u = y
//                   quant   q, s = _quant(u), row-major or in the GEMM's packed layout
//                 which covers k_in, k_attn_out, k_post_attn, k_gelu, k_post_ff, k_ple_gate and
//                 k_ple_out (pipeline.py:66-127).
// qkv             k_qkv (pipeline.py:72-85): per (token, head) dequant, RMSNorm over the head,
//                 rotary embedding, written head-major [heads, T, D].
//
// Every entry point that takes an int32 GEMM result with its scales has a `_y` twin that takes the
// dequantised bf16 rows instead -- what the GEMM's dequant epilogue writes, bf16((acc * sx) * sw),
// the same values the int32 entry computes first -- so a GEMM feeding these kernels can write half
// the bytes and the results are bit-identical.
//
// rms(x) = x * (mean(x^2) + eps)^-0.5 * w in fp32 (_rms, pipeline.py:43-46).  Every bf16 rounding
// the eager torch ops perform is performed here too; the row sums of squares are added in a
// different order than torch's, so normalised values agree to fp32 rounding, not bit for bit.
#include "w8a8_common.h"

namespace w8a8 {

typedef int v2i __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(256) void dequant_kernel(const int32_t* __restrict__ acc, int64_t ldacc,
                                                      const float* __restrict__ sx, const float* __restrict__ sw,
                                                      int M, int N, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= int64_t(M) * N) return;
  const int m = int(i / N), n = int(i % N);
  const float v = (float(acc[int64_t(m) * ldacc + n]) * sx[m]) * sw[n];
  out[int64_t(m) * ldo + n] = f32_to_bf16(v);
}

// Sum (or maximum) over a block of blockDim.x / 64 <= 4 waves, returned to every thread.  `slot`
// is 4 floats of LDS used by this reduction only.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* slot) {
  v = MAX ? wave_absmax_dpp(v) : wave_sum_dpp(v);
  const int nw = int(blockDim.x >> 6);
  if (nw == 1) return v;
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = slot[0];
  for (int i = 1; i < nw; ++i) r = MAX ? absmax2(r, slot[i]) : r + slot[i];
  return r;
}

enum RowOp { RC_NONE = 0, RC_GELU_MUL = 1, RC_NORM_RES = 2 };

struct RowChain {
  const void* in; int64_t ld_in;        // int32 GEMM result (dequantised with sx, sw) or bf16 rows
  int64_t head_stride; int head_len;    // bf16 input: element n of a row at (n / head_len) * head_stride + n % head_len
  const float* sx; const float* sw;
  int op;                               // RowOp
  const uint16_t* aux; int64_t ld_aux;  // NORM_RES: the residual; GELU_MUL: the multiplier (null: input column N + n)
  const uint16_t* w1;                   // NORM_RES weight (null: none)
  const uint16_t* scalar;               // one bf16 multiplier applied after the op (null: none)
  uint16_t* h; int64_t ldh;             // bf16 result of op + scale (null: not stored)
  int norm2; const uint16_t* w2;        // quantise bf16(rms(y) * w2) instead of y (w2 null: no weight)
  uint16_t* h2; int64_t ldh2;           // bf16 rows of what is quantised (the second norm's output); null: not stored
  int8_t* q; int64_t ldq; int KF;       // int8 rows, row-major (KF == 0) or packed (KF = 2 * ceil(N / 64)); null: none
  float* sq;                            // per-row scales of q
  float eps; int M, N;
};

// Eight input elements at (row, col): bf16, or the dequantised int32 result rounded to bf16 as
// _deq's .to(bfloat16) rounds it.
template <bool IN_I32>
__device__ __forceinline__ void load_in8(const RowChain& p, int row, int col, float sxm, float (&v)[8]) {
  if constexpr (IN_I32) {
    const int32_t* a = static_cast<const int32_t*>(p.in) + int64_t(row) * p.ld_in + col;
    const v4i a0 = *reinterpret_cast<const v4i*>(a), a1 = *reinterpret_cast<const v4i*>(a + 4);
    const v4f s0 = *reinterpret_cast<const v4f*>(p.sw + col), s1 = *reinterpret_cast<const v4f*>(p.sw + col + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = round_bf16((float(a0[i]) * sxm) * s0[i]);
      v[4 + i] = round_bf16((float(a1[i]) * sxm) * s1[i]);
    }
  } else {
    const int64_t off = int64_t(col / p.head_len) * p.head_stride + col % p.head_len;
    unpack8(*reinterpret_cast<const v4u*>(static_cast<const uint16_t*>(p.in) + int64_t(row) * p.ld_in + off), v);
  }
}

// One block of blockDim.x (64 .. 256) threads per row; thread t holds chunks c < CH of 8
// consecutive elements at k = 8 * (blockDim.x * c + t).  Every operand of the row (input, up /
// residual, norm weights, scalar) is fetched in one burst before the first reduction, so the row
// costs one memory round trip; each statistic is then a block reduction over registers.  Rows
// M .. gridDim.x-1 exist only for the packed layout and are written as zeros, as are its columns
// N .. 32*KF-1.  OP is the RowOp (the loads it needs are fixed at compile time).
template <int CH, bool IN_I32, int OP>
__global__ __launch_bounds__(256) void row_chain_kernel(RowChain p) {
  __shared__ float red[3][4];
  const int t = threadIdx.x, nt = int(blockDim.x);
  // Packed q: 8 consecutive rows share each 128-byte line of the layout, so rows are dealt out XCD
  // by XCD and each line is assembled in one L2.
  const int row = p.KF ? xcd_remap(int(blockIdx.x), int(gridDim.x)) : int(blockIdx.x);
  const int KQ = p.KF ? p.KF * 32 : p.N;  // q columns written
  auto qdst = [&](int k) -> int8_t* {
    return p.KF ? p.q + packed_act_offset(row, k & ~15, p.KF) + (k & 15) : p.q + int64_t(row) * p.ldq + k;
  };
  if (row >= p.M) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = 8 * (nt * c + t);
      if (k < KQ) *reinterpret_cast<v2u*>(qdst(k)) = v2u{0u, 0u};
    }
    return;
  }
  const float sxm = IN_I32 ? p.sx[row] : 0.0f;
  const float scl = p.scalar ? bf16_to_f32(*p.scalar) : 1.0f;
  float v[CH][8];
  float up[OP == RC_GELU_MUL ? CH : 1][8];  // GELU_MUL multiplier
  v4u res[OP == RC_NORM_RES ? CH : 1];     // NORM_RES residual (bf16 words)
  v4u w1[OP == RC_NORM_RES ? CH : 1];      // NORM_RES weight
  v4u w2[CH];                              // second-norm weight
  const v4u one = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};  // bf16 1.0 x 8
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int k = 8 * (nt * c + t);
    const bool in = k < p.N;
    if (in) {
      load_in8<IN_I32>(p, row, k, sxm, v[c]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = 0.0f;
    }
    if constexpr (OP == RC_GELU_MUL) {
      if (in && p.aux) {
        unpack8(*reinterpret_cast<const v4u*>(p.aux + int64_t(row) * p.ld_aux + k), up[c]);
      } else if (in) {
        load_in8<IN_I32>(p, row, p.N + k, sxm, up[c]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) up[c][i] = 0.0f;
      }
    }
    if constexpr (OP == RC_NORM_RES) {
      res[c] = (in && p.aux) ? *reinterpret_cast<const v4u*>(p.aux + int64_t(row) * p.ld_aux + k) : v4u{0u, 0u, 0u, 0u};
      w1[c] = (in && p.w1) ? *reinterpret_cast<const v4u*>(p.w1 + k) : one;
    }
    w2[c] = (in && (p.q || p.h2) && p.norm2 && p.w2) ? *reinterpret_cast<const v4u*>(p.w2 + k) : one;
  }

  if constexpr (OP == RC_GELU_MUL) {
    // bf16(bf16(gelu_tanh(y)) * up): F.gelu on a bf16 tensor rounds, and so does the product
    // (pipeline.py:106, 120).
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = round_bf16(round_bf16(gelu_tanh_f32(v[c][i])) * up[c][i]);
  }
  if constexpr (OP == RC_NORM_RES) {
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[c][i] * v[c][i];
    ss = block_reduce<false>(ss, red[0]);
    const float r = 1.0f / sqrtf(ss / float(p.N) + p.eps);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float rv[8], wv[8];
      unpack8(res[c], rv);
      unpack8(w1[c], wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float n = v[c][i] * r;
        if (p.w1) n = n * wv[i];
        v[c][i] = p.aux ? round_bf16(rv[i] + round_bf16(n)) : round_bf16(n);  // no residual: the norm alone
      }
    }
  }
  if (p.scalar) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = round_bf16(v[c][i] * scl);
  }
  if (p.h) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = 8 * (nt * c + t);
      if (k < p.N) *reinterpret_cast<v4u*>(p.h + int64_t(row) * p.ldh + k) = pack8(v[c]);
    }
  }
  if (!p.q && !p.h2) return;

  if (p.norm2) {
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[c][i] * v[c][i];
    ss = block_reduce<false>(ss, red[1]);
    const float r = 1.0f / sqrtf(ss / float(p.N) + p.eps);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float wv[8];
      unpack8(w2[c], wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float n = v[c][i] * r;
        if (p.w2) n = n * wv[i];
        v[c][i] = round_bf16(n);
      }
    }
  }
  if (p.h2) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = 8 * (nt * c + t);
      if (k < p.N) *reinterpret_cast<v4u*>(p.h2 + int64_t(row) * p.ldh2 + k) = pack8(v[c]);
    }
  }
  if (!p.q) return;
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = absmax2(amax, fabsf(v[c][i]));
  amax = block_reduce<true>(amax, red[2]);
  const float s = quant_scale(amax);
  const float rs = 1.0f / s;
  if (t == 0) p.sq[row] = s;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int k = 8 * (nt * c + t);
    if (k >= KQ) continue;
    uint32_t w[2] = {0u, 0u};
    if (k < p.N) {
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i >> 2] |= uint32_t(uint8_t(quant1_bf16(v[c][i], s, rs))) << (8 * (i & 3));
    }
    *reinterpret_cast<v2u*>(qdst(k)) = v2u{w[0], w[1]};
  }
}

// ---- k_qkv ------------------------------------------------------------------------------------
struct QkvParams {
  const int32_t* acc; int64_t ldacc;      // int32 GEMM result with its scales, or
  const float* sx; const float* sw;
  const uint16_t* y; int64_t ldy;         // the dequantised bf16 rows (then acc, sx, sw are unused)
  const uint16_t* cs; const uint16_t* sn; int64_t ldcs;  // cos / sin bf16 [T, D]
  const uint16_t* qw; const uint16_t* kw;                // q_norm / k_norm weights bf16 [D]
  uint16_t* q; uint16_t* k; uint16_t* v;                 // [H, T, D], [KV, T, D], [KV, T, D]
  float eps; int T, H, KV, slots;                        // slots = H (shared) or H + 2 KV
  // Non-null: k and v are a key / value cache [KV, kv_rows, D] and token t's rows go to row
  // *pos_dev + t (a decode step replayed from a graph); rows outside the cache are not written.
  const int* pos_dev; int kv_rows;
};

template <int E>
__device__ __forceinline__ void load_i32(const int32_t* p, int (&o)[E]) {
  if constexpr (E == 4) {
    const v4i a = *reinterpret_cast<const v4i*>(p);
    for (int i = 0; i < 4; ++i) o[i] = a[i];
  } else if constexpr (E == 2) {
    const v2i a = *reinterpret_cast<const v2i*>(p);
    o[0] = a[0]; o[1] = a[1];
  } else {
    o[0] = *p;
  }
}
template <int E>
__device__ __forceinline__ void load_f32(const float* p, float (&o)[E]) {
  if constexpr (E == 4) {
    const v4f a = *reinterpret_cast<const v4f*>(p);
    for (int i = 0; i < 4; ++i) o[i] = a[i];
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) o[i] = p[i];
  }
}
// One wave per (token, head slot): slots 0 .. H-1 are the query heads, then KV key heads, then KV
// value heads, at columns slot * D of the GEMM result (pipeline.py:76-82).  A lane holds E = D/128
// elements of each half of the head at positions p0 .. p0+E-1 and p0+D/2 .. : the rotation pairs
// element d with d + D/2, so RoPE needs no lane exchange.
template <int E, bool IN_BF16>
__global__ __launch_bounds__(256) void qkv_kernel(QkvParams p) {
  constexpr int D = 128 * E, HALF = 64 * E;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + int(threadIdx.x >> 6);
  if (item >= p.T * p.slots) return;
  const int t = item / p.slots, slot = item % p.slots;
  const int p0 = lane * E;
  const int col = slot * D + p0;
  float y1[E], y2[E];
  if constexpr (IN_BF16) {
    const uint16_t* yr = p.y + int64_t(t) * p.ldy;
    load_bf16<E>(yr + col, y1);
    load_bf16<E>(yr + col + HALF, y2);
  } else {
    const float sxm = p.sx[t];
    int a1[E], a2[E];
    float s1[E], s2[E];
    const int32_t* ar = p.acc + int64_t(t) * p.ldacc;
    load_i32<E>(ar + col, a1);
    load_i32<E>(ar + col + HALF, a2);
    load_f32<E>(p.sw + col, s1);
    load_f32<E>(p.sw + col + HALF, s2);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      y1[e] = round_bf16((float(a1[e]) * sxm) * s1[e]);
      y2[e] = round_bf16((float(a2[e]) * sxm) * s2[e]);
    }
  }
  const bool is_q = slot < p.H, is_k = !is_q && slot < p.H + p.KV;
  const uint16_t* w = is_q ? p.qw : (is_k ? p.kw : nullptr);
  qkv_head<E>(y1, y2, p.eps, w, (is_q || is_k) ? p.cs + int64_t(t) * p.ldcs : nullptr,
              (is_q || is_k) ? p.sn + int64_t(t) * p.ldcs : nullptr, p0);
  float (&n1)[E] = y1;
  float (&n2)[E] = y2;
  uint16_t* dst;
  if (is_q || is_k) {
    dst = is_q ? p.q + (int64_t(slot) * p.T + t) * D : p.k + (int64_t(slot - p.H) * p.T + t) * D;
  } else {
    dst = p.v + (int64_t(slot - p.H - p.KV) * p.T + t) * D;
  }
  if (p.pos_dev && slot >= p.H) {
    const int row = *p.pos_dev + t;
    if (row < 0 || row >= p.kv_rows) return;  // (the whole wave: one item per wave)
    const int hk = slot < p.H + p.KV ? slot - p.H : slot - p.H - p.KV;
    dst = (slot < p.H + p.KV ? p.k : p.v) + (int64_t(hk) * p.kv_rows + row) * D;
  }
  store_bf16<E>(dst + p0, n1);
  store_bf16<E>(dst + p0 + HALF, n2);
}

// ---- host side -------------------------------------------------------------------------------
static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Launch the row chain on M rows of N elements (q columns up to 32*KF when packed); the caller
// has validated shapes and alignment.
static int launch_row_chain(const RowChain& p, bool in_i32, hipStream_t stream, const char* what) {
  const int KQ = p.KF ? p.KF * 32 : p.N;
  // Rows up to 64 * 8 * 6 = 3072 elements go to one wave each: every reduction is then a DPP
  // reduction with no LDS exchange or barrier, and a CU holds many more rows at once.  Longer
  // rows spread over up to four waves.
  const int ch = KQ <= 3072 ? (KQ + 511) / 512 : (KQ + 2047) / 2048;
  const int CHs = ch <= 1 ? 1 : ch <= 2 ? 2 : ch <= 3 ? 3 : ch <= 4 ? 4 : 6;
  const int chunks = (KQ + 8 * CHs - 1) / (8 * CHs);
  const int threads = ((chunks + 63) / 64) * 64;
  const int rows = (p.q && p.KF) ? ((p.M + 31) / 32) * 32 : p.M;
  const dim3 grid{static_cast<unsigned>(rows)};
#define W8A8_RC(C)                                                                          \
  do {                                                                                      \
    if (in_i32 && p.op == RC_NORM_RES) row_chain_kernel<C, true, RC_NORM_RES><<<grid, threads, 0, stream>>>(p); \
    else if (in_i32 && p.op == RC_GELU_MUL) row_chain_kernel<C, true, RC_GELU_MUL><<<grid, threads, 0, stream>>>(p); \
    else if (!in_i32 && p.op == RC_NORM_RES) row_chain_kernel<C, false, RC_NORM_RES><<<grid, threads, 0, stream>>>(p); \
    else if (!in_i32 && p.op == RC_GELU_MUL) row_chain_kernel<C, false, RC_GELU_MUL><<<grid, threads, 0, stream>>>(p); \
    else if (!in_i32 && p.op == RC_NONE) row_chain_kernel<C, false, RC_NONE><<<grid, threads, 0, stream>>>(p); \
    else return fail(W8A8_EINVAL, "%s: unsupported row-chain combination", what);         \
  } while (0)
  switch (CHs) {
    case 1: W8A8_RC(1); break;
    case 2: W8A8_RC(2); break;
    case 3: W8A8_RC(3); break;
    case 4: W8A8_RC(4); break;
    default: W8A8_RC(6); break;
  }
#undef W8A8_RC
  return check_launch(what);
}

// Checks shared by every row-chain entry point: N % 8 == 0 and N (the q width when packed) within
// the 8 * 256 * 6 elements a block holds; 16-byte aligned rows for every bf16 / int32 operand.
static int check_rows(const char* what, int64_t M, int64_t N) {
  if (M < 0 || N <= 0) return fail(W8A8_EINVAL, "%s: bad shape M=%lld N=%lld", what, (long long)M, (long long)N);
  if (N % 8 != 0) return fail(W8A8_ENOTSUP, "%s: N=%lld must be a multiple of 8", what, (long long)N);
  if (N > 12288) return fail(W8A8_ENOTSUP, "%s: N=%lld above the 12288 elements a row block holds", what, (long long)N);
  if (M > INT32_MAX / 2) return fail(W8A8_ENOTSUP, "%s: too many rows", what);
  return W8A8_OK;
}

static int check_bf16_rows(const char* what, const char* name, const uint16_t* p, int64_t ld, int64_t N) {
  if (!p) return fail(W8A8_EINVAL, "%s: %s is null", what, name);
  if (ld < N) return fail(W8A8_EINVAL, "%s: leading dimension of %s (%lld) below N", what, name, (long long)ld);
  if (!al16(p) || ld % 8 != 0) return fail(W8A8_EALIGN, "%s: %s rows must be 16-byte aligned", what, name);
  return W8A8_OK;
}

static int check_vec16(const char* what, const char* name, const void* p) {
  if (p && !al16(p)) return fail(W8A8_EALIGN, "%s: %s must be 16-byte aligned", what, name);
  return W8A8_OK;
}

static int check_acc(const char* what, const int32_t* acc, int64_t ldacc, const float* sx, const float* sw,
                     int64_t N) {
  if (!acc || !sx || !sw) return fail(W8A8_EINVAL, "%s: null acc / sx / sw", what);
  if (ldacc < N) return fail(W8A8_EINVAL, "%s: ldacc below the columns read", what);
  if (!al16(acc) || ldacc % 4 != 0 || !al16(sw))
    return fail(W8A8_EALIGN, "%s: acc rows and sw must be 16-byte aligned", what);
  return W8A8_OK;
}

// q / sq / packed: row-major q needs 8-byte aligned rows (8-byte stores); packed needs 16 bytes.
static int set_q(const char* what, RowChain& p, int8_t* q, int64_t ldq, int q_packed, float* sq, int64_t N) {
  if (!q || !sq) return fail(W8A8_EINVAL, "%s: null q / sq", what);
  p.q = q;
  p.sq = sq;
  if (q_packed) {
    if (!al16(q)) return fail(W8A8_EALIGN, "%s: packed q must be 16-byte aligned", what);
    p.KF = int(2 * ((N + 63) / 64));
    if (p.KF * 32 > 12288) return fail(W8A8_ENOTSUP, "%s: packed width above 12288", what);
  } else {
    if (ldq < N) return fail(W8A8_EINVAL, "%s: ldq below N", what);
    if ((reinterpret_cast<uintptr_t>(q) & 7) || ldq % 8 != 0)
      return fail(W8A8_EALIGN, "%s: q rows must be 8-byte aligned", what);
    p.ldq = ldq;
  }
  return W8A8_OK;
}

#define W8A8_TRY(x)               \
  do {                            \
    const int rc_ = (x);          \
    if (rc_ != W8A8_OK) return rc_; \
  } while (0)

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
  const char* what = "rms_residual";
  if ((q == nullptr) != (sq == nullptr)) return fail(W8A8_EINVAL, "rms_residual: q and its scale go together");
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_bf16_rows(what, "y", y, ldy, N));
  if (res) W8A8_TRY(check_bf16_rows(what, "res", res, ldr, N));
  W8A8_TRY(check_bf16_rows(what, "h", h, ldh, N));
  W8A8_TRY(check_vec16(what, "w", w));
  RowChain p{};
  if (q) W8A8_TRY(set_q(what, p, q, ldq, 0, sq, N));
  if (M == 0) return W8A8_OK;
  p.in = y; p.ld_in = ldy; p.head_stride = N; p.head_len = int(N);
  p.op = RC_NORM_RES; p.aux = res; p.ld_aux = res ? ldr : 0; p.w1 = w;
  p.h = h; p.ldh = ldh;
  p.eps = eps; p.M = int(M); p.N = int(N);
  return launch_row_chain(p, false, stream, "rms_residual_bf16");
}

int w8a8_k_in(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps, int64_t M, int64_t N, int8_t* q,
              int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  const char* what = "k_in";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_bf16_rows(what, "x", x, ldx, N));
  W8A8_TRY(check_vec16(what, "w", w));
  RowChain p{};
  W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, N));
  if (M == 0) return W8A8_OK;
  p.in = x; p.ld_in = ldx; p.head_stride = N; p.head_len = int(N);
  p.op = RC_NONE; p.norm2 = 1; p.w2 = w;
  p.eps = eps; p.M = int(M); p.N = int(N);
  return launch_row_chain(p, false, stream, what);
}

int w8a8_k_attn_out(const uint16_t* o, int64_t head_stride, int64_t row_stride, int64_t H, int64_t T, int64_t D,
                    int8_t* q, int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  const char* what = "k_attn_out";
  if (H <= 0 || D <= 0 || D % 8 != 0) return fail(W8A8_EINVAL, "k_attn_out: bad H=%lld D=%lld", (long long)H, (long long)D);
  const int64_t N = H * D;
  W8A8_TRY(check_rows(what, T, N));
  if (!o) return fail(W8A8_EINVAL, "k_attn_out: o is null");
  if (row_stride < D || (H > 1 && head_stride < D)) return fail(W8A8_EINVAL, "k_attn_out: strides below D");
  if (!al16(o) || row_stride % 8 != 0 || head_stride % 8 != 0)
    return fail(W8A8_EALIGN, "k_attn_out: o rows must be 16-byte aligned");
  RowChain p{};
  W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, N));
  if (T == 0) return W8A8_OK;
  p.in = o; p.ld_in = row_stride; p.head_stride = head_stride; p.head_len = int(D);
  p.op = RC_NONE;
  p.M = int(T); p.N = int(N);
  return launch_row_chain(p, false, stream, what);
}

}  // extern "C"

namespace w8a8 {

// The input of a row-chain entry: an int32 GEMM result with its scales, or dequantised bf16 rows.
struct RowInput {
  const void* p; int64_t ld; const float* sx; const float* sw; bool i32;
};

static int check_input(const char* what, const RowInput& in, int64_t N) {
  if (in.i32) return check_acc(what, static_cast<const int32_t*>(in.p), in.ld, in.sx, in.sw, N);
  return check_bf16_rows(what, "y", static_cast<const uint16_t*>(in.p), in.ld, N);
}

static void set_input(RowChain& p, const RowInput& in, int64_t N) {
  p.in = in.p; p.ld_in = in.ld;
  if (in.i32) {
    p.sx = in.sx; p.sw = in.sw;
  } else {
    p.head_stride = N; p.head_len = int(N);
  }
}

static int k_post_attn(const RowInput& in, const uint16_t* res, int64_t ldr, const uint16_t* w_post,
                       const uint16_t* w_pre_ff, float eps, int64_t M, int64_t N, uint16_t* h, int64_t ldh, int8_t* q,
                       int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  const char* what = "k_post_attn";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_input(what, in, N));
  W8A8_TRY(check_bf16_rows(what, "res", res, ldr, N));
  W8A8_TRY(check_bf16_rows(what, "h", h, ldh, N));
  W8A8_TRY(check_vec16(what, "w_post", w_post));
  W8A8_TRY(check_vec16(what, "w_pre_ff", w_pre_ff));
  RowChain p{};
  W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, N));
  if (M == 0) return W8A8_OK;
  set_input(p, in, N);
  p.op = RC_NORM_RES; p.aux = res; p.ld_aux = ldr; p.w1 = w_post;
  p.h = h; p.ldh = ldh; p.norm2 = 1; p.w2 = w_pre_ff;
  p.eps = eps; p.M = int(M); p.N = int(N);
  return launch_row_chain(p, in.i32, stream, what);
}

static int k_post_ff(const RowInput& in, const uint16_t* res, int64_t ldr, const uint16_t* w_post_ff, float eps,
                     int64_t M, int64_t N, uint16_t* h, int64_t ldh, int8_t* q, int64_t ldq, int q_packed, float* sq,
                     hipStream_t stream) {
  const char* what = "k_post_ff";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_input(what, in, N));
  W8A8_TRY(check_bf16_rows(what, "res", res, ldr, N));
  W8A8_TRY(check_bf16_rows(what, "h", h, ldh, N));
  W8A8_TRY(check_vec16(what, "w_post_ff", w_post_ff));
  RowChain p{};
  W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, N));
  if (M == 0) return W8A8_OK;
  set_input(p, in, N);
  p.op = RC_NORM_RES; p.aux = res; p.ld_aux = ldr; p.w1 = w_post_ff;
  p.h = h; p.ldh = ldh;
  p.eps = eps; p.M = int(M); p.N = int(N);
  return launch_row_chain(p, in.i32, stream, what);
}

static int k_ple_gate(const RowInput& in, const uint16_t* ple, int64_t ldp, int64_t M, int64_t N, int8_t* q,
                      int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  const char* what = "k_ple_gate";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_input(what, in, N));
  W8A8_TRY(check_bf16_rows(what, "ple", ple, ldp, N));
  RowChain p{};
  W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, N));
  if (M == 0) return W8A8_OK;
  set_input(p, in, N);
  p.op = RC_GELU_MUL; p.aux = ple; p.ld_aux = ldp;
  p.M = int(M); p.N = int(N);
  return launch_row_chain(p, in.i32, stream, what);
}

// k_ple_out, and with w_next also the next layer's k_in on the rows it writes (the same launch: the
// second norm and the quant of the row kernel, on the values stored as out).
static int k_ple_out(const RowInput& in, const uint16_t* h, int64_t ldh, const uint16_t* w_post_ple,
                     const uint16_t* scalar, float eps, int64_t M, int64_t N, uint16_t* out, int64_t ldo,
                     hipStream_t stream, const uint16_t* w_next = nullptr, int8_t* q = nullptr, int64_t ldq = 0,
                     int q_packed = 0, float* sq = nullptr) {
  const char* what = w_next ? "k_ple_out_k_in" : "k_ple_out";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_input(what, in, N));
  W8A8_TRY(check_bf16_rows(what, "h", h, ldh, N));
  W8A8_TRY(check_bf16_rows(what, "out", out, ldo, N));
  W8A8_TRY(check_vec16(what, "w_post_ple", w_post_ple));
  if (!scalar) return fail(W8A8_EINVAL, "%s: scalar is null", what);
  RowChain p{};
  if (w_next) {
    W8A8_TRY(check_vec16(what, "w_next", w_next));
    W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, N));
  }
  if (M == 0) return W8A8_OK;
  set_input(p, in, N);
  p.op = RC_NORM_RES; p.aux = h; p.ld_aux = ldh; p.w1 = w_post_ple; p.scalar = scalar;
  p.h = out; p.ldh = ldo;
  if (w_next) {
    p.norm2 = 1;
    p.w2 = w_next;
  }
  p.eps = eps; p.M = int(M); p.N = int(N);
  return launch_row_chain(p, in.i32, stream, what);
}

static int k_qkv(const RowInput& in, const uint16_t* cos_, const uint16_t* sin_, int64_t ldcs, const uint16_t* qw,
                 const uint16_t* kw, float eps, int64_t T, int64_t H, int64_t KV, int64_t D, int shared, uint16_t* q,
                 uint16_t* k, uint16_t* v, hipStream_t stream, const int* pos_dev = nullptr, int64_t kv_rows = 0) {
  const char* what = "k_qkv";
  if (T < 0 || H <= 0 || KV < 0 || (!shared && KV <= 0))
    return fail(W8A8_EINVAL, "k_qkv: bad shape T=%lld H=%lld KV=%lld", (long long)T, (long long)H, (long long)KV);
  if (D != 128 && D != 256 && D != 512)
    return fail(W8A8_ENOTSUP, "k_qkv: head_dim D=%lld (supported: 128, 256, 512)", (long long)D);
  const int64_t slots = shared ? H : H + 2 * KV;
  W8A8_TRY(check_input(what, in, slots * D));
  if (!cos_ || !sin_ || !q || (!shared && (!k || !v))) return fail(W8A8_EINVAL, "k_qkv: null pointer");
  if (ldcs < D) return fail(W8A8_EINVAL, "k_qkv: ldcs below D");
  if (!al16(cos_) || !al16(sin_) || ldcs % 8 != 0 || !al16(q) || (!shared && (!al16(k) || !al16(v))))
    return fail(W8A8_EALIGN, "k_qkv: cos / sin rows and q / k / v must be 16-byte aligned");
  W8A8_TRY(check_vec16(what, "qw", qw));
  W8A8_TRY(check_vec16(what, "kw", kw));
  if (T * slots > INT32_MAX - 4) return fail(W8A8_ENOTSUP, "k_qkv: too large");
  if (T == 0) return W8A8_OK;
  QkvParams p{};
  if (in.i32) {
    p.acc = static_cast<const int32_t*>(in.p); p.ldacc = in.ld; p.sx = in.sx; p.sw = in.sw;
  } else {
    p.y = static_cast<const uint16_t*>(in.p); p.ldy = in.ld;
  }
  p.cs = cos_; p.sn = sin_; p.ldcs = ldcs; p.qw = qw; p.kw = shared ? nullptr : kw;
  p.q = q; p.k = k; p.v = v;
  p.eps = eps; p.T = int(T); p.H = int(H); p.KV = shared ? 0 : int(KV); p.slots = int(slots);
  p.pos_dev = pos_dev; p.kv_rows = int(kv_rows);
  const dim3 grid{static_cast<unsigned>((T * slots + 3) / 4)};
#define W8A8_QKV(E)                                                                  \
  do {                                                                               \
    if (in.i32) qkv_kernel<E, false><<<grid, 256, 0, stream>>>(p);                   \
    else qkv_kernel<E, true><<<grid, 256, 0, stream>>>(p);                           \
  } while (0)
  if (D == 128) W8A8_QKV(1);
  else if (D == 256) W8A8_QKV(2);
  else W8A8_QKV(4);
#undef W8A8_QKV
  return check_launch(what);
}

}  // namespace w8a8

extern "C" {

int w8a8_k_post_attn(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, const uint16_t* res,
                     int64_t ldr, const uint16_t* w_post, const uint16_t* w_pre_ff, float eps, int64_t M, int64_t N,
                     uint16_t* h, int64_t ldh, int8_t* q, int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  return w8a8::k_post_attn(RowInput{acc, ldacc, sx, sw, true}, res, ldr, w_post, w_pre_ff, eps, M, N, h, ldh, q, ldq,
                           q_packed, sq, stream);
}

int w8a8_k_post_attn_y(const uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldr, const uint16_t* w_post,
                       const uint16_t* w_pre_ff, float eps, int64_t M, int64_t N, uint16_t* h, int64_t ldh, int8_t* q,
                       int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  return w8a8::k_post_attn(RowInput{y, ldy, nullptr, nullptr, false}, res, ldr, w_post, w_pre_ff, eps, M, N, h, ldh,
                           q, ldq, q_packed, sq, stream);
}

int w8a8_k_gelu(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, int64_t M, int64_t I, int8_t* q,
                int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  const char* what = "k_gelu";
  W8A8_TRY(check_rows(what, M, I));
  W8A8_TRY(check_acc(what, acc, ldacc, sx, sw, 2 * I));
  RowChain p{};
  W8A8_TRY(set_q(what, p, q, ldq, q_packed, sq, I));
  if (M == 0) return W8A8_OK;
  p.in = acc; p.ld_in = ldacc; p.sx = sx; p.sw = sw;
  p.op = RC_GELU_MUL;
  p.M = int(M); p.N = int(I);
  return launch_row_chain(p, true, stream, what);
}

int w8a8_rms_residual_norm_bf16(const uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldr, const uint16_t* w1,
                                const uint16_t* scalar, const uint16_t* w2, float eps, int64_t M, int64_t N, uint16_t* h,
                                int64_t ldh, uint16_t* x, int64_t ldx, hipStream_t stream) {
  const char* what = "rms_residual_norm_bf16";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_bf16_rows(what, "y", y, ldy, N));
  W8A8_TRY(check_bf16_rows(what, "res", res, ldr, N));
  W8A8_TRY(check_bf16_rows(what, "h", h, ldh, N));
  W8A8_TRY(check_bf16_rows(what, "x", x, ldx, N));
  if ((w1 && !al16(w1)) || (w2 && !al16(w2))) return fail(W8A8_EALIGN, "%s: norm weights must be 16-byte aligned", what);
  if (M == 0) return W8A8_OK;
  RowChain p{};
  set_input(p, RowInput{y, ldy, nullptr, nullptr, false}, N);
  p.op = RC_NORM_RES; p.aux = res; p.ld_aux = ldr; p.w1 = w1; p.scalar = scalar;
  p.h = h; p.ldh = ldh;
  p.norm2 = 1; p.w2 = w2; p.h2 = x; p.ldh2 = ldx;
  p.eps = eps; p.M = int(M); p.N = int(N);
  return launch_row_chain(p, false, stream, what);
}

int w8a8_gelu_mul_bf16(const uint16_t* y, int64_t ldy, const uint16_t* mul, int64_t ldm, int64_t M, int64_t N,
                       uint16_t* out, int64_t ldo, hipStream_t stream) {
  const char* what = "gelu_mul_bf16";
  W8A8_TRY(check_rows(what, M, N));
  W8A8_TRY(check_bf16_rows(what, "y", y, ldy, mul ? N : 2 * N));
  if (mul) W8A8_TRY(check_bf16_rows(what, "mul", mul, ldm, N));
  W8A8_TRY(check_bf16_rows(what, "out", out, ldo, N));
  if (M == 0) return W8A8_OK;
  RowChain p{};
  set_input(p, RowInput{y, ldy, nullptr, nullptr, false}, N);
  p.op = RC_GELU_MUL; p.aux = mul; p.ld_aux = ldm;
  p.h = out; p.ldh = ldo;
  p.M = int(M); p.N = int(N);
  return launch_row_chain(p, false, stream, what);
}

int w8a8_k_post_ff(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, const uint16_t* res,
                   int64_t ldr, const uint16_t* w_post_ff, float eps, int64_t M, int64_t N, uint16_t* h, int64_t ldh,
                   int8_t* q, int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  return w8a8::k_post_ff(RowInput{acc, ldacc, sx, sw, true}, res, ldr, w_post_ff, eps, M, N, h, ldh, q, ldq, q_packed,
                         sq, stream);
}

int w8a8_k_post_ff_y(const uint16_t* y, int64_t ldy, const uint16_t* res, int64_t ldr, const uint16_t* w_post_ff,
                     float eps, int64_t M, int64_t N, uint16_t* h, int64_t ldh, int8_t* q, int64_t ldq, int q_packed,
                     float* sq, hipStream_t stream) {
  return w8a8::k_post_ff(RowInput{y, ldy, nullptr, nullptr, false}, res, ldr, w_post_ff, eps, M, N, h, ldh, q, ldq,
                         q_packed, sq, stream);
}

int w8a8_k_ple_gate(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, const uint16_t* ple,
                    int64_t ldp, int64_t M, int64_t N, int8_t* q, int64_t ldq, int q_packed, float* sq,
                    hipStream_t stream) {
  return w8a8::k_ple_gate(RowInput{acc, ldacc, sx, sw, true}, ple, ldp, M, N, q, ldq, q_packed, sq, stream);
}

int w8a8_k_ple_gate_y(const uint16_t* y, int64_t ldy, const uint16_t* ple, int64_t ldp, int64_t M, int64_t N,
                      int8_t* q, int64_t ldq, int q_packed, float* sq, hipStream_t stream) {
  return w8a8::k_ple_gate(RowInput{y, ldy, nullptr, nullptr, false}, ple, ldp, M, N, q, ldq, q_packed, sq, stream);
}

int w8a8_k_ple_out(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, const uint16_t* h,
                   int64_t ldh, const uint16_t* w_post_ple, const uint16_t* scalar, float eps, int64_t M, int64_t N,
                   uint16_t* out, int64_t ldo, hipStream_t stream) {
  return w8a8::k_ple_out(RowInput{acc, ldacc, sx, sw, true}, h, ldh, w_post_ple, scalar, eps, M, N, out, ldo, stream);
}

int w8a8_k_ple_out_k_in(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, const uint16_t* h,
                        int64_t ldh, const uint16_t* w_post_ple, const uint16_t* scalar, const uint16_t* w_in_next,
                        float eps, int64_t M, int64_t N, uint16_t* out, int64_t ldo, int8_t* q, int64_t ldq,
                        int q_packed, float* sq, hipStream_t stream) {
  if (!w_in_next) return fail(W8A8_EINVAL, "k_ple_out_k_in: w_in_next is null");
  return w8a8::k_ple_out(RowInput{acc, ldacc, sx, sw, true}, h, ldh, w_post_ple, scalar, eps, M, N, out, ldo, stream,
                         w_in_next, q, ldq, q_packed, sq);
}

int w8a8_k_ple_out_k_in_y(const uint16_t* y, int64_t ldy, const uint16_t* h, int64_t ldh, const uint16_t* w_post_ple,
                          const uint16_t* scalar, const uint16_t* w_in_next, float eps, int64_t M, int64_t N,
                          uint16_t* out, int64_t ldo, int8_t* q, int64_t ldq, int q_packed, float* sq,
                          hipStream_t stream) {
  if (!w_in_next) return fail(W8A8_EINVAL, "k_ple_out_k_in: w_in_next is null");
  return w8a8::k_ple_out(RowInput{y, ldy, nullptr, nullptr, false}, h, ldh, w_post_ple, scalar, eps, M, N, out, ldo,
                         stream, w_in_next, q, ldq, q_packed, sq);
}

int w8a8_k_ple_out_y(const uint16_t* y, int64_t ldy, const uint16_t* h, int64_t ldh, const uint16_t* w_post_ple,
                     const uint16_t* scalar, float eps, int64_t M, int64_t N, uint16_t* out, int64_t ldo,
                     hipStream_t stream) {
  return w8a8::k_ple_out(RowInput{y, ldy, nullptr, nullptr, false}, h, ldh, w_post_ple, scalar, eps, M, N, out, ldo,
                         stream);
}

int w8a8_k_qkv_cache_y(const uint16_t* y, int64_t ldy, const uint16_t* cos_, const uint16_t* sin_, int64_t ldcs,
                       const uint16_t* qw, const uint16_t* kw, float eps, int64_t T, int64_t H, int64_t KV, int64_t D,
                       uint16_t* q, uint16_t* k_cache, uint16_t* v_cache, int64_t kv_rows, const int32_t* pos,
                       hipStream_t stream) {
  if (!pos || !k_cache || !v_cache) return fail(W8A8_EINVAL, "k_qkv_cache: null pointer");
  if ((uintptr_t)pos % 4) return fail(W8A8_EALIGN, "k_qkv_cache: pos must be 4-byte aligned");
  if (kv_rows < 1 || kv_rows > INT32_MAX || KV * kv_rows * D > INT64_MAX / 2)
    return fail(W8A8_EINVAL, "k_qkv_cache: kv_rows=%lld", (long long)kv_rows);
  return w8a8::k_qkv(RowInput{y, ldy, nullptr, nullptr, false}, cos_, sin_, ldcs, qw, kw, eps, T, H, KV, D, 0, q,
                     k_cache, v_cache, stream, pos, kv_rows);
}

int w8a8_k_qkv(const int32_t* acc, int64_t ldacc, const float* sx, const float* sw, const uint16_t* cos_,
               const uint16_t* sin_, int64_t ldcs, const uint16_t* qw, const uint16_t* kw, float eps, int64_t T,
               int64_t H, int64_t KV, int64_t D, int shared, uint16_t* q, uint16_t* k, uint16_t* v,
               hipStream_t stream) {
  return w8a8::k_qkv(RowInput{acc, ldacc, sx, sw, true}, cos_, sin_, ldcs, qw, kw, eps, T, H, KV, D, shared, q, k, v,
                     stream);
}

int w8a8_k_qkv_y(const uint16_t* y, int64_t ldy, const uint16_t* cos_, const uint16_t* sin_, int64_t ldcs,
                 const uint16_t* qw, const uint16_t* kw, float eps, int64_t T, int64_t H, int64_t KV, int64_t D,
                 int shared, uint16_t* q, uint16_t* k, uint16_t* v, hipStream_t stream) {
  return w8a8::k_qkv(RowInput{y, ldy, nullptr, nullptr, false}, cos_, sin_, ldcs, qw, kw, eps, T, H, KV, D, shared,
                     q, k, v, stream);
}

}  // extern "C"
