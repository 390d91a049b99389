// Weight-only int8 GEMV / skinny GEMM for decode and the LM head.
//
// y[m, n] = bf16( (sum_k x[m,k] * w[n,k]) * s[n] ),  x bf16 [M<=16, K], w int8 [N, K] row-major,
// s bf16 or fp32 [N]: the contract of torch._weight_int8pack_mm as the reference calls it
// (gemma_npu.py:155-156, decode linears gemma_npu.py:120-121, Int8Head gemma_npu.py:159-172).
//
// The weight is streamed once from HBM with 16-byte loads; each byte is widened to bf16 (exact:
// |w| <= 128) and multiplied on the bf16 MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulate), with
// the M <= 16 activation rows as the MFMA's other operand.  A wave covers TPW 16-row n-tiles, so each activation fragment it loads serves
// TPW weight fragments; for shapes with few n-tiles, `split` waves of a workgroup share one
// n-tile's K range (k-blocks of 64 dealt round-robin) and their partial sums are added in LDS in
// fixed wave order, so the result is deterministic.
#include "w8a8_common.h"

namespace w8a8 {

struct GemvParams {
  const uint16_t* x; int64_t ldx;  // bf16 [M, K]
  const int8_t* w; int64_t ldw;    // int8 [N, K]
  const void* s; int s_f32;        // [N] scales, bf16 (0) or fp32 (1)
  uint16_t* y; int64_t ldy;        // bf16 [M, N]
  uint32_t x_bytes, w_bytes;
  int M, N, K, KB;                 // KB = ceil(K / 64)
  int split;                       // waves per group of n-tiles, each taking every split-th k-block
  // Activation epilogue (ACT template argument): 1, GELU pair: the weight is [gate; up] stacked
  // (N = 2I, I a multiple of 16) and y [M, I] = bf16(bf16(gelu_tanh(g)) * u) with g, u the bf16
  // outputs of the gate and up rows; 2, GELU times a multiplier: y = bf16(bf16(gelu_tanh(g)) * mul)
  // with mul bf16 [M, N] (ld = ldm).
  const uint16_t* mul; int64_t ldm;
  int half_tiles;                  // ACT 1: I / 16, the up rows' first tile
  // Row prologue (PRO template argument, M = 1): the activation row is not read from x but made by
  // every workgroup from the previous step's output, as w8a8_rms_residual_norm_bf16 (norm2 set) or
  // w8a8_rms_residual_bf16 (norm2 clear) would make it in a launch of its own:
  //   h = bf16(res + bf16(rms(pro_y) * w1)) [then bf16(h * scalar)],  x = norm2 ? bf16(rms(h) * w2) : h
  // (no res: h = bf16(rms(pro_y) * w1)).  Workgroup 0 stores h when pro_h is set.
  const uint16_t* pro_y; const uint16_t* pro_res; const uint16_t* pro_w1; const uint16_t* pro_scalar;
  const uint16_t* pro_w2; uint16_t* pro_h;
  float pro_eps; int pro_norm2, pro_ch;  // pro_ch: the row kernel's 8-element chunks per lane for K
  // Attention-merge prologue (PRO == 4, M = 1): the activation row is one token's decode attention
  // output [H * D], merged from the split-key kernel's chunk partials (part_o [KV][nchunk_grid][G][D],
  // part_ml [KV][nchunk_grid][G][2]) as attn_decode_merge_kernel merges them, for at most
  // DEC_MERGE_IN_GEMV_CHUNKS chunks; the live chunks follow from the position in device memory.
  const float* m_po; const float* m_ml; const int* m_pos;
  int m_window, m_nchunk_grid, m_G, m_D, m_chunk; float m_c;
};

// The merge prologue.  For at most 16 chunks attn_decode_merge_kernel's sums reduce to fixed orders,
// taken here: per head, its chunk weights w_c = exp2(M_c c - M c) and the weighted l over a 16-leaf
// tree (t + 8, t + 4, t + 2, t + 1), made once per workgroup by one thread per head into mw
// [16 heads][17] (w_0 .. w_15, then 1 / l); per element, the chunks in order, each term
// fma(w_c, o_c, 0), a +0 after them when fewer than 16 are live (the merge kernel's empty parts).
// Each thread makes elements e, e + 1 of the row (one head, columns d, d + 1); the partials of its
// first pair are fetched before the weights are made.
__device__ __forceinline__ void gemv_attn_merge_row(const GemvParams& p, uint16_t* xs, float* mw) {
  constexpr int NC = DEC_MERGE_IN_GEMV_CHUNKS;
  const int pos = *p.m_pos;
  const int klo = p.m_window > 0 ? max(0, pos - p.m_window + 1) : 0;
  const int nchunk = max(0, min((pos - klo) / p.m_chunk + 1, p.m_nchunk_grid));
  const int H = p.K / p.m_D;
  auto head_base = [&](int h) { return int64_t(h / p.m_G) * p.m_nchunk_grid * p.m_G + h % p.m_G; };
  // this thread's first pair: its partials now
  int e = 2 * int(threadIdx.x);
  v2f oc[NC];
  auto fetch = [&](int e) {
    const int h = e / p.m_D, d = e % p.m_D;
    const int64_t hb = head_base(h);
#pragma unroll
    for (int c = 0; c < NC; ++c)
      oc[c] = (c < nchunk && e < p.K) ? *reinterpret_cast<const v2f*>(p.m_po + (hb + int64_t(c) * p.m_G) * p.m_D + d)
                                      : v2f{0.0f, 0.0f};
  };
  fetch(e);
  if (int(threadIdx.x) < H) {
    const int h = int(threadIdx.x);
    const int64_t hb = head_base(h);
    float mc[NC], lc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const v2f ml = c < nchunk ? *reinterpret_cast<const v2f*>(p.m_ml + (hb + int64_t(c) * p.m_G) * 2)
                                : v2f{-__builtin_inff(), 0.0f};
      mc[c] = ml[0];
      lc[c] = ml[1];
    }
    float M = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < NC; ++c) M = fmaxf(M, mc[c]);
    const float ms = M == -__builtin_inff() ? 0.0f : M * p.m_c;
    float v[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float w = c < nchunk ? __builtin_amdgcn_exp2f(__builtin_fmaf(mc[c], p.m_c, -ms)) : 0.0f;
      mw[h * (NC + 1) + c] = w;
      v[c] = c < nchunk ? __builtin_fmaf(w, lc[c], 0.0f) : 0.0f;
    }
#pragma unroll
    for (int s = 8; s > 0; s >>= 1)
#pragma unroll
      for (int t = 0; t < s; ++t) v[t] = v[t] + v[t + s];
    mw[h * (NC + 1) + NC] = v[0] > 0.0f ? 1.0f / v[0] : 0.0f;
  }
  __syncthreads();
  for (; e < p.K; e += 2 * int(blockDim.x)) {
    if (e != 2 * int(threadIdx.x)) fetch(e);
    const float* wh = mw + (e / p.m_D) * (NC + 1);
    float a0 = 0.0f, a1 = 0.0f;
    if (nchunk > 0) {
      a0 = __builtin_fmaf(wh[0], oc[0][0], 0.0f);
      a1 = __builtin_fmaf(wh[0], oc[0][1], 0.0f);
    }
#pragma unroll
    for (int c = 1; c < NC; ++c)
      if (c < nchunk) {
        a0 = a0 + __builtin_fmaf(wh[c], oc[c][0], 0.0f);
        a1 = a1 + __builtin_fmaf(wh[c], oc[c][1], 0.0f);
      }
    if (nchunk < NC) {
      a0 = a0 + 0.0f;
      a1 = a1 + 0.0f;
    }
    const float inv = wh[NC];
    *reinterpret_cast<uint32_t*>(xs + e) = pack_bf16x2(a0 * inv, a1 * inv);
  }
}

// The row prologue on one wave, in the arithmetic and order of the row kernel's one-wave rows
// (row_chain_kernel with 64 threads, rowops.hip): lane t holds chunks c < CH of 8 elements at
// k = 8 * (64 c + t); the sums of squares are added chunk by chunk, element by element, then across
// the wave by wave_sum_dpp.  Its operands are fetched first (RowIn::load), before the kernel issues
// its weight loads, so the arithmetic (RowIn::make) waits for them alone; the result goes to
// xs [CH * 512] bf16 (zeros from K on).
template <int CH>
struct RowIn {
  v4u y[CH], res[CH], w1[CH], w2[CH];
  uint16_t scalar;

  __device__ __forceinline__ void load(const GemvParams& p) {
    const int t = threadIdx.x & 63;
    scalar = p.pro_scalar ? *p.pro_scalar : uint16_t(0x3f80);
    const v4u one = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};  // bf16 1.0 x 8
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = 8 * (64 * c + t);
      const bool in = k < p.K;
      y[c] = in ? *reinterpret_cast<const v4u*>(p.pro_y + k) : v4u{0u, 0u, 0u, 0u};
      res[c] = (in && p.pro_res) ? *reinterpret_cast<const v4u*>(p.pro_res + k) : v4u{0u, 0u, 0u, 0u};
      w1[c] = (in && p.pro_w1) ? *reinterpret_cast<const v4u*>(p.pro_w1 + k) : one;
      w2[c] = (in && p.pro_norm2 && p.pro_w2) ? *reinterpret_cast<const v4u*>(p.pro_w2 + k) : one;
    }
  }

  // The values stay packed as bf16 between steps (every intermediate the row kernel rounds to bf16
  // is exactly a bf16), which keeps the prologue's registers few while the weights are in flight.
  __device__ __forceinline__ void make(const GemvParams& p, uint16_t* xs) {
    const int t = threadIdx.x & 63, N = p.K;
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float v[8];
      unpack8(y[c], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
    }
    ss = wave_sum_dpp(ss);
    const float r = 1.0f / sqrtf(ss / float(N) + p.pro_eps);
    const float scl = bf16_to_f32(scalar);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float v[8], rv[8], wv[8];
      unpack8(y[c], v);
      unpack8(res[c], rv);
      unpack8(w1[c], wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float n = v[i] * r;
        if (p.pro_w1) n = n * wv[i];
        v[i] = p.pro_res ? round_bf16(rv[i] + round_bf16(n)) : round_bf16(n);
        if (p.pro_scalar) v[i] = round_bf16(v[i] * scl);
      }
      y[c] = pack8(v);  // h
    }
    if (p.pro_h && blockIdx.x == 0) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int k = 8 * (64 * c + t);
        if (k < N) *reinterpret_cast<v4u*>(p.pro_h + k) = y[c];
      }
    }
    if (p.pro_norm2) {
      float s2 = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        float v[8];
        unpack8(y[c], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) s2 += v[i] * v[i];
      }
      s2 = wave_sum_dpp(s2);
      const float r2 = 1.0f / sqrtf(s2 / float(N) + p.pro_eps);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        float v[8], wv[8];
        unpack8(y[c], v);
        unpack8(w2[c], wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float n = v[i] * r2;
          if (p.pro_w2) n = n * wv[i];
          v[i] = round_bf16(n);
        }
        y[c] = pack8(v);
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = 8 * (64 * c + t);
      *reinterpret_cast<v4u*>(xs + k) = k < N ? y[c] : v4u{0u, 0u, 0u, 0u};
    }
  }
};

// Widen 8 signed bytes (two dwords) to 8 bf16 values, exactly.
__device__ __forceinline__ v8bf widen8(uint32_t lo, uint32_t hi) {
  v4u r;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t d = i ? hi : lo;
    const float f0 = float(int8_t(d & 0xff));
    const float f1 = float(int8_t((d >> 8) & 0xff));
    const float f2 = float(int8_t((d >> 16) & 0xff));
    const float f3 = float(int8_t(d >> 24));
    r[2 * i] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
    r[2 * i + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
  }
  return __builtin_bit_cast(v8bf, r);
}

// A wave multiplies TPW n-tiles of 16 weight rows against the M <= 16 activation rows: per k-block
// of 64 it loads the activation fragment once and TPW weight fragments, and issues 2*TPW MFMAs.
// With split > 1 the waves of a group take interleaved k-blocks and their partial sums are added
// in LDS in wave order (deterministic).
//
// PACKED: the weight is in the GEMV fragment layout (pack_gemv_weight_kernel): fragment (t, kb) =
// 1 KiB at (t * KB + kb) * 1024 whose byte 16*l + b is W[16t + l%16][64kb + 16(l/16) + b], the
// bytes lane l feeds the MFMA.  Every weight load is then one contiguous KiB of whole cache
// lines, which the stream reads with the streaming (sc0 nt) policy: measured on MI355X for the
// LM head (K=1536, N=262144), 6.2 TB/s against 5.0 TB/s for the row-major weight, where each load
// takes 64-byte pieces of 16 rows.  Row-major weights keep the default policy (a streamed half
// line would be fetched twice).
template <int TPW, int U, bool PACKED, int NWB, int ACT = 0, int PRO = 0>
__global__ __launch_bounds__(NWB * 64) void gemv_kernel(GemvParams p) {
  static_assert(ACT != 1 || TPW == 2, "a GELU pair is one gate and one up tile per wave");
  __shared__ v4f red[NWB][TPW][64];
  __shared__ __attribute__((aligned(16))) uint16_t xs[PRO == 4 ? 4096 : PRO ? PRO * 512 : 8];  // PRO: the row
  __shared__ float mw[PRO == 4 ? 16 * (DEC_MERGE_IN_GEMV_CHUNKS + 1) : 1];     // PRO 4: chunk weights
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int group_in_block = wave / p.split;
  const int ks = wave % p.split;
  const int groups_per_block = NWB / p.split;
  const int group = blockIdx.x * groups_per_block + group_in_block;
  // ACT 1: group g multiplies gate tile g and up tile g + half_tiles
  const int tile0 = ACT == 1 ? group : group * TPW;
  const int tstride = ACT == 1 ? p.half_tiles : 1;
  const int ntiles = (p.N + 15) >> 4;
  const bool active = ACT == 1 ? tile0 < p.half_tiles : tile0 < ntiles;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, p.w_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, p.x_bytes);
  const int kc = (lane >> 4) * 16;           // this lane's 16-byte chunk inside each 64-wide k-block
  const int mrow = lane & 15;                // activation row this lane supplies
  // Weight rows past N and activation rows past M start at or past the buffer ends and read 0.
  uint32_t wbase[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    wbase[t] = PACKED ? uint32_t(tile0 + t * tstride) * uint32_t(p.KB) * 1024u + uint32_t(lane) * 16u
                      : uint32_t((tile0 + t * tstride) * 16 + (lane & 15)) * uint32_t(p.ldw) + uint32_t(kc);
  constexpr uint32_t W_KB = PACKED ? 1024u : 64u;  // weight bytes between k-blocks
  constexpr int W_POL = PACKED ? 3 : 0;              // sc0 nt for the packed stream
  const uint32_t xbase = (uint32_t(mrow) * uint32_t(p.ldx) + uint32_t(kc)) * 2u;

  v4f acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  // PRO: the activation row is made once per workgroup by its first wave (one row: M = 1) while
  // every wave's first round of weight fragments is in flight.
  RowIn<(PRO >= 1 && PRO <= 3) ? PRO : 1> row;
  v4i wpre[U][TPW];
  if constexpr (PRO) {
    if (PRO <= 3 && wave == 0) row.load(p);
    // Issued without branches (a fragment outside the weight is read past the buffer's end as
    // zeros), so the prologue's arithmetic can wait for its own operands and leave these in flight.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kb = ks + u * p.split;
      const bool ok = active && kb < p.KB && kb * 64 + kc < p.K;
#pragma unroll
      for (int t = 0; t < TPW; ++t)
        wpre[u][t] = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? wbase[t] + uint32_t(kb) * W_KB : 0x80000000u, 0, W_POL));
    }
    if constexpr (PRO == 4)
      gemv_attn_merge_row(p, xs, mw);
    else if (wave == 0)
      row.make(p, xs);
    __syncthreads();
  }
  if (active) {
    const int stride = p.split * U;
    int kb0 = ks;
    if constexpr (PRO) {
      // the first round: its weights are in registers, the row in LDS
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kb = kb0 + u * p.split;
        v4i xa = {0, 0, 0, 0}, xb = {0, 0, 0, 0};
        if (kb < p.KB && kb * 64 + kc < p.K && mrow == 0) {
          const v4i* xv = reinterpret_cast<const v4i*>(xs + kb * 64 + kc);
          xa = xv[0];
          xb = xv[1];
        }
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          const v8bf wa = widen8(uint32_t(wpre[u][t][0]), uint32_t(wpre[u][t][1]));
          const v8bf wb = widen8(uint32_t(wpre[u][t][2]), uint32_t(wpre[u][t][3]));
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, __builtin_bit_cast(v8bf, xa), acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, __builtin_bit_cast(v8bf, xb), acc[t], 0, 0, 0);
        }
      }
      kb0 += stride;
    }
    for (; kb0 < p.KB; kb0 += stride) {
      v4i wv[U][TPW], xa[U], xb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kb = kb0 + u * p.split;
        if (kb < p.KB && kb * 64 + kc < p.K) {
          if constexpr (PRO) {
            const v4i* xv = reinterpret_cast<const v4i*>(xs + kb * 64 + kc);
            xa[u] = mrow == 0 ? xv[0] : v4i{0, 0, 0, 0};
            xb[u] = mrow == 0 ? xv[1] : v4i{0, 0, 0, 0};
          } else {
            xa[u] = buf_load16(rx, xbase + uint32_t(kb) * 128u);
            xb[u] = buf_load16(rx, xbase + uint32_t(kb) * 128u + 16u);
          }
#pragma unroll
          for (int t = 0; t < TPW; ++t)
            wv[u][t] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, wbase[t] + uint32_t(kb) * W_KB, 0, W_POL));
        } else {
          xa[u] = v4i{0, 0, 0, 0};
          xb[u] = v4i{0, 0, 0, 0};
#pragma unroll
          for (int t = 0; t < TPW; ++t) wv[u][t] = v4i{0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          const v8bf w0 = widen8(uint32_t(wv[u][t][0]), uint32_t(wv[u][t][1]));
          const v8bf w1 = widen8(uint32_t(wv[u][t][2]), uint32_t(wv[u][t][3]));
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, __builtin_bit_cast(v8bf, xa[u]), acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, __builtin_bit_cast(v8bf, xb[u]), acc[t], 0, 0, 0);
        }
    }
  }

  if (p.split > 1) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      acc[t] = red[wave][t][lane];
      for (int q = 1; q < p.split; ++q) acc[t] += red[wave + q][t][lane];
    }
  }
  if (!active) return;

  // acc[t] lane l: row m = l % 16, columns n0 .. n0+3 with n0 = (tile0 + t)*16 + 4*(l/16).
  const int m = lane & 15;
  if (m >= p.M) return;
  auto scale_at = [&](int nn) -> float {
    return p.s_f32 ? reinterpret_cast<const float*>(p.s)[nn] : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.s)[nn]);
  };
  if constexpr (ACT != 0) {
    // the bf16 GEMV outputs, then the activation with the row kernel's roundings
    const int n0 = tile0 * 16 + 4 * (lane >> 4);
    const int Nout = ACT == 1 ? p.half_tiles * 16 : p.N;
    if (n0 >= Nout) return;
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nn = n0 + r;
      if (nn >= Nout) { o[r] = 0.0f; continue; }
      const float g = round_bf16(acc[0][r] * scale_at(nn));
      const float u = ACT == 1 ? round_bf16(acc[1][r] * scale_at(p.half_tiles * 16 + nn))
                               : bf16_to_f32(p.mul[int64_t(m) * p.ldm + nn]);
      o[r] = round_bf16(round_bf16(gelu_tanh_f32(g)) * u);
    }
    uint16_t* dst = p.y + int64_t(m) * p.ldy + n0;
    if (n0 + 3 < Nout && ((reinterpret_cast<uintptr_t>(dst) & 7) == 0)) {
      *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n0 + r < Nout) dst[r] = f32_to_bf16(o[r]);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int n0 = (tile0 + t) * 16 + 4 * (lane >> 4);
    if (n0 >= p.N) continue;
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nn = n0 + r;
      float sc = 0.0f;
      if (nn < p.N) sc = p.s_f32 ? reinterpret_cast<const float*>(p.s)[nn]
                                 : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.s)[nn]);
      o[r] = acc[t][r] * sc;
    }
    uint16_t* dst = p.y + int64_t(m) * p.ldy + n0;
    if (n0 + 3 < p.N && ((reinterpret_cast<uintptr_t>(dst) & 7) == 0)) {
      *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n0 + r < p.N) dst[r] = f32_to_bf16(o[r]);
    }
  }
}

// Row-major int8 W [N, K] (ld = ldw) -> GEMV fragment layout, one thread per 16-byte piece;
// rows past N and k past K are zero.
__global__ __launch_bounds__(256) void pack_gemv_weight_kernel(const int8_t* __restrict__ w, int64_t ldw, int N, int K,
                                                               int KB, int64_t npieces, int8_t* __restrict__ out) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (c >= npieces) return;
  const int lane = int(c & 63);
  const int64_t f = c >> 6;
  const int t = int(f / KB), kb = int(f % KB);
  const int row = 16 * t + (lane & 15);
  const int k = 64 * kb + 16 * (lane >> 4);
  v4u v = {0u, 0u, 0u, 0u};
  if (row < N && k < K) v = *reinterpret_cast<const v4u*>(w + int64_t(row) * ldw + k);
  *reinterpret_cast<v4u*>(out + c * 16) = v;
}

static int gemv_cu_count() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

// Waves of a workgroup sharing one n-tile's K range on the few-tile shapes: doubled up to 16 while
// the chip holds fewer than ~4096 waves and each wave keeps two k-blocks, but not to 16 (1024-thread
// workgroups, one per CU) when there are more tiles than CUs: those would run in two rounds, where 8
// (two workgroups per CU) runs in one (the full-attention qkv, N = 5120: 12.5 -> 7.5 us).
static int few_tile_split(int64_t ntiles, int KB) {
  int split = 1;
  while (split < 16 && ntiles * split < 4096 && split * 2 <= KB) split *= 2;
  if (split == 16 && ntiles > gemv_cu_count()) split = 8;
  return split;
}

template <bool PACKED>
static void gemv_launch(const GemvParams& p0, hipStream_t stream) {
  GemvParams p = p0;
  const int64_t ntiles = (p.N + 15) / 16;
  if (ntiles >= 4096) {
    // Many n-tiles (the LM head): each activation fragment serves two (M <= 8) or four
    // weight tiles per wave.
    p.split = 1;
    if (p.M <= 8) {
      const int64_t groups = (ntiles + 1) / 2;
      gemv_kernel<2, 4, PACKED, 4><<<unsigned((groups + 3) / 4), 256, 0, stream>>>(p);
    } else {
      const int64_t groups = (ntiles + 3) / 4;
      gemv_kernel<4, 2, PACKED, 4><<<unsigned((groups + 3) / 4), 256, 0, stream>>>(p);
    }
  } else {
    // Few n-tiles (the per-layer decode shapes: 96-768 tiles): one tile per group of `split`
    // waves that share its K range, up to 16 waves of one workgroup, aiming for ~4096 waves over
    // the chip's 1024 SIMDs, each with at least two k-blocks.  The weights here are 3-19 MB, so
    // what bounds them is how many bytes are in flight: with at most four waves per tile the
    // down projection (96 tiles) ran 384 waves and reached ~1 TB/s.
    const int split = few_tile_split(ntiles, p.KB);
    p.split = split;
    if (split <= 4) {
      const int gpb = 4 / split;
      gemv_kernel<1, 4, PACKED, 4><<<unsigned((ntiles + gpb - 1) / gpb), 256, 0, stream>>>(p);
    } else if (split == 8) {
      gemv_kernel<1, 4, PACKED, 8><<<unsigned(ntiles), 512, 0, stream>>>(p);
    } else if ((p.KB + 15) / 16 > 4 && (p.KB + 15) / 16 <= 6) {
      // five or six k-blocks per wave (the down projection, K=6144): all of them in one round
      // trip instead of two (M=1 cold token 837 -> 826 us)
      gemv_kernel<1, 6, PACKED, 16><<<unsigned(ntiles), 1024, 0, stream>>>(p);
    } else {
      gemv_kernel<1, 4, PACKED, 16><<<unsigned(ntiles), 1024, 0, stream>>>(p);
    }
  }
}

// The few-tile launch with an activation epilogue: ACT 1 over I / 16 gate/up tile pairs (two tiles
// per wave), ACT 2 over the N / 16 tiles.  The split and the unroll depth are the plain launch's
// for the whole N (gemv_launch), so every tile's sum is added in the same order and the result is
// the plain GEMV's, bit for bit, before the activation.  ACT 0 is the plain few-tile launch; PRO
// (1..3, the prologue row's chunks per lane) adds the row prologue.
template <bool PACKED, int ACT, int PRO = 0>
static void gemv_launch_act(const GemvParams& p0, hipStream_t stream) {
  GemvParams p = p0;
  const int64_t ntiles = (p.N + 15) / 16;
  const int64_t groups = ACT == 1 ? p.half_tiles : ntiles;
  const int split = few_tile_split(ntiles, p.KB);
  p.split = split;
  constexpr int TPW = ACT == 1 ? 2 : 1;
  if (split <= 4) {
    const int gpb = 4 / split;
    gemv_kernel<TPW, 4, PACKED, 4, ACT, PRO><<<unsigned((groups + gpb - 1) / gpb), 256, 0, stream>>>(p);
  } else if (split == 8) {
    gemv_kernel<TPW, 4, PACKED, 8, ACT, PRO><<<unsigned(groups), 512, 0, stream>>>(p);
  } else if (!PRO && (p.KB + 15) / 16 > 4 && (p.KB + 15) / 16 <= 6) {  // K > 4096: never with the prologue
    gemv_kernel<TPW, 6, PACKED, 16, ACT, 0><<<unsigned(groups), 1024, 0, stream>>>(p);
  } else {
    gemv_kernel<TPW, 4, PACKED, 16, ACT, PRO><<<unsigned(groups), 1024, 0, stream>>>(p);
  }
}

}  // namespace w8a8

using namespace w8a8;

extern "C" int64_t w8a8_gemv_packed_bytes(int64_t N, int64_t K) {
  if (N < 1 || K < 1 || N > INT32_MAX || K > INT32_MAX) return -1;
  return (N + 15) / 16 * ((K + 63) / 64) * 1024;
}

extern "C" int w8a8_pack_gemv_weight(const int8_t* w, int64_t ldw, int64_t N, int64_t K, int8_t* packed,
                                     hipStream_t stream) {
  if (!w || !packed) return fail(W8A8_EINVAL, "pack_gemv_weight: null pointer");
  if (N < 1 || K < 16 || ldw < K) return fail(W8A8_EINVAL, "pack_gemv_weight: bad shape N=%lld K=%lld ldw=%lld",
                                              (long long)N, (long long)K, (long long)ldw);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "pack_gemv_weight: K=%lld must be a multiple of 16", (long long)K);
  if (ldw % 16 != 0 || (uintptr_t)w % 16 != 0 || (uintptr_t)packed % 16 != 0)
    return fail(W8A8_EALIGN, "pack_gemv_weight: w rows and packed must be 16-byte aligned");
  const int64_t bytes = w8a8_gemv_packed_bytes(N, K);
  if (bytes < 0 || bytes > INT32_MAX + 1ll) return fail(W8A8_ENOTSUP, "pack_gemv_weight: packed weight above 2 GiB");
  const int64_t pieces = bytes / 16;
  pack_gemv_weight_kernel<<<unsigned((pieces + 255) / 256), 256, 0, stream>>>(w, ldw, int(N), int(K),
                                                                            int((K + 63) / 64), pieces, packed);
  return check_launch("pack_gemv_weight");
}

extern "C" int w8a8_gemv_packed_bf16(const uint16_t* x, int64_t ldx, int64_t M, const int8_t* packed, int64_t N,
                                     int64_t K, const void* scales, int scale_is_f32, uint16_t* y, int64_t ldy,
                                     hipStream_t stream) {
  if (!x || !packed || !scales || !y) return fail(W8A8_EINVAL, "gemv_packed: null pointer");
  if (M < 1 || M > 16) return fail(W8A8_EINVAL, "gemv_packed: M=%lld, the GEMV takes 1..16 rows", (long long)M);
  if (N < 1 || K < 16) return fail(W8A8_EINVAL, "gemv_packed: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "gemv_packed: K=%lld must be a multiple of 16", (long long)K);
  if (ldx < K || ldy < N) return fail(W8A8_EINVAL, "gemv_packed: leading dimension too small");
  if (ldx % 8 != 0 || (uintptr_t)x % 16 != 0 || (uintptr_t)packed % 16 != 0)
    return fail(W8A8_EALIGN, "gemv_packed: x rows and the packed weight must be 16-byte aligned");
  const int64_t wb = w8a8_gemv_packed_bytes(N, K);
  const int64_t xb = ((M - 1) * ldx + K) * 2;
  if (wb > INT32_MAX || xb > INT32_MAX) return fail(W8A8_ENOTSUP, "gemv_packed: operands above 2 GiB");
  GemvParams p;
  p.x = x; p.ldx = ldx; p.w = packed; p.ldw = 0; p.s = scales; p.s_f32 = scale_is_f32 ? 1 : 0;
  p.y = y; p.ldy = ldy; p.x_bytes = uint32_t(xb); p.w_bytes = uint32_t(wb);
  p.M = int(M); p.N = int(N); p.K = int(K); p.KB = int((K + 63) / 64);
  gemv_launch<true>(p, stream);
  return check_launch("gemv_packed_bf16");
}

extern "C" int w8a8_gemv_packed_act_bf16(const uint16_t* x, int64_t ldx, int64_t M, const int8_t* packed, int64_t N,
                                         int64_t K, const void* scales, int scale_is_f32, int act, const uint16_t* mul,
                                         int64_t ldm, uint16_t* y, int64_t ldy, hipStream_t stream) {
  if (!x || !packed || !scales || !y || (act == 2 && !mul)) return fail(W8A8_EINVAL, "gemv_packed_act: null pointer");
  if (act != 1 && act != 2) return fail(W8A8_EINVAL, "gemv_packed_act: act %d (1: GELU pair, 2: GELU times mul)", act);
  if (M < 1 || M > 16) return fail(W8A8_EINVAL, "gemv_packed_act: M=%lld, the GEMV takes 1..16 rows", (long long)M);
  if (N < 1 || K < 16) return fail(W8A8_EINVAL, "gemv_packed_act: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "gemv_packed_act: K=%lld must be a multiple of 16", (long long)K);
  if (act == 1 && N % 32 != 0)
    return fail(W8A8_ENOTSUP, "gemv_packed_act: a GELU pair needs N = 2I with I a multiple of 16, got N=%lld",
                (long long)N);
  const int64_t nout = act == 1 ? N / 2 : N;
  if ((N + 15) / 16 >= 4096) return fail(W8A8_ENOTSUP, "gemv_packed_act: N=%lld above the few-tile shapes", (long long)N);
  if (ldx < K || ldy < nout || (act == 2 && ldm < N)) return fail(W8A8_EINVAL, "gemv_packed_act: leading dimension too small");
  if (ldx % 8 != 0 || (uintptr_t)x % 16 != 0 || (uintptr_t)packed % 16 != 0)
    return fail(W8A8_EALIGN, "gemv_packed_act: x rows and the packed weight must be 16-byte aligned");
  const int64_t wb = w8a8_gemv_packed_bytes(N, K);
  const int64_t xb = ((M - 1) * ldx + K) * 2;
  if (wb > INT32_MAX || xb > INT32_MAX) return fail(W8A8_ENOTSUP, "gemv_packed_act: operands above 2 GiB");
  GemvParams p{};
  p.x = x; p.ldx = ldx; p.w = packed; p.ldw = 0; p.s = scales; p.s_f32 = scale_is_f32 ? 1 : 0;
  p.y = y; p.ldy = ldy; p.x_bytes = uint32_t(xb); p.w_bytes = uint32_t(wb);
  p.M = int(M); p.N = int(N); p.K = int(K); p.KB = int((K + 63) / 64);
  p.mul = mul; p.ldm = ldm; p.half_tiles = int(N / 32);
  if (act == 1)
    gemv_launch_act<true, 1>(p, stream);
  else
    gemv_launch_act<true, 2>(p, stream);
  return check_launch("gemv_packed_act_bf16");
}

static bool overlaps(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
  if (!a || !b) return false;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  return a0 < b0 + uintptr_t(bbytes) && b0 < a0 + uintptr_t(abytes);
}

extern "C" int w8a8_gemv_packed_norm_bf16(const uint16_t* y, const uint16_t* res, const uint16_t* w1,
                                          const uint16_t* scalar, int norm2, const uint16_t* w2, float eps, uint16_t* h,
                                          const int8_t* packed, int64_t N, int64_t K, const void* scales,
                                          int scale_is_f32, int act, const uint16_t* mul, uint16_t* out,
                                          hipStream_t stream) {
  const char* what = "gemv_packed_norm";
  if (!y || !packed || !scales || !out || (act == 2 && !mul)) return fail(W8A8_EINVAL, "%s: null pointer", what);
  if (act < 0 || act > 2) return fail(W8A8_EINVAL, "%s: act %d (0: none, 1: GELU pair, 2: GELU times mul)", what, act);
  if (N < 1 || K < 16) return fail(W8A8_EINVAL, "%s: bad shape N=%lld K=%lld", what, (long long)N, (long long)K);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "%s: K=%lld must be a multiple of 16", what, (long long)K);
  if (K > 1536) return fail(W8A8_ENOTSUP, "%s: K=%lld above the prologue's row of 1536", what, (long long)K);
  if ((N + 15) / 16 >= 4096) return fail(W8A8_ENOTSUP, "%s: N=%lld above the few-tile shapes", what, (long long)N);
  if (act == 1 && N % 32 != 0)
    return fail(W8A8_ENOTSUP, "%s: a GELU pair needs N = 2I with I a multiple of 16, got N=%lld", what, (long long)N);
  for (const void* q : {static_cast<const void*>(y), static_cast<const void*>(res), static_cast<const void*>(w1),
                        static_cast<const void*>(w2), static_cast<const void*>(h), static_cast<const void*>(packed)})
    if ((reinterpret_cast<uintptr_t>(q) & 15) != 0)
      return fail(W8A8_EALIGN, "%s: the rows, norm weights and packed weight must be 16-byte aligned", what);
  const int64_t nout = act == 1 ? N / 2 : N;
  const int64_t rb = K * 2, ob = nout * 2;
  // every workgroup reads y and res while workgroup 0 writes h and all of them write out
  if (overlaps(h, rb, y, rb) || overlaps(h, rb, res, rb) || overlaps(h, rb, out, ob))
    return fail(W8A8_EINVAL, "%s: h must not overlap y, res or out", what);
  if (overlaps(out, ob, y, rb) || overlaps(out, ob, res, rb) || (act == 2 && overlaps(out, ob, mul, N * 2)))
    return fail(W8A8_EINVAL, "%s: out must not overlap y, res or mul", what);
  const int64_t wb = w8a8_gemv_packed_bytes(N, K);
  if (wb > INT32_MAX) return fail(W8A8_ENOTSUP, "%s: packed weight above 2 GiB", what);
  GemvParams p{};
  p.x = nullptr; p.ldx = K; p.w = packed; p.ldw = 0; p.s = scales; p.s_f32 = scale_is_f32 ? 1 : 0;
  p.y = out; p.ldy = nout; p.x_bytes = 0; p.w_bytes = uint32_t(wb);
  p.M = 1; p.N = int(N); p.K = int(K); p.KB = int((K + 63) / 64);
  p.mul = mul; p.ldm = N; p.half_tiles = int(N / 32);
  p.pro_y = y; p.pro_res = res; p.pro_w1 = w1; p.pro_scalar = scalar; p.pro_w2 = w2; p.pro_h = h;
  p.pro_eps = eps; p.pro_norm2 = norm2 ? 1 : 0;
  // the row kernel's chunks of 8 per lane for a row of K (K <= 1536: one wave, at most three)
  p.pro_ch = int((K + 511) / 512);
#define W8A8_NORM_GEMV(CH)                                                   \
  do {                                                                       \
    if (act == 0) gemv_launch_act<true, 0, CH>(p, stream);                   \
    else if (act == 1) gemv_launch_act<true, 1, CH>(p, stream);              \
    else gemv_launch_act<true, 2, CH>(p, stream);                            \
  } while (0)
  if (p.pro_ch == 1) W8A8_NORM_GEMV(1);
  else if (p.pro_ch == 2) W8A8_NORM_GEMV(2);
  else W8A8_NORM_GEMV(3);
#undef W8A8_NORM_GEMV
  return check_launch("gemv_packed_norm_bf16");
}

extern "C" int w8a8_gemv_packed_attn_merge_bf16(const void* workspace, const int32_t* q_pos, int64_t H, int64_t KV,
                                                int64_t Tk, int64_t D, int64_t window, float scale,
                                                const int8_t* packed, int64_t N, const void* scales, int scale_is_f32,
                                                uint16_t* out, hipStream_t stream) {
  const char* what = "gemv_packed_attn_merge";
  if (!workspace || !q_pos || !packed || !scales || !out) return fail(W8A8_EINVAL, "%s: null pointer", what);
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 16)
    return fail(W8A8_EINVAL, "%s: H=%lld KV=%lld (H a multiple of KV, at most 16 per KV head)", what, (long long)H,
                (long long)KV);
  if (D != 128 && D != 256 && D != 512) return fail(W8A8_ENOTSUP, "%s: head_dim %lld", what, (long long)D);
  if (Tk < 1 || Tk > INT32_MAX || window < 0 || window > INT32_MAX)
    return fail(W8A8_EINVAL, "%s: Tk=%lld window=%lld", what, (long long)Tk, (long long)window);
  const int nchunk_grid = decode_grid_chunks(D, Tk, window);
  if (nchunk_grid > DEC_MERGE_IN_GEMV_CHUNKS)
    return fail(W8A8_ENOTSUP, "%s: %d key chunks (at most %d)", what, nchunk_grid, DEC_MERGE_IN_GEMV_CHUNKS);
  const int64_t K = H * D;
  if (K > 4096) return fail(W8A8_ENOTSUP, "%s: H * D = %lld above 4096", what, (long long)K);
  if (N < 1 || (N + 15) / 16 >= 4096) return fail(W8A8_ENOTSUP, "%s: N=%lld outside the few-tile shapes", what, (long long)N);
  if (!(scale > 0.0f) || scale == __builtin_inff()) return fail(W8A8_EINVAL, "%s: scale must be positive", what);
  if ((uintptr_t)workspace % 16 || (uintptr_t)packed % 16 || (uintptr_t)q_pos % 4)
    return fail(W8A8_EALIGN, "%s: workspace and packed 16-byte aligned, q_pos 4-byte aligned", what);
  const int64_t wb = w8a8_gemv_packed_bytes(N, K);
  if (wb > INT32_MAX) return fail(W8A8_ENOTSUP, "%s: packed weight above 2 GiB", what);
  GemvParams p{};
  p.x = nullptr; p.ldx = K; p.w = packed; p.ldw = 0; p.s = scales; p.s_f32 = scale_is_f32 ? 1 : 0;
  p.y = out; p.ldy = N; p.x_bytes = 0; p.w_bytes = uint32_t(wb);
  p.M = 1; p.N = int(N); p.K = int(K); p.KB = int((K + 63) / 64);
  const int G = int(H / KV);
  p.m_po = static_cast<const float*>(workspace);
  p.m_ml = p.m_po + int64_t(KV) * nchunk_grid * G * D;
  p.m_pos = q_pos; p.m_window = int(window); p.m_nchunk_grid = nchunk_grid; p.m_G = G; p.m_D = int(D);
  p.m_chunk = dec_chunk(int(D));
  p.m_c = scale * 1.4426950408889634f;  // the attention's exp2 factor, computed as it computes it
  gemv_launch_act<true, 0, 4>(p, stream);
  return check_launch("gemv_packed_attn_merge_bf16");
}

extern "C" int w8a8_gemv_bf16(const uint16_t* x, int64_t ldx, int64_t M, const int8_t* w, int64_t ldw, int64_t N,
                              int64_t K, const void* scales, int scale_is_f32, uint16_t* y, int64_t ldy,
                              hipStream_t stream) {
  if (!x || !w || !scales || !y) return fail(W8A8_EINVAL, "gemv: null pointer");
  if (M < 1 || M > 16) return fail(W8A8_EINVAL, "gemv: M=%lld, the GEMV takes 1..16 rows", (long long)M);
  if (N < 1 || K < 16) return fail(W8A8_EINVAL, "gemv: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  if (K % 16 != 0) return fail(W8A8_ENOTSUP, "gemv: K=%lld must be a multiple of 16", (long long)K);
  if (ldx < K || ldw < K || ldy < N) return fail(W8A8_EINVAL, "gemv: leading dimension too small");
  if (ldx % 8 != 0 || ldw % 16 != 0 || (uintptr_t)x % 16 != 0 || (uintptr_t)w % 16 != 0)
    return fail(W8A8_EALIGN, "gemv: x and w rows must be 16-byte aligned (ldx %% 8, ldw %% 16)");
  const int64_t wb = (N - 1) * ldw + K;
  const int64_t xb = ((M - 1) * ldx + K) * 2;
  if (wb > INT32_MAX || xb > INT32_MAX) return fail(W8A8_ENOTSUP, "gemv: operands above 2 GiB");
  GemvParams p;
  p.x = x; p.ldx = ldx; p.w = w; p.ldw = ldw; p.s = scales; p.s_f32 = scale_is_f32 ? 1 : 0;
  p.y = y; p.ldy = ldy; p.x_bytes = uint32_t(xb); p.w_bytes = uint32_t(wb);
  p.M = int(M); p.N = int(N); p.K = int(K); p.KB = int((K + 63) / 64);
  gemv_launch<false>(p, stream);
  return check_launch("gemv_bf16");
}
