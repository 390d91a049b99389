// int8 x int8 -> int32 GEMM on CDNA4 MFMA (v_mfma_i32_32x32x32_i8), with fused epilogues.
//
// Replaces the Triton kernel matmul_i8_k (npu_kernels.py:40-56): C[M,N] = A[M,K] @ W with
// int32 accumulation, W held resident in HBM in the packed fragment layout written by
// pack_weight (quant.hip), and the reference's neighbouring element-wise work fused into the
// store:
//   EPI_I32       C int32                                     (npu_kernels.py:56)
//   EPI_BF16      bf16((acc * sx[m]) * sw[n])                 (_deq, pipeline.py:55-57)
//   EPI_GELU      bf16(gelu_tanh(gate) * up) on the dequantised bf16 gate/up pair
//                                                             (k_gelu, pipeline.py:102-107)
//   EPI_RESID     bf16(res + bf16(dequant))                   (plain residual add)
//
// Data movement.  A block owns a BM x BN tile of C and walks K in k-tiles of 64.  Every
// operand fragment (32 rows x 32 k, 1 KiB, lane l's 16 bytes = row l%32, k 16*(l/32)..+16,
// the MFMA's operand order) goes from HBM straight into an NS-deep LDS ring with
// buffer_load_dwordx4 ... lds, NS-1 k-tiles ahead of the multiply.  Lane l's 16 bytes land at
// 16*l of the fragment, so every ds_read_b128 is a contiguous, conflict-free 1 KiB.  No VGPRs
// are spent on staging and no fence drains the in-flight loads: each wave waits on its own
// vmcnt and meets the others at a bare s_barrier.  Buffer loads past the A / W extents return
// zero, which is how ragged M, N and K are handled without branches in the loop.
//
// Compute.  WGM x WGN waves, each owning (BM/WGM) x (BN/WGN) of C as 32 x 32 MFMA tiles.  The
// MFMA is issued as W-fragment x A-fragment, so a lane's accumulator holds four consecutive
// output columns of one row per register group and stores go out as 16-byte vectors.
#include "gemm.h"
#include "w8a8_common.h"

namespace w8a8 {

typedef int v16i __attribute__((ext_vector_type(16)));

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in bits
// [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}


// Epilogue for one 32x32 accumulator tile.  Lane l holds row m and, for register group
// g = 0..3, packed columns t*32 + 8g + lcol + r (r = 0..3, lcol = 4*(l/32)).  sxm is the row's
// scale; swt points at the LDS copy of the per-channel scales of this tile's packed columns
// (swt[8g + r] belongs to packed column t*32 + 8g + lcol + r; for GELU, swt + 32 is the up tile).
template <int EPI>
__device__ __forceinline__ void store_tile(const GemmParams& p, const v16i& acc, const v16i* acc_up, int m, int t,
                                           int lcol, float sxm, const float* swt) {
  if constexpr (EPI == EPI_I32) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = t * 32 + 8 * g + lcol;
      int32_t* dst = p.c + int64_t(m) * p.ldc + n;
      const v4i v = {acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
      if (p.vec_store && n + 3 < p.N) {
        *reinterpret_cast<v4i*>(dst) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < p.N) dst[r] = v[r];
      }
    }
  } else if constexpr (EPI == EPI_BF16 || EPI == EPI_RESID) {
    // The residual may alias the output: every residual value this lane needs is loaded before
    // any of its stores, and each element is read and written by this lane only.
    v2u rv[4];
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = t * 32 + 8 * g + lcol;
        const uint16_t* rs = p.res + int64_t(m) * p.ldr + n;
        if (p.res_vec && n + 3 < p.N) {
          rv[g] = *reinterpret_cast<const v2u*>(rs);
        } else {
          uint32_t h[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) h[r] = n + r < p.N ? rs[r] : 0u;
          rv[g] = v2u{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = t * 32 + 8 * g + lcol;
      const v4f sw = *reinterpret_cast<const v4f*>(swt + 8 * g);
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = bf16_to_f32(f32_to_bf16((float(acc[4 * g + r]) * sxm) * sw[r]));
      if constexpr (EPI == EPI_RESID) {
        y[0] += bf16_to_f32(uint16_t(rv[g][0]));
        y[1] += bf16_to_f32(uint16_t(rv[g][0] >> 16));
        y[2] += bf16_to_f32(uint16_t(rv[g][1]));
        y[3] += bf16_to_f32(uint16_t(rv[g][1] >> 16));
      }
      uint16_t* dst = p.out + int64_t(m) * p.ldo + n;
      if (p.vec_store && n + 3 < p.N) {
        *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < p.N) dst[r] = f32_to_bf16(y[r]);
      }
    }
  } else if constexpr (EPI == EPI_GELU) {
    // t is an even (gate) tile u = t/2; acc_up is the matching up tile t+1.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = (t >> 1) * 32 + 8 * g + lcol;  // logical gate column
      const v4f swg = *reinterpret_cast<const v4f*>(swt + 8 * g);
      const v4f swu = *reinterpret_cast<const v4f*>(swt + 32 + 8 * g);
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gate = bf16_to_f32(f32_to_bf16((float(acc[4 * g + r]) * sxm) * swg[r]));
        const float up = bf16_to_f32(f32_to_bf16((float((*acc_up)[4 * g + r]) * sxm) * swu[r]));
        const float ge = bf16_to_f32(f32_to_bf16(gelu_tanh_f32(gate)));
        o[r] = ge * up;
      }
      uint16_t* dst = p.out + int64_t(m) * p.ldo + c;
      if (p.vec_store && c + 3 < p.I) {
        *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c + r < p.I) dst[r] = f32_to_bf16(o[r]);
      }
    }
  }
}

// int32 store of a wave's WTM x WTN accumulator tiles (rows m0 + 32 i .., packed column tiles
// t0 + j) through a 4 KiB LDS area private to the wave, so that every store instruction writes
// eight whole 128-byte lines (8 rows x 32 columns) instead of 32 bytes of each of 32 rows.  Lane l
// holds row l % 32 of a tile and its 16-byte column chunks 2g + l / 32 (g = 0..3); chunk c of row r
// sits at chunk position c ^ (r / 2 % 8) of a 128-byte LDS row, which keeps both the writes (16
// rows of one chunk per 16 lanes) and the reads (two whole rows per 16 lanes) free of bank
// conflicts.  The wave's LDS operations run in the order it issues them, so the reads see the
// writes and the next tile's writes follow this tile's reads without a barrier.
template <int WTM, int WTN>
__device__ __forceinline__ void store_i32_lines(const GemmParams& p, const v16i (&acc)[WTM][WTN], char* st, int m0,
                                                int t0, int lane) {
  const int lrow = lane & 31, half = lane >> 5;
  const int rr = lane >> 3, c = lane & 7;
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cw = 2 * g + half;
        *reinterpret_cast<v4i*>(st + lrow * 128 + 16 * (cw ^ ((lrow >> 1) & 7))) =
            v4i{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = 8 * k + rr;
        const v4i v = *reinterpret_cast<const v4i*>(st + r * 128 + 16 * (c ^ ((r >> 1) & 7)));
        const int m = m0 + 32 * i + r;
        const int n = (t0 + j) * 32 + 4 * c;
        if (m < p.M) {
          int32_t* dst = p.c + int64_t(m) * p.ldc + n;
          if (p.vec_store && n + 3 < p.N) {
            *reinterpret_cast<v4i*>(dst) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < p.N) dst[e] = v[e];
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
}

// bf16 epilogue values of one 32x32 output tile, as lane l's row l % 32 and columns 8g + 4(l / 32)
// .. +3 (g = 0..3), packed two per dword: `bf16((acc sx) sw)` (EPI_BF16 and, before its residual,
// EPI_RESID) or `bf16(bf16(gelu_tanh(gate)) up)` from the gate tile `acc` and the up tile `acc_up`
// (EPI_GELU).  The same operations, in the same order, as store_tile.
template <int EPI>
__device__ __forceinline__ void tile_bf16(const v16i& acc, const v16i* acc_up, float sxm, const float* swt, v2u (&y)[4]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float o[4];
    if constexpr (EPI == EPI_GELU) {
      const v4f swg = *reinterpret_cast<const v4f*>(swt + 8 * g);
      const v4f swu = *reinterpret_cast<const v4f*>(swt + 32 + 8 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gate = bf16_to_f32(f32_to_bf16((float(acc[4 * g + r]) * sxm) * swg[r]));
        const float up = bf16_to_f32(f32_to_bf16((float((*acc_up)[4 * g + r]) * sxm) * swu[r]));
        const float ge = bf16_to_f32(f32_to_bf16(gelu_tanh_f32(gate)));
        o[r] = ge * up;
      }
    } else {
      const v4f sw = *reinterpret_cast<const v4f*>(swt + 8 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (float(acc[4 * g + r]) * sxm) * sw[r];
    }
    y[g] = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
}

// Store of one 32x32 bf16 output tile (rows m0 .., columns n0 .., n < ncols) through a 2 KiB LDS
// area private to the wave, so that each store instruction writes 16 rows x 64 contiguous bytes
// instead of 16 bytes of each of 32 rows.  y is tile_bf16's lane layout; the 16-byte column chunk c
// of row r sits at chunk position c ^ (r / 4 % 4).  EPI_RESID adds the residual after the
// exchange, each lane reading the residual elements it then writes (the residual may alias the
// output).  The wave's LDS operations run in the order it issues them.
template <int EPI>
__device__ __forceinline__ void store_bf16_lines(const GemmParams& p, const v2u (&y)[4], char* st, int m0, int n0,
                                                 int ncols, int lane) {
  const int lrow = lane & 31, half = lane >> 5;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<v2u*>(st + lrow * 64 + 16 * (g ^ ((lrow >> 2) & 3)) + 8 * half) = y[g];
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int r = 16 * k + (lane >> 2), c = lane & 3;
    v4u v = *reinterpret_cast<const v4u*>(st + r * 64 + 16 * (c ^ ((r >> 2) & 3)));
    const int m = m0 + r, n = n0 + 8 * c;
    if (m >= p.M) continue;
    uint16_t* dst = p.out + int64_t(m) * p.ldo + n;
    const bool whole = n + 7 < ncols;
    if constexpr (EPI == EPI_RESID) {
      const uint16_t* rs = p.res + int64_t(m) * p.ldr + n;
      uint16_t rv[8];
      if (whole && (reinterpret_cast<uintptr_t>(rs) & 15) == 0) {
        const v4u t = *reinterpret_cast<const v4u*>(rs);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          rv[2 * e] = uint16_t(t[e]);
          rv[2 * e + 1] = uint16_t(t[e] >> 16);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) rv[e] = n + e < ncols ? rs[e] : uint16_t(0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16_to_f32(uint16_t(v[e])) + bf16_to_f32(rv[2 * e]);
        const float hi = bf16_to_f32(uint16_t(v[e] >> 16)) + bf16_to_f32(rv[2 * e + 1]);
        v[e] = pack_bf16x2(lo, hi);
      }
    }
    if (whole && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
      *reinterpret_cast<v4u*>(dst) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < ncols) dst[e] = uint16_t(v[e >> 1] >> (16 * (e & 1)));
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// Epilogue of gemm_kernel, from the accumulators staged in LDS.  `red` holds the KW waves'
// partial tiles (KW = 1: the one tile) as row-major int32 [KW][BM][LDR].  Thread q of a row (TPR = BN/16 threads per row) adds the partials of 4
// columns in each quarter of the tile, columns 4q + (BN/4)*st (st = 0..3), so in each step the
// TPR threads of a row read and store one contiguous run.  For GELU (BN of 64 or 128) the gate
// column c of a [gate | up] pair of 32-channel tiles sits in quarter st and its up column c + 32
// in quarter st + 128/BN.
template <int EPI, int BM, int BN, int KW, int NW, int LDR>
__device__ __forceinline__ void ksplit_epilogue(const GemmParams& p, const int32_t* red, const float* s_scale,
                                                int m0, int t0) {
  constexpr int TPR = BN / 16;
  constexpr int RPP = NW * 64 / TPR;
  static_assert(RPP * TPR == NW * 64, "each row is covered by whole threads");
  static_assert(EPI != EPI_GELU || BN == 64 || BN == 128, "GELU pairing needs a 64- or 128-wide tile");
  const int q = int(threadIdx.x) % TPR;
  for (int r = int(threadIdx.x) / TPR; r < BM; r += RPP) {
    const int m = m0 + r;
    if (m >= p.M) break;
    v4i acc[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int col = 4 * q + (BN / 4) * st;
      acc[st] = *reinterpret_cast<const v4i*>(red + r * LDR + col);
#pragma unroll
      for (int k = 1; k < KW; ++k) acc[st] += *reinterpret_cast<const v4i*>(red + (k * BM + r) * LDR + col);
    }
    const float sxm = EPI == EPI_I32 ? 0.0f : s_scale[r];
    if constexpr (EPI == EPI_I32) {
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int n = t0 * 32 + 4 * q + (BN / 4) * st;
        int32_t* dst = p.c + int64_t(m) * p.ldc + n;
        if (p.vec_store && n + 3 < p.N) {
          *reinterpret_cast<v4i*>(dst) = acc[st];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n + i < p.N) dst[i] = acc[st][i];
        }
      }
    } else if constexpr (EPI == EPI_BF16 || EPI == EPI_RESID) {
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int col = 4 * q + (BN / 4) * st;
        const int n = t0 * 32 + col;
        const v4f sw = *reinterpret_cast<const v4f*>(s_scale + BM + col);
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = round_bf16((float(acc[st][i]) * sxm) * sw[i]);
        if constexpr (EPI == EPI_RESID) {
          const uint16_t* rs = p.res + int64_t(m) * p.ldr + n;
          if (p.res_vec && n + 3 < p.N) {
            const v2u rv = *reinterpret_cast<const v2u*>(rs);
            y[0] += bf16_to_f32(uint16_t(rv[0]));
            y[1] += bf16_to_f32(uint16_t(rv[0] >> 16));
            y[2] += bf16_to_f32(uint16_t(rv[1]));
            y[3] += bf16_to_f32(uint16_t(rv[1] >> 16));
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (n + i < p.N) y[i] += bf16_to_f32(rs[i]);
          }
        }
        uint16_t* dst = p.out + int64_t(m) * p.ldo + n;
        if (p.vec_store && n + 3 < p.N) {
          *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n + i < p.N) dst[i] = f32_to_bf16(y[i]);
        }
      }
    } else {  // EPI_GELU
      constexpr int UP = 128 / BN;  // quarters between a gate column and its up column
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        if ((((BN / 4) * st) / 32) % 2 != 0) continue;  // up quarter: handled with its gate quarter
        const int su = st + UP < 4 ? st + UP : st;         // the up quarter (always st + UP here)
        const int col = 4 * q + (BN / 4) * st;
        const int c = ((t0 + col / 32) >> 1) * 32 + col % 32;  // gate / up channel
        const v4f swg = *reinterpret_cast<const v4f*>(s_scale + BM + col);
        const v4f swu = *reinterpret_cast<const v4f*>(s_scale + BM + col + 32);
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gate = round_bf16((float(acc[st][i]) * sxm) * swg[i]);
          const float up = round_bf16((float(acc[su][i]) * sxm) * swu[i]);
          o[i] = round_bf16(gelu_tanh_f32(gate)) * up;
        }
        uint16_t* dst = p.out + int64_t(m) * p.ldo + c;
        if (p.vec_store && c + 3 < p.I) {
          *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (c + i < p.I) dst[i] = f32_to_bf16(o[i]);
        }
      }
    }
  }
}

// Logical tile -> output tile.  Blocks are handed to the 8 XCDs round-robin (b % 8); xcd_remap
// gives each XCD a contiguous run of logical tiles, and the logical order walks groups of `gm` row
// tiles across all column tiles, so the ~32 blocks an XCD runs at once cover a compact
// gm x (32/gm) patch and share its A row-tiles and W column-tiles in that XCD's L2.
__device__ __forceinline__ void tile_coords(int t, int ntm, int ntn, int gm, int& tm, int& tn) {
  const int per_group = gm * ntn;
  const int first = (t / per_group) * gm;
  const int gsz = min(ntm - first, gm);
  const int r = t % per_group;
  tm = first + r % gsz;
  tn = r / gsz;
}

template <int BM, int BN, int WGM, int WGN, int KW, int KS, int NS, int EPI, bool A_PACKED, int MINB>
__global__ __launch_bounds__(WGM * WGN * KW * 64, MINB) void gemm_kernel(GemmParams p) {
  constexpr int NW = WGM * WGN * KW;  // KW waves share each output sub-tile, splitting its k-steps
  constexpr int MT = BM / 32;         // A row-tiles per block
  constexpr int NTB = BN / 32;        // W column-tiles per block
  constexpr int F = KS * (MT + NTB);  // fragments per k-tile (one ring slot)
  static_assert((KS * MT) % NW == 0 && (KS * NTB) % NW == 0, "each wave moves whole A and W fragments");
  constexpr int FA = KS * MT / NW, FB = KS * NTB / NW;  // fragments per wave per k-tile
  constexpr int FW = FA + FB;
  constexpr int WTM = MT / WGM;       // 32-row tiles per wave
  constexpr int WTN = NTB / WGN;      // 32-column tiles per wave
  static_assert(WTM * WGM == MT && WTN * WGN == NTB, "wave grid must divide the block tile");
  static_assert(EPI != EPI_GELU || (WTN % 2 == 0), "GELU pairs need an even tile count per wave");
  static_assert(KS % (2 * KW) == 0, "each wave's k-steps alternate between two register sets");
  constexpr int SW = KS / KW;  // k-steps per wave per k-tile
  static_assert(NS >= 2, "the ring needs one slot being read and one landing");
  static_assert(FW * (NS - 1) < 64, "outstanding loads must fit the 6-bit vmcnt");
  constexpr int NQ = WTM * WTN;                   // MFMAs per k-step
  constexpr int EARLY = NQ >= 8 ? NQ / 4 : 1;     // MFMAs issued before the next fragment reads

  // Slot layout: A fragments (s, mt) at (s*MT + mt) KiB, then W fragments (s, nt) at
  // (KS*MT + s*NTB + nt) KiB, s = 0 .. KS-1 the 32-wide k-steps of the k-tile.  After the NS
  // slots: the tile's per-row scales sx (first BM) and per-packed-column scales sw (next BN),
  // parked in LDS so the epilogue never waits on memory for them.  Ring and scales are one LDS
  // object: with a second one the compiler cannot tell the ring's fragment reads from the
  // in-flight DMA writes and waits for every outstanding load before each read, which removes
  // the prefetch.
  constexpr int NSCALE = EPI == EPI_I32 ? 0 : BM + BN;
  constexpr int SCALE_PER_THREAD = NSCALE ? (NSCALE + NW * 64 - 1) / (NW * 64) : 1;
  constexpr int RING = NS * F * 1024;
  __shared__ __attribute__((aligned(1024))) char lds[RING + NSCALE * 4];
  float* const s_scale = reinterpret_cast<float*>(lds + RING);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kw = wave / (WGM * WGN);  // this wave takes k-steps kw, kw + KW, ... of every k-tile
  const int wm = (wave % (WGM * WGN)) / WGN, wn = wave % WGN;

  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT + NTB - 1) / NTB;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, ntm * ntn), ntm, ntn, p.gm, tm, tn);
  const int m0 = tm * BM;
  const int t0 = tn * NTB;
  const int KT = (p.KF + KS - 1) / KS;  // k-tiles over the whole K
  // k-steps (of 32) in the last k-tile: K is padded to 64, not to 32 * KS.
  const int last_steps = p.KF - (KT - 1) * KS;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.wp, p.w_bytes);

  // Scales are fetched before the operand DMA starts and written to LDS once the prologue's
  // loads have landed, so their latency hides under the first k-tiles.
  float scale_v[SCALE_PER_THREAD];
#pragma unroll
  for (int u = 0; u < SCALE_PER_THREAD; ++u) {
    scale_v[u] = 0.0f;
    if constexpr (EPI != EPI_I32) {
      const int i = int(threadIdx.x) + u * NW * 64;
      if (i < BM) {
        if (m0 + i < p.M) scale_v[u] = p.sx[m0 + i];
      } else if (i < BM + BN) {
        const int pc = i - BM, tt = t0 + pc / 32;
        if constexpr (EPI == EPI_GELU) {
          const int c = (tt >> 1) * 32 + pc % 32;  // gate / up channel of interleaved tile tt
          if (c < p.I) scale_v[u] = p.sw[(tt & 1 ? p.I : 0) + c];
        } else {
          const int n = tt * 32 + pc % 32;
          if (n < p.N) scale_v[u] = p.sw[n];
        }
      }
    }
  }

  // This lane's byte offsets for k-tile 0 of each fragment it moves; fragment f = (s, mt) of
  // A is rows m0 + 32*mt + l%32, k 32*s + 16*(l/32) (row-major A: at row*lda + k; packed A: in
  // fragment (m0/32 + mt, s)); fragment f = (s, nt) of W is packed fragment (t0 + nt, s).
  uint32_t offa[FA], offb[FB];
#pragma unroll
  for (int i = 0; i < FA; ++i) {
    const int f = i * NW + wave;
    const int s = f / MT, mt = f % MT;
    if constexpr (A_PACKED)
      offa[i] = (uint32_t(m0 / 32 + mt) * uint32_t(p.KF) + uint32_t(s)) * 1024u + uint32_t(lane) * 16u;
    else
      offa[i] = uint32_t(m0 + mt * 32 + (lane & 31)) * uint32_t(p.lda) + uint32_t(s * 32 + (lane >> 5) * 16);
  }
#pragma unroll
  for (int i = 0; i < FB; ++i) {
    const int f = i * NW + wave;
    const int s = f / NTB, nt = f % NTB;
    offb[i] = (uint32_t(t0 + nt) * uint32_t(p.KF) + uint32_t(s)) * 1024u + uint32_t(lane) * 16u;
  }
  constexpr uint32_t A_STEP = A_PACKED ? KS * 1024u : KS * 32u;  // bytes per k-tile
  constexpr uint32_t W_STEP = KS * 1024u;

  // Fragments past K (a partial last k-tile) are loaded but never multiplied; loads past the
  // end of A or W read zero.
  auto issue = [&](int kt) {
    char* slot = lds + (kt % NS) * (F * 1024);
#pragma unroll
    for (int i = 0; i < FA; ++i) dma16(ra, slot + (i * NW + wave) * 1024, offa[i] + uint32_t(kt) * A_STEP);
#pragma unroll
    for (int i = 0; i < FB; ++i) dma16(rw, slot + (KS * MT + i * NW + wave) * 1024, offb[i] + uint32_t(kt) * W_STEP);
  };
  // This wave's operand fragments of k-step s of k-tile kt.
  auto read = [&](int kt, int s, v4i (&a)[WTM], v4i (&b)[WTN]) {
    const char* slot = lds + (kt % NS) * (F * 1024);
#pragma unroll
    for (int j = 0; j < WTN; ++j)
      b[j] = *reinterpret_cast<const v4i*>(slot + (KS * MT + s * NTB + wn * WTN + j) * 1024 + lane * 16);
#pragma unroll
    for (int i = 0; i < WTM; ++i)
      a[i] = *reinterpret_cast<const v4i*>(slot + (s * MT + wm * WTM + i) * 1024 + lane * 16);
  };

  v16i acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  // MFMAs q in [lo, hi) of one k-step, q = i * WTN + j.
  auto mma = [&](const v4i (&a)[WTM], const v4i (&b)[WTN], int lo, int hi) {
#pragma unroll
    for (int q = lo; q < hi; ++q)
      acc[q / WTN][q % WTN] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[q % WTN], a[q / WTN], acc[q / WTN][q % WTN], 0, 0, 0);
  };

  // Pipeline.  All NS slots are filled up front; k-tile kt+NS is issued into k-tile kt's slot
  // as soon as every wave has finished reading it, so NS-1 k-tiles are in flight while one is
  // multiplied.  Fragments are read from LDS one k-step ahead of their MFMAs, and the reads
  // that refill a register set are issued only after EARLY MFMAs of the other set, so they never
  // wait on MFMAs still reading the set they overwrite; sched_barrier keeps the compiler from
  // reordering the phases.  One barrier per k-tile publishes the next k-tile and frees the
  // current slot.
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (s < KT) issue(s);
  if (NS <= KT)
    wait_vmcnt<FW * (NS - 1)>();
  else
    wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  if constexpr (EPI != EPI_I32) {
#pragma unroll
    for (int u = 0; u < SCALE_PER_THREAD; ++u) {
      const int i = int(threadIdx.x) + u * NW * 64;
      if (i < NSCALE) s_scale[i] = scale_v[u];
    }
  }

  v4i a0[WTM], b0[WTN], a1[WTM], b1[WTN];
  if (KT > 0) read(0, kw, a0, b0);
  for (int kt = 0; kt < KT; ++kt) {
    const bool more = kt + 1 < KT;
#pragma unroll
    for (int j = 0; j < SW; ++j) {
      const int s = kw + j * KW;  // k-step within the k-tile
      v4i(&ca)[WTM] = (j % 2 == 0) ? a0 : a1;
      v4i(&cb)[WTN] = (j % 2 == 0) ? b0 : b1;
      v4i(&na)[WTM] = (j % 2 == 0) ? a1 : a0;
      v4i(&nb)[WTN] = (j % 2 == 0) ? b1 : b0;
      const bool live = more || s < last_steps;  // k-step inside K
      if (live) mma(ca, cb, 0, EARLY);
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < SW) {
        read(kt, s + KW, na, nb);
      } else if (more) {
        // Every read of this k-tile has completed (lgkmcnt 0) and, after the barrier, on every
        // wave: its slot takes k-tile kt+NS.  k-tile kt+1 has landed once at most the NS-2
        // k-tiles issued after it are in flight.
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        if (kt + NS - 1 < KT)
          wait_vmcnt<FW * (NS - 2)>();
        else
          wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (kt + NS < KT) issue(kt + NS);
        read(kt + 1, kw, na, nb);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (live) mma(ca, cb, EARLY, NQ);
    }
  }

  // ---- row-major epilogue through LDS: wave split-K tiles add their KW partials there, and every
  // tile stages its accumulators there, so that each store instruction writes whole row segments
  // instead of 16 or 32 bytes of 32 rows -------------------------------------------------------
  constexpr int LDR = BN + 4;  // padded row (int32) of the staged tiles
  static_assert(KW * BM * LDR * 4 <= RING, "the staged partial tiles must fit in the ring");
  static_assert((NW * 64) % (BN / 16) == 0, "whole threads per staged row");
  static_assert(EPI != EPI_GELU || BN == 64 || BN == 128, "GELU pairing in the staged epilogue");
  int32_t* red = reinterpret_cast<int32_t*>(lds);
  // Every DMA has landed (the last k-tiles waited for vmcnt 0) and, after this barrier, every
  // wave has finished reading the ring.
  __syncthreads();
  const int lrow = lane & 31, lcol = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = (wm * WTM + i) * 32 + lrow;
        const int col = (wn * WTN + j) * 32 + 8 * g + lcol;
        *reinterpret_cast<v4i*>(red + (kw * BM + row) * LDR + col) =
            v4i{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
      }
  __syncthreads();
  ksplit_epilogue<EPI, BM, BN, KW, NW, LDR>(p, red, s_scale, m0, t0);
}


// ---- direct-W kernel ----------------------------------------------------------------------------
// NWN waves side by side along N, each owning all BM rows of the block tile and WTN 32-column
// tiles.  Only A goes through LDS (two slots of KS k-steps, DMA'd one k-tile ahead, shared by all
// waves); each wave loads its own W fragments straight into registers from the packed layout --
// a fragment is 1 KiB of contiguous 16-byte lane slices, the MFMA operand as it lies in memory --
// PW k-steps ahead of their MFMAs.  LDS then carries A only, and a barrier comes once per KS
// k-steps, in a k-tile's last k-step: it publishes the next k-tile's A (DMA'd a k-tile earlier)
// and frees the current slot for the k-tile after next.
template <int BM, int NWN, int WTN, int KS, int PW, int EPI, bool A_PACKED, int MINB>
__global__ __launch_bounds__(NWN * 64, MINB) void gemm_dw_kernel(GemmParams p) {
  constexpr int NW = NWN;
  constexpr int MT = BM / 32;
  constexpr int NTB = NWN * WTN;
  constexpr int BN = NTB * 32;
  constexpr int FA = KS * MT / NW;  // A fragments each wave DMAs per k-tile
  static_assert(FA * NW == KS * MT, "each wave moves whole A fragments");
  static_assert(KS % PW == 0 && PW >= 1, "the W register ring must divide the k-tile");
  static_assert(EPI != EPI_GELU || WTN % 2 == 0, "GELU pairs need an even tile count per wave");
  static_assert(FA + (KS > PW ? KS : PW) * WTN < 64, "outstanding loads must fit the 6-bit vmcnt");
  static_assert(KS % 2 == 0, "k-steps alternate between two A register sets");
  constexpr int SLOT = KS * MT * 1024;
  constexpr int NSCALE = EPI == EPI_I32 ? 0 : BM + BN;
  constexpr int SCALE_PER_THREAD = NSCALE ? (NSCALE + NW * 64 - 1) / (NW * 64) : 1;
  __shared__ __attribute__((aligned(1024))) char lds[2 * SLOT + NSCALE * 4];
  float* const s_scale = reinterpret_cast<float*>(lds + 2 * SLOT);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT + NTB - 1) / NTB;
  const int lb = xcd_remap(blockIdx.x, ntm * ntn);
  int tm, tn;
  tile_coords(lb, ntm, ntn, p.gm, tm, tn);
  const int m0 = tm * BM;
  const int t0 = tn * NTB;
  const int KT = (p.KF + KS - 1) / KS;
  const int last_steps = p.KF - (KT - 1) * KS;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.wp, p.w_bytes);

  float scale_v[SCALE_PER_THREAD];
#pragma unroll
  for (int u = 0; u < SCALE_PER_THREAD; ++u) {
    scale_v[u] = 0.0f;
    if constexpr (EPI != EPI_I32) {
      const int i = int(threadIdx.x) + u * NW * 64;
      if (i < BM) {
        if (m0 + i < p.M) scale_v[u] = p.sx[m0 + i];
      } else if (i < BM + BN) {
        const int pc = i - BM, tt = t0 + pc / 32;
        if constexpr (EPI == EPI_GELU) {
          const int c = (tt >> 1) * 32 + pc % 32;
          if (c < p.I) scale_v[u] = p.sw[(tt & 1 ? p.I : 0) + c];
        } else {
          const int n = tt * 32 + pc % 32;
          if (n < p.N) scale_v[u] = p.sw[n];
        }
      }
    }
  }

  uint32_t offa[FA];
#pragma unroll
  for (int i = 0; i < FA; ++i) {
    const int f = i * NW + wave;
    const int s = f / MT, mt = f % MT;
    if constexpr (A_PACKED)
      offa[i] = (uint32_t(m0 / 32 + mt) * uint32_t(p.KF) + uint32_t(s)) * 1024u + uint32_t(lane) * 16u;
    else
      offa[i] = uint32_t(m0 + mt * 32 + (lane & 31)) * uint32_t(p.lda) + uint32_t(s * 32 + (lane >> 5) * 16);
  }
  constexpr uint32_t A_STEP = A_PACKED ? KS * 1024u : KS * 32u;
  // W fragment (t, g) of this wave's tile j: packed fragment t0 + wave*WTN + j, k-step g.  Tiles
  // past NT read past the buffer (zero); k-steps past KF read the next tile's data and are never
  // multiplied.
  uint32_t offw[WTN];
#pragma unroll
  for (int j = 0; j < WTN; ++j)
    offw[j] = uint32_t(t0 + wave * WTN + j) * uint32_t(p.KF) * 1024u + uint32_t(lane) * 16u;

  auto issue_a = [&](int kt) {
    char* slot = lds + (kt & 1) * SLOT;
#pragma unroll
    for (int i = 0; i < FA; ++i) dma16(ra, slot + (i * NW + wave) * 1024, offa[i] + uint32_t(kt) * A_STEP);
  };
  auto load_w = [&](int g, v4i (&w)[WTN]) {
#pragma unroll
    for (int j = 0; j < WTN; ++j) w[j] = buf_load16(rw, offw[j] + uint32_t(g) * 1024u);
  };
  auto read_a = [&](int kt, int s, v4i (&a)[MT]) {
    const char* slot = lds + (kt & 1) * SLOT;
#pragma unroll
    for (int i = 0; i < MT; ++i) a[i] = *reinterpret_cast<const v4i*>(slot + (s * MT + i) * 1024 + lane * 16);
  };

  v16i acc[MT][WTN];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  v4i wr[PW][WTN];
  issue_a(0);
  if (KT > 1) issue_a(1);
#pragma unroll
  for (int u = 0; u < PW; ++u) load_w(u, wr[u]);
  // A(0) landed once at most A(1) and the PW k-steps of W are outstanding
  if (KT > 1)
    wait_vmcnt<FA + PW * WTN>();
  else
    wait_vmcnt<PW * WTN>();
  __builtin_amdgcn_s_barrier();
  if constexpr (EPI != EPI_I32) {
#pragma unroll
    for (int u = 0; u < SCALE_PER_THREAD; ++u) {
      const int i = int(threadIdx.x) + u * NW * 64;
      if (i < NSCALE) s_scale[i] = scale_v[u];
    }
  }

  // Each step reads the next step's A fragments before its own MFMAs.  In a k-tile's last step,
  // once every read of this k-tile's slot has completed (lgkmcnt 0) and this wave's part of the
  // next k-tile's A has landed, a barrier publishes that A and frees this slot, which then takes
  // the DMA of the k-tile after next; the next k-tile's first fragments are read after it.
  v4i a0[MT], a1[MT];
  read_a(0, 0, a0);
  for (int kt = 0; kt < KT; ++kt) {
    const bool more = kt + 1 < KT;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      v4i(&ca)[MT] = (s % 2 == 0) ? a0 : a1;
      v4i(&na)[MT] = (s % 2 == 0) ? a1 : a0;
      if (s + 1 < KS) {
        read_a(kt, s + 1, na);
      } else if (more) {
        // A(kt+1) was issued before at least KS*WTN W loads (the last k-step of the previous
        // k-tile and the KS-1 before this one, or the prologue's PW and KS-1 here)
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        wait_vmcnt<KS * WTN>();
        __builtin_amdgcn_s_barrier();
        if (kt + 2 < KT) issue_a(kt + 2);
        read_a(kt + 1, 0, na);
      }
      __builtin_amdgcn_sched_barrier(0);
      const bool live = more || s < last_steps;
      if (live) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < WTN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wr[s % PW][j], ca[i], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_w(kt * KS + s + PW, wr[s % PW]);
    }
  }

  if constexpr (EPI == EPI_I32) {
    // every wave has read its last A fragments: the ring is free to stage the int32 tiles
    static_assert(2 * SLOT >= NW * 4096, "the ring holds a staging tile per wave");
    __syncthreads();
    store_i32_lines<MT, WTN>(p, acc, lds + wave * 4096, m0, t0 + wave * WTN, lane);
    return;
  }
  // s_scale is visible to every wave, and every wave has read its last A fragments: the ring is
  // free to stage the output tiles
  static_assert(2 * SLOT >= NW * 2048, "the ring holds a staging tile per wave");
  __syncthreads();
  char* const st = lds + wave * 2048;
  const int lrow = lane & 31;
  const int lcol = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const float sxm = s_scale[i * 32 + lrow];
    const float* swt = s_scale + BM + wave * WTN * 32 + lcol;
    v2u y[4];
    if constexpr (EPI == EPI_GELU) {
#pragma unroll
      for (int j = 0; j < WTN; j += 2) {
        tile_bf16<EPI>(acc[i][j], &acc[i][j + 1], sxm, swt + j * 32, y);
        store_bf16_lines<EPI>(p, y, st, m0 + i * 32, ((t0 + wave * WTN + j) >> 1) * 32, p.I, lane);
      }
    } else {
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        tile_bf16<EPI>(acc[i][j], nullptr, sxm, swt + j * 32, y);
        store_bf16_lines<EPI>(p, y, st, m0 + i * 32, (t0 + wave * WTN + j) * 32, p.N, lane);
      }
    }
  }
}

// ---- software-pipelined persistent kernel, one wave per SIMD ---------------------------------------
// Four waves in a WGM x (4/WGM) grid, each owning a (BM/WGM) x (BN*WGM/4) part of the block tile as
// 32 x 32 MFMA tiles held in the accumulator registers (256 x 256 on 2 x 2: sixteen 16-register
// accumulators per wave).
// k-tiles are 64 deep (two k-steps): the packed layouts pad K to 64, so every k-step of every
// k-tile is live and the loop has no branches.  A and W fragments go HBM -> LDS by DMA into an
// NS-slot ring.  With one wave per SIMD nothing else fills a gap in a wave's MFMA stream, so the
// LDS reads and DMA issues are placed behind the MFMAs (sched_barrier fences fix the order) and
// issue while those run.
//
// Persistent: block b multiplies the logical tiles xcd_remap(b) + i * gridDim.x, and the ring runs
// as one stream of k-tiles across them (stream index g = i * KT + kt), so the first k-tiles of a
// tile land while the previous tile's last k-tiles are multiplied and its epilogue stores go out.
// Per k-tile:
//   k-step 0: MFMAs on register set 0 (k-step 0 of g), reading k-step 1 of g into set 1 and issuing
//             the second half of the DMAs of stream k-tile g - 1 + NS;
//   k-step 1: once set 1 has landed (so this wave reads slot g no more) and this wave's DMAs of
//             g+1 have landed, one barrier; then MFMAs on set 1, reading k-step 0 of g+1 into
//             set 0 and issuing the first half of the DMAs of g + NS into the slot of g, which no
//             wave reads again.
// The DMAs are spread that way, evenly among the reads, because the path from L2 into a CU moves
// about 30 bytes per clock (measured on MI355X with every CU loading): a wave that issues its
// loads back to back fills the request queue and then stalls its MFMA stream behind it.
// DMAs past the block's last k-tile go through a buffer resource with no records: they return
// zeros and touch no memory, and every k-tile keeps the same count of loads in flight.
template <int BM, int BN, int WGM, int NS, int EPI, bool A_PACKED, int MINB>
__global__ __launch_bounds__(256, MINB) void gemm_pipe_kernel(GemmParams p) {
  constexpr int KS = 2, NW = 4, WGN = NW / WGM;
  constexpr int MT = BM / 32, NTB = BN / 32;
  constexpr int WTM = MT / WGM, WTN = NTB / WGN;
  constexpr int NQ = WTM * WTN;
  constexpr int F = KS * (MT + NTB);
  constexpr int FA = KS * MT / NW, FB = KS * NTB / NW, FW = FA + FB;
  constexpr int FH = FW / 2;             // DMAs of a k-tile issued right after the barrier that frees its slot
  constexpr int NR = WTM + WTN;          // fragment reads per k-step
  constexpr int PRE = NQ >= 4 ? 2 : 1;   // MFMAs of k-step 1 issued before its barrier
  static_assert(WGM * WGN == NW && WTM * WGM == MT && WTN * WGN == NTB, "waves tile the block");
  static_assert(FA * NW == KS * MT && FB * NW == KS * NTB, "each wave moves whole A and W fragments");
  static_assert(FW * (NS - 1) < 64, "outstanding loads must fit the 6-bit vmcnt");
  static_assert(NS >= 3, "one slot read, one landing, at least one in flight");
  static_assert(PRE < NQ, "k-step 1 has MFMAs after its barrier");
  static_assert(EPI != EPI_GELU || WTN % 2 == 0, "GELU pairs need an even tile count per wave");
  constexpr int NSCALE = EPI == EPI_I32 ? 0 : BM + BN;
  constexpr int SCALE_PER_THREAD = NSCALE ? (NSCALE + 255) / 256 : 1;
  constexpr int SLOT = F * 1024;
  constexpr int RING = NS * SLOT;
  // int32 epilogue: one 32x32 tile per wave staged here, so each store writes whole 128-byte lines
  constexpr int STAGE = EPI == EPI_I32 ? NW * 4096 : 0;
  __shared__ __attribute__((aligned(1024))) char lds[RING + NSCALE * 4 + STAGE];
  float* const s_scale = reinterpret_cast<float*>(lds + RING);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT + NTB - 1) / NTB;
  const int ntiles = ntm * ntn;
  const int G = int(gridDim.x);
  const int r0 = xcd_remap(int(blockIdx.x), G);
  const int my_tiles = r0 < ntiles ? (ntiles - 1 - r0) / G + 1 : 0;
  const int KT = p.KF / KS;  // KF is even: K is padded to 64

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.wp, p.w_bytes);
  const __amdgpu_buffer_rsrc_t ra_dead = make_rsrc(p.a, 0);
  const __amdgpu_buffer_rsrc_t rw_dead = make_rsrc(p.wp, 0);

  // First row and first 32-column tile of this block's tile i.
  auto tile_origin = [&](int i, int& m0, int& t0) {
    int tm, tn;
    tile_coords(r0 + i * G, ntm, ntn, p.gm, tm, tn);
    m0 = tm * BM;
    t0 = tn * NTB;
  };

  // Lane parts of the DMA offsets (fragment f = i * NW + wave of a k-tile: A (s, mt) =
  // (f / MT, f % MT), W (s, nt) = (f / NTB, f % NTB)); the tile and k-tile parts are uniform.
  uint32_t la[FA], lw[FB];
#pragma unroll
  for (int i = 0; i < FA; ++i) {
    const int f = i * NW + wave;
    const int s = f / MT, mt = f % MT;
    if constexpr (A_PACKED)
      la[i] = (uint32_t(mt) * uint32_t(p.KF) + uint32_t(s)) * 1024u + uint32_t(lane) * 16u;
    else
      la[i] = uint32_t(mt * 32 + (lane & 31)) * uint32_t(p.lda) + uint32_t(s * 32 + (lane >> 5) * 16);
  }
#pragma unroll
  for (int i = 0; i < FB; ++i) {
    const int f = i * NW + wave;
    const int s = f / NTB, nt = f % NTB;
    lw[i] = (uint32_t(nt) * uint32_t(p.KF) + uint32_t(s)) * 1024u + uint32_t(lane) * 16u;
  }
  constexpr uint32_t A_STEP = A_PACKED ? KS * 1024u : KS * 32u;
  constexpr uint32_t W_STEP = KS * 1024u;

  // Uniform DMA state of a stream k-tile: its A / W base offsets and resources (dead past the end).
  struct DmaBase {
    uint32_t a, w;
    __amdgpu_buffer_rsrc_t ra, rw;
  };
  // DMA cursor: stream k-tiles are DMA'd in order, each once, so the next one's tile (di), k-tile
  // in that tile (dk) and the tile's base offsets advance without divisions.
  int di = 0, dk = 0;
  uint32_t da0 = 0, dw0 = 0;
  auto cursor_tile = [&]() {
    int m0, t0;
    tile_origin(di, m0, t0);
    if constexpr (A_PACKED)
      da0 = uint32_t(m0 / 32) * uint32_t(p.KF) * 1024u;
    else
      da0 = uint32_t(m0) * uint32_t(p.lda);
    dw0 = uint32_t(t0) * uint32_t(p.KF) * 1024u;
  };
  auto next_dma = [&]() {
    DmaBase d;
    const bool live = di < my_tiles;
    d.a = da0 + uint32_t(dk) * A_STEP;
    d.w = dw0 + uint32_t(dk) * W_STEP;
    d.ra = live ? ra : ra_dead;
    d.rw = live ? rw : rw_dead;
    if (++dk == KT) {
      dk = 0;
      if (++di < my_tiles) cursor_tile();
    }
    return d;
  };
  // One DMA (fragment d < FA of A, else of W) of stream k-tile h into its ring slot.
  auto dma_one = [&](int d, int h, const DmaBase& b) {
    char* slot = lds + (h % NS) * SLOT;
    if (d < FA)
      dma16(b.ra, slot + (d * NW + wave) * 1024, la[d] + b.a);
    else
      dma16(b.rw, slot + (KS * MT + (d - FA) * NW + wave) * 1024, lw[d - FA] + b.w);
  };
  // One fragment read (r < WTN: W fragment r, else A fragment r - WTN) of k-step s of stream k-tile g.
  auto read_one = [&](int r, int g, int s, v4i (&a)[WTM], v4i (&b)[WTN]) {
    const char* slot = lds + (g % NS) * SLOT;
    if (r < WTN)
      b[r] = *reinterpret_cast<const v4i*>(slot + (KS * MT + s * NTB + wn * WTN + r) * 1024 + lane * 16);
    else
      a[r - WTN] = *reinterpret_cast<const v4i*>(slot + (s * MT + wm * WTM + r - WTN) * 1024 + lane * 16);
  };

  // This thread's per-row / per-column scales of tile i (fetched at the start of the tile's main
  // loop, parked in LDS just before its epilogue).
  float scale_v[SCALE_PER_THREAD];
  auto fetch_scales = [&](int i) {
    int m0, t0;
    tile_origin(i, m0, t0);
#pragma unroll
    for (int u = 0; u < SCALE_PER_THREAD; ++u) {
      scale_v[u] = 0.0f;
      if constexpr (EPI != EPI_I32) {
        const int e = int(threadIdx.x) + u * 256;
        if (e < BM) {
          if (m0 + e < p.M) scale_v[u] = p.sx[m0 + e];
        } else if (e < BM + BN) {
          const int pc = e - BM, tt = t0 + pc / 32;
          if constexpr (EPI == EPI_GELU) {
            const int c = (tt >> 1) * 32 + pc % 32;
            if (c < p.I) scale_v[u] = p.sw[(tt & 1 ? p.I : 0) + c];
          } else {
            const int n = tt * 32 + pc % 32;
            if (n < p.N) scale_v[u] = p.sw[n];
          }
        }
      }
    }
  };

  v16i acc[WTM][WTN];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  };
  auto mma_one = [&](int q, const v4i (&a)[WTM], const v4i (&b)[WTN]) {
    acc[q / WTN][q % WTN] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[q % WTN], a[q / WTN], acc[q / WTN][q % WTN], 0, 0, 0);
  };
  // The n ops of a k-step, nd of them DMAs placed evenly among the reads: op o is a DMA when the
  // running count (o * nd) / n steps up at o, and the op's index among its kind is that count (DMA)
  // or o minus it (read).  The ops are then dealt evenly over the k-step's MFMA slots.
  auto run_ops = [&](int slot, int nslots, int nd, auto&& read, auto&& dma) {
    const int n = NR + nd;
    const int lo = slot * n / nslots, hi = (slot + 1) * n / nslots;
#pragma unroll
    for (int o = 0; o < NR + FW; ++o) {
      if (o < lo || o >= hi || o >= n) continue;
      const int before = o * nd / n;
      if ((o + 1) * nd / n != before)
        dma(before);
      else
        read(o - before);
    }
  };

  if (my_tiles == 0) return;
  fetch_scales(0);
  cursor_tile();
  DmaBase pend;  // the stream k-tile whose second half of DMAs is still to go out
#pragma unroll
  for (int h = 0; h < NS; ++h) {
    const DmaBase b = next_dma();
#pragma unroll
    for (int d = 0; d < (h + 1 < NS ? FW : FH); ++d) dma_one(d, h, b);
    if (h + 1 == NS) pend = b;
  }
  wait_vmcnt<FW * (NS - 1) - (FW - FH)>();
  __builtin_amdgcn_s_barrier();

  v4i a0[WTM], b0[WTN], a1[WTM], b1[WTN];
#pragma unroll
  for (int r = 0; r < NR; ++r) read_one(r, 0, 0, a0, b0);
  const int lrow = lane & 31;
  const int lcol = 4 * (lane >> 5);
  int g = 0;  // stream k-tile
  for (int it = 0; it < my_tiles; ++it) {
    zero_acc();
    for (int kt = 0; kt < KT; ++kt, ++g) {
      // k-step 0: MFMAs on set 0; reads of k-step 1 of g into set 1 and the second half of the
      // DMAs of g - 1 + NS (its slot was freed at the barrier of g - 1)
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): set 0 has landed
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        mma_one(q, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        run_ops(q, NQ, FW - FH, [&](int r) { read_one(r, g, 1, a1, b1); },
                [&](int d) { dma_one(FH + d, g - 1 + NS, pend); });
        __builtin_amdgcn_sched_barrier(0);
      }
      // k-step 1: PRE MFMAs on set 1, the barrier, then the remaining MFMAs with the reads of
      // k-step 0 of g+1 (into set 0; past the block's last k-tile they are stale and never
      // multiplied) and the first half of the DMAs of g + NS.
      const DmaBase nb = next_dma();  // stream k-tile g + NS
      __builtin_amdgcn_s_waitcnt(0xc07f);  // set 1 has landed: this wave reads slot g no more
#pragma unroll
      for (int q = 0; q < PRE; ++q) {
        mma_one(q, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vmcnt<FW * (NS - 2)>();  // this wave's part of g+1 has landed
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = PRE; q < NQ; ++q) {
        mma_one(q, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        run_ops(q - PRE, NQ - PRE, FH, [&](int r) { read_one(r, g + 1, 0, a0, b0); },
                [&](int d) { dma_one(d, g + NS, nb); });
        __builtin_amdgcn_sched_barrier(0);
      }
      pend = nb;
    }

    // ---- epilogue of tile it, while the next tile's first k-tiles land in the ring ----
    int m0, t0;
    tile_origin(it, m0, t0);
    if constexpr (EPI != EPI_I32) {
      // Every wave finished the previous epilogue's reads of s_scale long ago (KT barriers since).
#pragma unroll
      for (int u = 0; u < SCALE_PER_THREAD; ++u) {
        const int e = int(threadIdx.x) + u * 256;
        if (e < NSCALE) s_scale[e] = scale_v[u];
      }
      __syncthreads();
    }
    if constexpr (EPI == EPI_I32) {
      store_i32_lines<WTM, WTN>(p, acc, lds + RING + wave * 4096, m0 + wm * WTM * 32, t0 + wn * WTN, lane);
    } else {
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const int ml = (wm * WTM + i) * 32 + lrow;
        const int m = m0 + ml;
        if (m >= p.M) continue;
        const float sxm = s_scale[ml];
        const float* swt = s_scale + BM + wn * WTN * 32 + lcol;
        if constexpr (EPI == EPI_GELU) {
#pragma unroll
          for (int j = 0; j < WTN; j += 2)
            store_tile<EPI>(p, acc[i][j], &acc[i][j + 1], m, t0 + wn * WTN + j, lcol, sxm, swt + j * 32);
        } else {
#pragma unroll
          for (int j = 0; j < WTN; ++j)
            store_tile<EPI>(p, acc[i][j], nullptr, m, t0 + wn * WTN + j, lcol, sxm, swt + j * 32);
        }
      }
    }
    // The epilogue's loads and stores are behind the ring's DMAs in the count of loads in
    // flight: drain them so the counts the main loop waits for hold again.
    wait_vmcnt<0>();
    if (it + 1 < my_tiles) fetch_scales(it + 1);
  }
}

// ---- host-side launch ----------------------------------------------------------------------

// Tile configurations, numbered 0 .. 10 as the C ABI's tile_cfg: the ones the automatic choice
// (gemm_pick_config) takes for some shape, and no others.
//
// gemm_kernel (0 - 3): block tile BM x BN, waves (WGM x WGN sub-tiles, kw waves per sub-tile taking
// alternate k-steps, their partials added in LDS), k-tile depth 32*KS, LDS ring of NS k-tiles.
struct TileCfg {
  int bm, bn, waves, ks, ns;
  int kw = 1;
};
static constexpr TileCfg kCfg[] = {
    {64, 128, 4, 4, 2},     // 0: 24 KiB slots, 48 KiB ring (three blocks per CU)
    {64, 64, 2, 4, 2},      // 1: 16 KiB slots, 32 KiB ring, 2 waves (four blocks per CU)
    {64, 128, 4, 8, 3, 2},  // 2: two 64x64 sub-tiles side by side, 2 waves each; 144 KiB ring
    {64, 64, 4, 16, 2, 4},  // 3: one 64x64 sub-tile, 4 waves; k-tile 512, 128 KiB ring
};
static constexpr int kNumCfg = int(sizeof(kCfg) / sizeof(kCfg[0]));

// gemm_dw_kernel (4 - 9): block tile BM x (NWN*WTN*32), A k-tiles of 32*KS, W register ring of PW
// k-steps.
struct DwCfg {
  int bm, nwn, wtn, ks, pw;
  int minb = 1;  // blocks per CU the registers are budgeted for
};
static constexpr DwCfg kDw[] = {
    {64, 4, 2, 8, 4, 2},   // 4: 64x256, k-tile 256, W 4 k-steps ahead, two blocks per CU
    {128, 4, 2, 8, 8},     // 5: 128x256, k-tile 256, W 8 k-steps ahead, one block per CU
    {128, 4, 2, 8, 4, 2},  // 6: 128x256, k-tile 256, W 4 k-steps ahead, two blocks per CU
    {96, 4, 2, 8, 8},      // 7: 96x256, k-tile 256, W 8 k-steps ahead, one block per CU
    {160, 4, 2, 8, 8},     // 8: 160x256, the same
    {192, 4, 2, 8, 8},     // 9: 192x256, the same
};
static constexpr int kNumDw = int(sizeof(kDw) / sizeof(kDw[0]));

// gemm_pipe_kernel (10): block tile BM x BN, waves along M (the other 4 / wgm along N), NS-slot
// ring of 64-deep k-tiles, blocks per CU the registers are budgeted for.
struct PipeCfg {
  int bm, bn, wgm, ns, minb;
};
static constexpr PipeCfg kPipe[] = {
    {256, 256, 2, 4, 1},  // 10: 128x128 per wave, 32 KiB slots, 128 KiB ring
};
static constexpr int kNumPipe = int(sizeof(kPipe) / sizeof(kPipe[0]));
static_assert(kNumCfg == 4 && kNumDw == 6 && kNumPipe == 1, "every configuration needs its case in gemm_launch");
enum { CFG_64x128 = 0, CFG_64x64 = 1, CFG_64x128_KW2 = 2, CFG_64x64_KW4 = 3, CFG_DW_64x256 = 4,
       CFG_DW_128x256_PW8 = 5, CFG_DW_128x256 = 6, CFG_DW_96x256 = 7, CFG_DW_160x256 = 8, CFG_DW_192x256 = 9,
       CFG_PIPE_256x256 = 10 };

int gemm_config_count() { return kNumCfg + kNumDw + kNumPipe; }

// Blocks per CU the tile is built for: as many rings as fit in the 160 KiB of LDS, at most four.
template <int BM, int BN, int KS, int NS>
constexpr int blocks_per_cu() {
  constexpr int ring = NS * KS * (BM / 32 + BN / 32) * 1024 + 2048;
  return 4 * ring <= 160 * 1024 ? 4 : (3 * ring <= 160 * 1024 ? 3 : (2 * ring <= 160 * 1024 ? 2 : 1));
}

template <int BM, int BN, int WGM, int WGN, int KW, int KS, int NS, bool AP>
static void launch_epi(GemmParams p, int epi, hipStream_t stream) {
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT * 32 + BN - 1) / BN;
  p.gm = min(ntm, BM >= BN ? 4 : 8);
  const dim3 grid(unsigned(ntm * ntn));
  const int threads = WGM * WGN * KW * 64;
  constexpr int B = blocks_per_cu<BM, BN, KS, NS>();
  switch (epi) {
    case EPI_I32: gemm_kernel<BM, BN, WGM, WGN, KW, KS, NS, EPI_I32, AP, B><<<grid, threads, 0, stream>>>(p); break;
    case EPI_BF16: gemm_kernel<BM, BN, WGM, WGN, KW, KS, NS, EPI_BF16, AP, B><<<grid, threads, 0, stream>>>(p); break;
    case EPI_GELU: gemm_kernel<BM, BN, WGM, WGN, KW, KS, NS, EPI_GELU, AP, B><<<grid, threads, 0, stream>>>(p); break;
    case EPI_RESID: gemm_kernel<BM, BN, WGM, WGN, KW, KS, NS, EPI_RESID, AP, B><<<grid, threads, 0, stream>>>(p); break;
  }
}

template <int CFG>
static void launch(const GemmParams& p, int epi, bool a_packed, hipStream_t stream) {
  constexpr TileCfg c = kCfg[CFG];
  // The waves / kw wave groups laid out along the longer side of the block tile: 4 as 2x2, 2 as
  // 2x1 (BM >= BN) or 1x2, 1 as 1x1.
  constexpr int WG = c.waves / c.kw;
  constexpr int WGM = WG == 1 ? 1 : WG == 2 ? (c.bm >= c.bn ? 2 : 1) : 2;
  constexpr int WGN = WG / WGM;
  static_assert(WGM * WGN == WG, "wave grid");
  if (a_packed)
    launch_epi<c.bm, c.bn, WGM, WGN, c.kw, c.ks, c.ns, true>(p, epi, stream);
  else
    launch_epi<c.bm, c.bn, WGM, WGN, c.kw, c.ks, c.ns, false>(p, epi, stream);
}

template <int BM, int NWN, int WTN, int KS, int PW, int MINB, bool AP>
static void launch_dw_epi(GemmParams p, int epi, hipStream_t stream) {
  constexpr int BN = NWN * WTN * 32;
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT * 32 + BN - 1) / BN;
  p.gm = min(ntm, BM >= BN ? 4 : 8);
  const dim3 grid{unsigned(ntm * ntn)};
  const int threads = NWN * 64;
  switch (epi) {
    case EPI_I32: gemm_dw_kernel<BM, NWN, WTN, KS, PW, EPI_I32, AP, MINB><<<grid, threads, 0, stream>>>(p); break;
    case EPI_BF16: gemm_dw_kernel<BM, NWN, WTN, KS, PW, EPI_BF16, AP, MINB><<<grid, threads, 0, stream>>>(p); break;
    case EPI_GELU: gemm_dw_kernel<BM, NWN, WTN, KS, PW, EPI_GELU, AP, MINB><<<grid, threads, 0, stream>>>(p); break;
    case EPI_RESID: gemm_dw_kernel<BM, NWN, WTN, KS, PW, EPI_RESID, AP, MINB><<<grid, threads, 0, stream>>>(p); break;
  }
}

template <int D>
static void launch_dw(const GemmParams& p, int epi, bool a_packed, hipStream_t stream) {
  constexpr DwCfg c = kDw[D];
  if (a_packed)
    launch_dw_epi<c.bm, c.nwn, c.wtn, c.ks, c.pw, c.minb, true>(p, epi, stream);
  else
    launch_dw_epi<c.bm, c.nwn, c.wtn, c.ks, c.pw, c.minb, false>(p, epi, stream);
}

// Compute units of the current device (256 on MI355X), read once.
static int cu_count() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

// Blocks of the persistent kernels: one per CU per block the registers allow, at most one per tile.
static int persistent_blocks(int tiles, int per_cu) { return min(tiles, cu_count() * per_cu); }

template <int BM, int BN, int WGM, int NS, int MINB, bool AP>
static void launch_pipe_epi(GemmParams p, int epi, hipStream_t stream) {
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT * 32 + BN - 1) / BN;
  p.gm = min(ntm, BM >= BN ? 4 : 8);
  const dim3 grid{unsigned(persistent_blocks(ntm * ntn, MINB))};
  switch (epi) {
    case EPI_I32: gemm_pipe_kernel<BM, BN, WGM, NS, EPI_I32, AP, MINB><<<grid, 256, 0, stream>>>(p); break;
    case EPI_BF16: gemm_pipe_kernel<BM, BN, WGM, NS, EPI_BF16, AP, MINB><<<grid, 256, 0, stream>>>(p); break;
    case EPI_GELU: gemm_pipe_kernel<BM, BN, WGM, NS, EPI_GELU, AP, MINB><<<grid, 256, 0, stream>>>(p); break;
    case EPI_RESID: gemm_pipe_kernel<BM, BN, WGM, NS, EPI_RESID, AP, MINB><<<grid, 256, 0, stream>>>(p); break;
  }
}

template <int D>
static void launch_pipe(const GemmParams& p, int epi, bool a_packed, hipStream_t stream) {
  constexpr PipeCfg c = kPipe[D];
  if (a_packed)
    launch_pipe_epi<c.bm, c.bn, c.wgm, c.ns, c.minb, true>(p, epi, stream);
  else
    launch_pipe_epi<c.bm, c.bn, c.wgm, c.ns, c.minb, false>(p, epi, stream);
}

// The pipelined kernel's 256x256 tiles leave a nearly empty last round on the CUs.
static bool pipe_tail_is_short(int M, int NP) {
  const int cus = cu_count();
  const int tail = ((M + 255) / 256) * ((NP + 255) / 256) % cus;
  return tail > 0 && 4 * tail <= cus;
}

// Tile choice.  Every rule was set by timing the configurations on MI355X (the measured times are
// tabulated with the design notes); the reasons, briefly:
//  * One 512-row micro-batch (M <= 1024): the GEMMs are bound by how fast each CU streams its
//    operands, so small tiles spread over many CUs.  Narrow long-K GEMMs (the output and down
//    projections) have only ~192 64x64 tiles, one per CU, so four waves split each tile's k-steps
//    with 512-deep k-tiles (3).  The gate/up GEMM with its GELU epilogue runs on the direct-W 64x256
//    tile, two blocks per CU (4).  Narrow short-K GEMMs take 64x64 (1).  Wide ones take 64x128 with
//    two waves per sub-tile while those tiles fit one round on the CUs (2), then one round of
//    direct-W 64x256 tiles (4), else 64x128 three blocks per CU (0).
//  * Past one micro-batch: the GELU epilogue on the direct-W 128x256 tile, two blocks per CU (6).
//    GEMMs up to N = 4096 stream (BM + BN) * K bytes per tile at the per-CU L2 delivery rate, so
//    one round of the smallest direct-W BMx256 tile that fits the CUs (BM = 96, 128, 160, 192:
//    7, 5, 8, 9) wins where its bytes per CU undercut the 64x128 three-per-CU tiles'.  The wide
//    int32 GEMMs (N >= 8192) take the software-pipelined persistent 256x256 kernel (10), which
//    reads each weight half as often, unless its last round would be nearly empty; everything
//    else the 128x256 two-per-CU tile (6), or 64x128 (0) where 6's tiles are fewer than the CUs or
//    leave a nearly empty last round.
int gemm_pick_config(int M, int NP, int K, int epi) {
  const int cus = cu_count();
  if (M <= 1024) {
    if (K >= 2048 && NP <= 4096) return CFG_64x64_KW4;
    if (epi == EPI_GELU) return CFG_DW_64x256;
    if (NP <= 2048) return CFG_64x64;
    const int mt = (M + 63) / 64;
    if (mt * ((NP + 127) / 128) <= cus) return CFG_64x128_KW2;
    return mt * ((NP + 255) / 256) <= cus ? CFG_DW_64x256 : CFG_64x128;
  }
  if (epi == EPI_GELU) return CFG_DW_128x256;
  auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((NP + bn - 1) / bn); };
  if (K >= 1024 && NP <= 4096) {
    // one round of direct-W BMx256 tiles, smallest BM first, where the busiest CU moves fewer bytes
    // than on the 64x128 three-per-CU tiles
    const int cost0 = (tiles(64, 128) + cus - 1) / cus * (64 + 128);
    constexpr int kBm[4] = {96, 128, 160, 192};
    constexpr int kCfgOf[4] = {CFG_DW_96x256, CFG_DW_128x256_PW8, CFG_DW_160x256, CFG_DW_192x256};
    for (int i = 0; i < 4; ++i)
      if (tiles(kBm[i], 256) <= cus) {
        if (kBm[i] + 256 < cost0) return kCfgOf[i];
        break;
      }
  }
  const bool pipe = NP >= 8192 && epi == EPI_I32 && !pipe_tail_is_short(M, NP);
  if (M > 8192) return pipe ? CFG_PIPE_256x256 : CFG_DW_128x256;
  if (K >= 4096 && NP <= 2048) return CFG_DW_128x256;  // long-K narrow past one round of 128x256
  if (NP >= 8192) return pipe ? CFG_PIPE_256x256 : CFG_DW_128x256;
  const int t6 = tiles(128, 256), tail = t6 % cus;
  return t6 >= cus && !(tail > 0 && 4 * tail <= cus) ? CFG_DW_128x256 : CFG_64x128;
}

int gemm_launch(const GemmParams& p, int epi, int cfg, bool a_packed, hipStream_t stream) {
  if (cfg < 0) cfg = gemm_pick_config(p.M, p.NT * 32, p.KF * 32, epi);
  switch (cfg) {
    case 0: launch<0>(p, epi, a_packed, stream); break;
    case 1: launch<1>(p, epi, a_packed, stream); break;
    case 2: launch<2>(p, epi, a_packed, stream); break;
    case 3: launch<3>(p, epi, a_packed, stream); break;
    case 4: launch_dw<0>(p, epi, a_packed, stream); break;
    case 5: launch_dw<1>(p, epi, a_packed, stream); break;
    case 6: launch_dw<2>(p, epi, a_packed, stream); break;
    case 7: launch_dw<3>(p, epi, a_packed, stream); break;
    case 8: launch_dw<4>(p, epi, a_packed, stream); break;
    case 9: launch_dw<5>(p, epi, a_packed, stream); break;
    case 10: launch_pipe<0>(p, epi, a_packed, stream); break;
    default: return fail(W8A8_EINVAL, "gemm: unknown tile config %d", cfg);
  }
  return check_launch("gemm");
}

}  // namespace w8a8
