// int8 x int8 -> int32 GEMM on CDNA4 MFMA (v_mfma_i32_16x16x64_i8), with fused epilogues.
//
// Replaces the Triton kernel matmul_i8_k (npu_kernels.py:40-56): C[M,N] = A[M,K] @ W, int32
// accumulate, here with W held resident in the packed fragment layout written by
// pack_weight (quant.hip) and with the reference's neighbouring element-wise work fused into
// the store:
//   EPI_I32       C int32                                     (npu_kernels.py:56)
//   EPI_BF16      bf16((acc * sx[m]) * sw[n])                 (_deq, pipeline.py:55-57)
//   EPI_GELU      bf16(gelu_tanh(gate) * up) on the dequantised bf16 gate/up pair
//                                                             (k_gelu, pipeline.py:102-107)
//   EPI_RESID     bf16(res + bf16(dequant))                   (plain residual add)
//
// Block tile BM x BN, four waves in a 2 x 2 grid, each wave owns (BM/2) x (BN/2) of C as
// 16 x 16 MFMA tiles.  Per pipeline stage the block stages S k-tiles of 64 (A: BM/16 and
// W: BN/16 fragments of 1 KiB each) in LDS, double-buffered: the global loads of stage s+1
// are in flight while stage s is multiplied.  Both operands sit in LDS in MFMA fragment
// order (lane l's 16 bytes at 16*l), so every ds_read_b128 is a contiguous 1 KiB and
// conflict-free.  The MFMA is issued as W-fragment x A-fragment, so a lane's accumulator
// holds four consecutive output columns of one row and stores go out as 16-byte vectors.
#include "w8a8_common.h"
#include "gemm.h"

namespace w8a8 {

__device__ __forceinline__ float gelu_tanh_f32(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), the approximate="tanh" form.
  const float kBeta = 0.7978845608028654f;
  const float kKappa = 0.044715f;
  const float inner = kBeta * (x + kKappa * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

template <int BM, int BN, int S, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmParams p) {
  constexpr int MT = BM / 16;       // A fragments per k-tile
  constexpr int NTB = BN / 16;      // W fragments per k-tile
  constexpr int FA = MT * S;        // A fragments per stage
  constexpr int FB = NTB * S;       // W fragments per stage
  constexpr int F = FA + FB;
  static_assert(FA % 4 == 0 && FB % 4 == 0, "fragments must split evenly over four waves");
  constexpr int FPW = F / 4;        // fragments each wave moves per stage
  constexpr int WTM = BM / 32;      // m-tiles per wave
  constexpr int WTN = BN / 32;      // n-tiles per wave
  static_assert(EPI != EPI_GELU || (WTN % 2 == 0), "GELU pairs need an even n-tile count per wave");

  __shared__ __attribute__((aligned(1024))) char lds[2][F * 1024];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: M fastest, so blocks resident together share the same weight columns.
  const int ntm = (p.M + BM - 1) / BM;
  const int tm = blockIdx.x % ntm;
  const int tn = blockIdx.x / ntm;
  const int m0 = tm * BM;
  const int t0 = tn * NTB;  // first packed n-tile of this block

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.wp, p.w_bytes);

  // Per-lane byte offsets of this lane's 16 bytes in each fragment it loads (k-tile 0).
  uint32_t off[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = i * 4 + wave;
    if (i * 4 < FA) {  // A fragment (uniform per i since FA % 4 == 0)
      const int s = f / MT, mt = f % MT;
      const int row = m0 + mt * 16 + (lane & 15);
      off[i] = uint32_t(row) * uint32_t(p.lda) + uint32_t(s * 64 + (lane >> 4) * 16);
    } else {
      const int g = f - FA;
      const int s = g / NTB, nt = g % NTB;
      off[i] = (uint32_t(t0 + nt) * uint32_t(p.KT) + uint32_t(s)) * 1024u + uint32_t(lane) * 16u;
    }
  }
  // Rows past M (and k past K on the last row) lie at or past p.a_bytes = (M-1)*lda + K,
  // so the buffer load returns zeros for them.

  v4i acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int nst = (p.KT + S - 1) / S;
  v4i pf[FPW];

  auto load_stage = [&](int st) {
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      const int f = i * 4 + wave;
      int s;
      if (i * 4 < FA) s = f / MT; else s = (f - FA) / NTB;
      const int kt = st * S + s;
      if (kt < p.KT) {
        if (i * 4 < FA)
          pf[i] = buf_load16(ra, off[i] + uint32_t(st * S * 64));
        else
          pf[i] = buf_load16(rw, off[i] + uint32_t(st * S) * 1024u);
      } else {
        pf[i] = v4i{0, 0, 0, 0};
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      const int f = i * 4 + wave;
      *reinterpret_cast<v4i*>(&lds[buf][f * 1024 + lane * 16]) = pf[i];
    }
  };

  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    if (st + 1 < nst) load_stage(st + 1);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      v4i a[WTM], b[WTN];
#pragma unroll
      for (int i = 0; i < WTM; ++i)
        a[i] = *reinterpret_cast<const v4i*>(&lds[cur][(s * MT + wm * WTM + i) * 1024 + lane * 16]);
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        b[j] = *reinterpret_cast<const v4i*>(&lds[cur][(FA + s * NTB + wn * WTN + j) * 1024 + lane * 16]);
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[j], a[i], acc[i][j], 0, 0, 0);
    }
    if (st + 1 < nst) store_stage(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue ---------------------------------------------------------------------------
  // acc[i][j] lane l: row m = m0 + (wm*WTM+i)*16 + l%16, packed columns
  // pc = (t0 + wn*WTN + j)*16 + 4*(l/16) + r, r = 0..3.
  const int lrow = lane & 15;
  const int lcol = 4 * (lane >> 4);
#pragma unroll
  for (int i = 0; i < WTM; ++i) {
    const int m = m0 + (wm * WTM + i) * 16 + lrow;
    if (m >= p.M) continue;
    if constexpr (EPI == EPI_I32) {
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int n = (t0 + wn * WTN + j) * 16 + lcol;
        int32_t* dst = p.c + int64_t(m) * p.ldc + n;
        if (p.vec_store && n + 3 < p.N) {
          *reinterpret_cast<v4i*>(dst) = acc[i][j];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < p.N) dst[r] = acc[i][j][r];
        }
      }
    } else if constexpr (EPI == EPI_BF16 || EPI == EPI_RESID) {
      const float sxm = p.sx[m];
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int n = (t0 + wn * WTN + j) * 16 + lcol;
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float swn = (n + r < p.N) ? p.sw[n + r] : 0.0f;
          y[r] = bf16_to_f32(f32_to_bf16((float(acc[i][j][r]) * sxm) * swn));
        }
        if constexpr (EPI == EPI_RESID) {
          const uint16_t* rs = p.res + int64_t(m) * p.ldr + n;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < p.N) y[r] = y[r] + bf16_to_f32(rs[r]);
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
      const float sxm = p.sx[m];
#pragma unroll
      for (int j = 0; j < WTN; j += 2) {
        const int t = t0 + wn * WTN + j;   // even: gate tile u = t/2; t+1 is the matching up tile
        const int g = (t >> 1) * 16 + lcol; // logical gate column
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = g + r < p.I;
          const float swg = ok ? p.sw[g + r] : 0.0f;
          const float swu = ok ? p.sw[p.I + g + r] : 0.0f;
          const float gate = bf16_to_f32(f32_to_bf16((float(acc[i][j][r]) * sxm) * swg));
          const float up = bf16_to_f32(f32_to_bf16((float(acc[i][j + 1][r]) * sxm) * swu));
          const float ge = bf16_to_f32(f32_to_bf16(gelu_tanh_f32(gate)));
          o[r] = ge * up;
        }
        uint16_t* dst = p.out + int64_t(m) * p.ldo + g;
        if (p.vec_store && g + 3 < p.I) {
          *reinterpret_cast<v2u*>(dst) = v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (g + r < p.I) dst[r] = f32_to_bf16(o[r]);
        }
      }
    }
  }
}

// ---- host-side launch ----------------------------------------------------------------------

template <int BM, int BN, int S>
static void launch_cfg(const GemmParams& p, int epi, hipStream_t stream) {
  const int np = p.NT * 16;  // packed columns
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (np + BN - 1) / BN;
  dim3 grid(unsigned(ntm * ntn));
  switch (epi) {
    case EPI_I32: gemm_kernel<BM, BN, S, EPI_I32><<<grid, 256, 0, stream>>>(p); break;
    case EPI_BF16: gemm_kernel<BM, BN, S, EPI_BF16><<<grid, 256, 0, stream>>>(p); break;
    case EPI_GELU: gemm_kernel<BM, BN, S, EPI_GELU><<<grid, 256, 0, stream>>>(p); break;
    case EPI_RESID: gemm_kernel<BM, BN, S, EPI_RESID><<<grid, 256, 0, stream>>>(p); break;
  }
}

int gemm_config_count() { return 3; }

// Picks a tile shape: large tiles when they still fill the 256 CUs, smaller ones otherwise.
int gemm_pick_config(int M, int NP, int K) {
  (void)K;
  const long t256 = long((M + 255) / 256) * ((NP + 255) / 256);
  const long t128x256 = long((M + 127) / 128) * ((NP + 255) / 256);
  if (t256 >= 256) return 2;
  if (t128x256 >= 256) return 1;
  return 0;
}

int gemm_launch(const GemmParams& p, int epi, int cfg, hipStream_t stream) {
  if (cfg < 0) cfg = gemm_pick_config(p.M, p.NT * 16, p.KT * 64);
  switch (cfg) {
    case 0: launch_cfg<128, 128, 2>(p, epi, stream); break;
    case 1: launch_cfg<128, 256, 2>(p, epi, stream); break;
    case 2: launch_cfg<256, 256, 1>(p, epi, stream); break;
    default: return fail(W8A8_EINVAL, "gemm: unknown tile config %d", cfg);
  }
  return check_launch("gemm");
}

}  // namespace w8a8
