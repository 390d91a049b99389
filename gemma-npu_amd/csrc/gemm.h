// GEMM launch parameters shared by gemm.hip and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w8a8 {

enum { EPI_I32 = 0, EPI_BF16 = 1, EPI_GELU = 2, EPI_RESID = 3 };

struct GemmParams {
  const int8_t* a;      // activations: [M, K] row-major (leading dimension lda) or packed
                        // 32-row MFMA fragments (pack_act / quant_rows_packed)
  const int8_t* wp;     // packed weight fragments (pack_weight)
  uint32_t a_bytes;     // (M-1)*lda + K: loads at or past this offset read zero
  uint32_t w_bytes;     // NT * KF * 1024
  int64_t lda;
  int M, N, KF, NT;     // N: logical output columns (EPI_GELU: 2*I); KF = 32-wide k fragments per
                        // 32-channel tile (K padded to 64); NT = packed 32-channel tiles
  int I;                // EPI_GELU: width of the gate (and up) half
  int vec_store;        // output rows allow 4-wide vector stores (alignment checked on the host)
  int res_vec;          // residual rows allow 4-wide (8-byte) vector loads
  int gm;               // row tiles per group in the block -> tile order (set by the launcher)
  int32_t* c; int64_t ldc;          // EPI_I32
  const float* sx; const float* sw; // per-row / per-channel scales
  uint16_t* out; int64_t ldo;       // bf16 epilogues
  const uint16_t* res; int64_t ldr; // EPI_RESID
};

int gemm_config_count();
// Automatic tile configuration for [M, NP, K] with epilogue epi.
int gemm_pick_config(int M, int NP, int K, int epi);
int gemm_launch(const GemmParams& p, int epi, int cfg, bool a_packed, hipStream_t stream);

}  // namespace w8a8
