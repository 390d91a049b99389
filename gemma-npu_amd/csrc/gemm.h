// GEMM launch parameters shared by gemm.hip and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w8a8 {

enum { EPI_I32 = 0, EPI_BF16 = 1, EPI_GELU = 2, EPI_RESID = 3 };

struct GemmParams {
  const int8_t* a;      // activations [M, K] row-major, leading dimension lda (bytes)
  const int8_t* wp;     // packed weight fragments (pack_weight)
  uint32_t a_bytes;     // (M-1)*lda + K: loads at or past this offset read zero
  uint32_t w_bytes;     // NT * KT * 1024
  int64_t lda;
  int M, N, KT, NT;     // N: logical output columns (EPI_GELU: 2*I); KT = ceil(K/64); NT packed n-tiles
  int I;                // EPI_GELU: width of the gate (and up) half
  int vec_store;        // output rows allow 4-wide vector stores (alignment checked on the host)
  int32_t* c; int64_t ldc;          // EPI_I32
  const float* sx; const float* sw; // per-row / per-channel scales
  uint16_t* out; int64_t ldo;       // bf16 epilogues
  const uint16_t* res; int64_t ldr; // EPI_RESID
};

int gemm_config_count();
int gemm_pick_config(int M, int NP, int K);
int gemm_launch(const GemmParams& p, int epi, int cfg, hipStream_t stream);

}  // namespace w8a8
