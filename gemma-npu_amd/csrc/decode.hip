// The decode step's tail: the logit softcap, the greedy argmax and the step's bookkeeping, in two
// launches (the reference's decode loop, gemma_npu.py:292-295: logits -> argmax -> next token).
//
// head_tail_candidates_kernel: each workgroup softcaps 2048 logits as the model's bf16 ops do
// (HF Gemma 4's final_logit_softcapping on bf16 logits: t = bf16(y * (1 / cap)) -- torch divides a
// floating tensor by a scalar as a product with its reciprocal -- u = bf16(tanh(t)), v = bf16(u * cap)),
// writes them as fp32 and parks its maximum and the first index holding it.  head_tail_pick_kernel
// (one workgroup) takes the first index of the overall maximum (NaN counts as the largest, as
// torch.argmax), writes it as the next token and into the emitted list, and advances the position.
#include "w8a8_common.h"

namespace w8a8 {

constexpr int TAIL_PER_BLOCK = 2048;  // logits per candidates workgroup (256 threads x 8)

struct Cand {
  float v;
  int i;
};

// a replaces b as the maximum: larger, or NaN over a number, or equal with a smaller index
__device__ __forceinline__ bool cand_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return an;
  if (an) return ai < bi;
  return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ Cand block_best(Cand c, Cand* sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(c.v, o, 64);
    const int oi = __shfl_xor(c.i, o, 64);
    if (cand_better(ov, oi, c.v, c.i)) c = Cand{ov, oi};
  }
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[wave] = c;
  __syncthreads();
  Cand best = sh[0];
  for (int w = 1; w < nw; ++w)
    if (cand_better(sh[w].v, sh[w].i, best.v, best.i)) best = sh[w];
  return best;
}

__global__ __launch_bounds__(256) void head_tail_candidates_kernel(const uint16_t* __restrict__ y, int V, float cap,
                                                                   float* __restrict__ logits, Cand* __restrict__ cand) {
  __shared__ Cand sh[4];
  const int base = blockIdx.x * TAIL_PER_BLOCK + threadIdx.x * 8;
  const float inv = cap > 0.0f ? 1.0f / cap : 0.0f;
  Cand c{-__builtin_inff(), 0x7fffffff};
  float v[8];
  if (base + 8 <= V) {
    unpack8(*reinterpret_cast<const v4u*>(y + base), v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = base + e < V ? bf16_to_f32(y[base + e]) : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = v[e];
    if (cap > 0.0f) x = round_bf16(round_bf16(tanhf(round_bf16(x * inv))) * cap);
    v[e] = x;
    if (base + e < V && cand_better(x, base + e, c.v, c.i)) c = Cand{x, base + e};
  }
  if (base + 8 <= V) {
    *reinterpret_cast<v4f*>(logits + base) = v4f{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<v4f*>(logits + base + 4) = v4f{v[4], v[5], v[6], v[7]};
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (base + e < V) logits[base + e] = v[e];
  }
  const Cand best = block_best(c, sh);
  if (threadIdx.x == 0) cand[blockIdx.x] = best;
}

__global__ __launch_bounds__(256) void head_tail_pick_kernel(const Cand* __restrict__ cand, int ncand,
                                                             int32_t* pos, int64_t* pos64, int64_t* tok,
                                                             int64_t* emitted, int64_t* n_emitted, int64_t max_emitted) {
  __shared__ Cand sh[4];
  Cand c{-__builtin_inff(), 0x7fffffff};
  for (int j = threadIdx.x; j < ncand; j += 256)
    if (cand_better(cand[j].v, cand[j].i, c.v, c.i)) c = cand[j];
  const Cand best = block_best(c, sh);
  if (threadIdx.x == 0) {
    const int64_t n = *n_emitted;
    *tok = best.i;
    if (n >= 0 && n < max_emitted) emitted[n] = best.i;
    *n_emitted = n + 1;
    *pos += 1;
    *pos64 += 1;
  }
}

}  // namespace w8a8

using namespace w8a8;

extern "C" int64_t w8a8_decode_tail_workspace_bytes(int64_t V) {
  if (V < 1 || V > INT32_MAX - TAIL_PER_BLOCK) return -1;
  return (V + TAIL_PER_BLOCK - 1) / TAIL_PER_BLOCK * int64_t(sizeof(Cand));
}

extern "C" int w8a8_decode_tail(const uint16_t* y, int64_t V, float cap, float* logits, int32_t* pos, int64_t* pos64,
                                int64_t* tok, int64_t* emitted, int64_t* n_emitted, int64_t max_emitted,
                                void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  const char* what = "decode_tail";
  if (!y || !logits || !pos || !pos64 || !tok || !emitted || !n_emitted || !workspace)
    return fail(W8A8_EINVAL, "%s: null pointer", what);
  const int64_t need = w8a8_decode_tail_workspace_bytes(V);
  if (need < 0) return fail(W8A8_EINVAL, "%s: V=%lld", what, (long long)V);
  if (workspace_bytes < need)
    return fail(W8A8_EINVAL, "%s: workspace of %lld bytes, %lld needed", what, (long long)workspace_bytes,
                (long long)need);
  if (!(cap >= 0.0f) || cap == __builtin_inff()) return fail(W8A8_EINVAL, "%s: cap must be >= 0 (0: none)", what);
  if (max_emitted < 0) return fail(W8A8_EINVAL, "%s: max_emitted < 0", what);
  if ((uintptr_t)y % 16 || (uintptr_t)logits % 16 || (uintptr_t)workspace % 8 || (uintptr_t)pos % 4 ||
      (uintptr_t)pos64 % 8 || (uintptr_t)tok % 8 || (uintptr_t)emitted % 8 || (uintptr_t)n_emitted % 8)
    return fail(W8A8_EALIGN, "%s: y and logits 16-byte aligned, the counters naturally aligned", what);
  const int ncand = int(need / int64_t(sizeof(Cand)));
  Cand* cand = static_cast<Cand*>(workspace);
  head_tail_candidates_kernel<<<unsigned(ncand), 256, 0, stream>>>(y, int(V), cap, logits, cand);
  head_tail_pick_kernel<<<1, 256, 0, stream>>>(cand, ncand, pos, pos64, tok, emitted, n_emitted, max_emitted);
  return check_launch("decode_tail");
}
