// Prefill attention on the bf16 MFMA: causal, optionally sliding-window, grouped-query.
//
//   o[h, i, :] = sum_j softmax_j(scale * q[h, i] . k[g, j]) v[g, j],   g = h / (H / KV),
//
// over the keys j the query at position p = q_start + i may see: j <= p and, with a window W > 0,
// p - j < W.  This is what the reference's CPU prefill computes for Gemma's two layer kinds:
// full_attention (pipeline.py:140-155: causal sdpa over the micro-batch's own keys, merged by
// logsumexp with a non-causal pass over the earlier ones) and sliding_attention
// (pipeline.py:158-180, local_attn.py:91-107: 128-query blocks against the W + 128 keys their
// window reaches, masked k >= 0, k <= q, q - k < W).  One pass over the visible keys with an
// online softmax gives the same function without the two-part merge.
//
// Work split.  A workgroup of 8 waves owns 128 query rows of one KV group: with G = H / KV heads
// per group the rows are (position, head) pairs, G heads x 128/G consecutive positions, so the
// group's G heads share every K / V block the workgroup loads and the 128/G positions waste few
// masked keys.  Each wave owns 16 rows and walks the keys in blocks of BN:
//
//   S^T = K Q^T   (v_mfma_f32_16x16x32_bf16, K from LDS as the A operand, Q held in registers as
//                  the B operand), so a lane's accumulator column is one query and the softmax
//                  statistics are lane-local but for two exchanges between the four lane groups;
//   P^T = exp2(S^T * scale * log2 e - ms), rounded to bf16, where the reference ms trails the
//                  running maximum of S^T * scale * log2 e by at most 8 (it moves only when a
//                  block exceeds it by more than that);
//   O^T += V^T P^T  (V^T from LDS as the A operand, P^T straight from the S^T accumulators as the
//                  B operand), so O's rescaling when ms moves is lane-local too.
//
// For P^T to be usable in place, the rows of each pair of 16-key S^T tiles hold their 32 keys in
// the order that makes register i of lane group qq hold keys 8 qq + {i, 4 + i}: exactly the
// k-slot order of the next MFMA's B operand, whose V^T operand is then 8 consecutive keys, one
// ds_read_b128.
//
// Data movement.  K blocks go from HBM (mostly L2: every workgroup of a group reads the same
// keys) straight into a 2-slot LDS ring with buffer_load ... lds, one block ahead; 16-byte chunks
// of a key row are XOR-swizzled by the row so that the 16 rows one ds_read_b128 touches hit
// distinct banks.  V blocks are loaded into registers one block ahead and written transposed
// (V^T [D][BN + 8], 8-byte stores of 4 keys) into a 2-slot ring.  Loads past the end of K / V
// read zero and are masked.  One barrier per block.
#include <algorithm>
#include <map>
#include <mutex>
#include <queue>
#include <tuple>
#include <type_traits>
#include <vector>

#include "w8a8_common.h"

namespace w8a8 {

typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));

// v combined over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the same row of an MFMA tile in the four
// 16-lane groups) by the gfx950 lane swaps, in VALU instead of two ds_bpermute round trips through
// LDS: v_permlane16_swap exchanges 16-lane groups 0 <-> 1 and 2 <-> 3, v_permlane32_swap the two
// halves, and of the two results one holds the lane's own value and the other its partner's.  The
// pairs are those of a xor-16 then xor-32 butterfly and both combines are commutative, so the result
// is bit-identical to that butterfly on every lane.
__device__ __forceinline__ float lanes4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float lanes4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

constexpr int ATTN_NW = 8;        // waves per workgroup, 16 query rows each
constexpr int ATTN_MAX_SEG = 16;     // segments of the causal work list (= most parts of one tile)
constexpr int ATTN_FWD2_NW = 8;      // waves of attn_fwd2_kernel (4, one per SIMD, measured slower)
constexpr int ATTN_MAX_ORDER = 1536;  // items of a launch-order table (kernel arguments < 4 KiB)

struct AttnParams {
  const uint16_t* q; int64_t qhs, qrs;  // bf16 [H, Tq, D] (element strides, last dim contiguous)
  const uint16_t* k; int64_t khs, krs;  // bf16 [KV, Tk, D]
  const uint16_t* v; int64_t vhs, vrs;  // bf16 [KV, Tk, D]
  uint16_t* o; int64_t ohs, ors;        // bf16 [H, Tq, D]
  float* lse;                           // fp32 [H, Tq] natural-log logsumexp of the scaled scores, or null
  uint32_t k_bytes, v_bytes;            // extent of one KV group's K / V rows, bytes
  int H, KV, G, PB, Tq, Tk, q_start, window;
  int ntiles;                           // ceil(Tq / PB) query tiles per KV group
  // Work items of a KV group, in launch order (causal calls): the tiles from the longest down;
  // segment s holds tiles seg_tile[s], seg_tile[s] - 1, .. , each computed by seg_k[s] workgroups
  // over consecutive ranges of its key blocks (the last part to finish merges them), starting at
  // item seg_item[s].  Split tiles come first: they are the group's nsplit_tiles longest tiles and
  // its first nsplit_items items.  Sliding windows: one item per tile, nseg = 1.
  int per_group, nseg, nsplit_tiles, nsplit_items;
  int seg_tile[ATTN_MAX_SEG], seg_k[ATTN_MAX_SEG], seg_item[ATTN_MAX_SEG + 1];
  float* part;                          // [KV][nsplit_items] parked partial tiles, slot-major
  int* counters;                        // [KV][nsplit_tiles] arrival counts, zero between calls
  float scale, c;                       // c = scale * log2(e)
  // 0: the last part of a split tile to arrive merges the parts; 1: the parts are only parked and
  // attn_merge_kernel, launched next on the stream, merges every split tile.
  int merge_mode;
  // Quantised output (k_attn_out fused, one KV group): instead of o, the per-token int8 rows of the
  // [Tq, H*D] output in the packed activation layout (qKF fragments per row, rows zero up to qMp) and
  // their scales.  Null: o is written.
  int8_t* qpk; float* qsx; int qKF, qMp;
  // Launch order of the items: workgroup j * KV + g runs item order[j] of group g (item j when
  // `ordered` is 0).  Last, after every pointer and scalar.
  int ordered;
  uint16_t order[ATTN_MAX_ORDER];
};
static_assert(sizeof(AttnParams) <= 4096, "kernel arguments");

template <int N>
__device__ __forceinline__ void attn_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ void attn_dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Key `key` is visible to the query at `pos`: key <= pos, pos - key < the window (wlim = window, or
// 2^31 for no window) and key < Tk -- one unsigned compare per bound, combined bitwise, so the mask
// compiles to compares and selects.  A short-circuit chain (key <= pos && ... && (win == 0 || ...))
// was compiled here to divergent branches, and in one register assignment of attn_fwd_kernel the
// -inf store of a masked key was hoisted above the branch that then reused its register, leaving
// keys outside the window unmasked.
__device__ __forceinline__ bool attn_key_visible(int key, int pos, int Tk, uint32_t wlim) {
  return (uint32_t(pos - key) < wlim) & (key < Tk);
}
__device__ __forceinline__ uint32_t attn_window_limit(int window) {
  return window > 0 ? uint32_t(window) : 0x80000000u;
}
// s where `vis`, else -inf, as a select of the bit patterns
__device__ __forceinline__ float attn_mask(float s, bool vis) {
  return __uint_as_float(vis ? __float_as_uint(s) : 0xff800000u);
}

__device__ __forceinline__ int attn_xcd_remap(int b, int nblocks) {
  const int full = nblocks & ~7;
  if (b >= full) return b;
  const int per = full >> 3;
  return (b & 7) * per + (b >> 3);
}


// k_attn_out (pipeline.py:88-92) on a tile's normalised bf16 output rows staged in LDS (row r =
// head r % G of position r / G, orow bytes apart): token t = i0 + r / G is the row [head 0 | head 1 |
// ...] of G * D values, quantised per token as _quant does and written to the packed activation
// layout with its scale.  4G consecutive threads (one wave or half of one) take a token: the absmax
// of their 16-element chunks, xor shuffles over those lanes, then the codes, 16 bytes per store.  The
// workgroup of the last tile also zero-fills the packed rows from Tq up to the padded row count.
template <int D, int NT>
__device__ __forceinline__ void attn_quant_tokens(const AttnParams& p, const char* st, int orow, int i0, int tile,
                                                  int tid) {
  const int G = p.G, TPT = NT / p.PB;
  const int NCH = G * D / 16;
  const int pl = tid / TPT, j = tid % TPT, t = i0 + pl;
  const bool live = pl < p.PB && t < p.Tq;
  auto chunk = [&](int c, v4u& a, v4u& b) __attribute__((always_inline)) {
    const char* src = st + (pl * G + (16 * c) / D) * orow + ((16 * c) % D) * 2;
    a = *reinterpret_cast<const v4u*>(src);
    b = *reinterpret_cast<const v4u*>(src + 16);
  };
  float amax = 0.0f;
  if (live)
    for (int c = j; c < NCH; c += TPT) {
      v4u a, b;
      chunk(c, a, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        amax = absmax2(amax, absmax2(fabsf(__uint_as_float(a[e] << 16)), fabsf(__uint_as_float(a[e] & 0xffff0000u))));
        amax = absmax2(amax, absmax2(fabsf(__uint_as_float(b[e] << 16)), fabsf(__uint_as_float(b[e] & 0xffff0000u))));
      }
    }
  for (int o = 1; o < TPT; o <<= 1) amax = absmax2(amax, __shfl_xor(amax, o, 64));
  const float s = quant_scale(amax);
  const float rs = 1.0f / s;
  if (live) {
    if (j == 0) p.qsx[t] = s;
    for (int c = j; c < NCH; c += TPT) {
      v4u h[2];
      chunk(c, h[0], h[1]);
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = uint8_t(quant1_bf16(__uint_as_float(h[hh][e] << 16), s, rs));
          const uint32_t hi = uint8_t(quant1_bf16(__uint_as_float(h[hh][e] & 0xffff0000u), s, rs));
          w[2 * hh + (e >> 1)] |= (lo | (hi << 8)) << (16 * (e & 1));
        }
      *reinterpret_cast<v4u*>(p.qpk + packed_act_offset(t, 16 * c, p.qKF)) = v4u{w[0], w[1], w[2], w[3]};
    }
  }
  if (tile == p.ntiles - 1)
    for (int x = tid; x < (p.qMp - p.Tq) * NCH; x += NT)
      *reinterpret_cast<v4u*>(p.qpk + packed_act_offset(p.Tq + x / NCH, 16 * (x % NCH), p.qKF)) = v4u{0u, 0u, 0u, 0u};
}

template <int D, int BN, int NW>
__global__ __launch_bounds__(NW * 64, 1) void attn_fwd_kernel(AttnParams p) {
  static_assert(D == 128 || D == 256 || D == 512, "head_dim 128, 256 or 512");
  static_assert(BN == 32 || BN == 64 || BN == 128, "key block 32, 64 or 128");
  constexpr int NT = NW * 64;
  constexpr int KCH = D / 8;                          // 16-byte chunks per key row
  constexpr int K_SLOT = BN * D * 2;                  // bytes of one K block
  constexpr int VLD = BN + 8;                         // padded V^T row, elements
  constexpr int V_SLOT = D * VLD * 2;                 // bytes of one V^T block
  constexpr int NKC = BN / 32;                        // 32-key chunks per block
  constexpr int KU = BN * KCH / NT;                   // K DMA instructions per wave per block
  constexpr int KG = BN / 4;                          // 4-key groups of a V block
  constexpr int VP = D * BN / (8 * 4 * NT);           // V staging passes per thread
  constexpr int NDT = D / 16;                         // 16-wide d tiles of O^T
  constexpr int NKK = D / 32;                         // k-steps of S^T
  static_assert(KU * NT == BN * KCH && VP * 8 * 4 * NT == D * BN, "tiling");
  constexpr int V_OFF = 2 * K_SLOT;
  static_assert(V_OFF + 2 * V_SLOT <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char lds[V_OFF + 2 * V_SLOT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 15, qq = lane >> 4;  // query column, lane group

  // ---- which KV group and query rows -------------------------------------------------------
  // Unsplit sliding windows: one workgroup per tile, neighbouring tiles (sharing their keys) on one
  // XCD.  Otherwise item b of every KV group in turn, so the longest items of all groups start
  // first (split sliding windows: every tile in the same number of parts).
  int g, b, tile, part = 0, nparts = 1;
  if (p.window > 0 && p.nsplit_tiles == 0) {
    const int lb = attn_xcd_remap(blockIdx.x, p.KV * p.per_group);
    g = lb / p.per_group;
    b = tile = lb % p.per_group;
  } else {
    g = int(blockIdx.x) % p.KV;
    b = int(blockIdx.x) / p.KV;
    if (p.ordered) b = p.order[b];
    if (b >= p.per_group) return;  // (never: the order table is a permutation of the items)
    int s = 0;
    while (s + 1 < p.nseg && b >= p.seg_item[s + 1]) ++s;
    nparts = p.seg_k[s];
    const int off = b - p.seg_item[s];
    tile = p.seg_tile[s] - off / nparts;
    part = off % nparts;
    if (tile < 0 || (nparts > 1 && b >= p.nsplit_items)) return;  // (never, as above)
  }
  const bool split_tile = nparts > 1;
  const int i0 = tile * p.PB;
  const int r = wave * 16 + qi;
  const int hl = r % p.G, pl = r / p.G;
  const int qrow = i0 + pl;
  const bool valid = pl < p.PB && qrow < p.Tq;
  const int h = g * p.G + hl;
  const int pos = p.q_start + qrow;

  const int pmin = p.q_start + i0;
  const int pmax = p.q_start + min(i0 + p.PB, p.Tq) - 1;
  const int khi = min(pmax, p.Tk - 1);
  const int klo = p.window > 0 ? max(0, pmin - p.window + 1) : 0;
  const int kb_first = (klo / BN) * BN;
  const int nblk_tile = khi >= kb_first ? (khi - kb_first) / BN + 1 : 0;
  // this workgroup's key blocks: part `part` of `nparts` consecutive ranges
  const int n_lo = part * nblk_tile / nparts;
  const int n_hi = (part + 1) * nblk_tile / nparts;
  const int kb0 = kb_first + n_lo * BN;
  const int nblk = n_hi - n_lo;

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + int64_t(g) * p.khs, p.k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + int64_t(g) * p.vhs, p.v_bytes);

  // ---- staging ------------------------------------------------------------------------------
  // K chunk x = (u * NW + wave) * 64 + lane of a block: key row x / KCH, stored chunk x % KCH,
  // holding source chunk (x % KCH) ^ swz(row), swz(row) = (row & 3) | ((row >> 1) & 12).
  uint32_t koff[KU];
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int x = (u * NW + wave) * 64 + lane;
    const int row = x / KCH, cs = x % KCH;
    const int c = cs ^ ((row & 3) | ((row >> 1) & 12));
    koff[u] = uint32_t(row) * uint32_t(p.krs) * 2u + uint32_t(c) * 16u;
  }
  auto issue_k = [&](int kb, int slot) {
    char* base = lds + slot * K_SLOT;
    const uint32_t rowoff = uint32_t(kb) * uint32_t(p.krs) * 2u;
#pragma unroll
    for (int u = 0; u < KU; ++u) attn_dma16(rk, base + (u * NW + wave) * 1024, rowoff + koff[u]);
  };
  // V: thread t stages keys 4*kg .. 4*kg+3 (kg = t % KG) at d = 8*(t / KG + ps * NT/KG) .. +7.
  const int kg = tid % KG, dg = tid / KG;
  v4i vr[VP][4];
  auto load_v = [&](int kb) {
#pragma unroll
    for (int ps = 0; ps < VP; ++ps)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t off = (uint32_t(kb + 4 * kg + e) * uint32_t(p.vrs) + uint32_t(8 * (dg + ps * (NT / KG)))) * 2u;
        vr[ps][e] = buf_load16(rv, off);
      }
  };
  auto store_vt = [&](int slot) {
    char* base = lds + V_OFF + slot * V_SLOT;
#pragma unroll
    for (int ps = 0; ps < VP; ++ps) {
      const int d0 = 8 * (dg + ps * (NT / KG));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int w = j >> 1;
        const uint32_t a0 = uint32_t(vr[ps][0][w]), a1 = uint32_t(vr[ps][1][w]);
        const uint32_t a2 = uint32_t(vr[ps][2][w]), a3 = uint32_t(vr[ps][3][w]);
        v2u pk;
        if (j & 1) {
          pk[0] = (a0 >> 16) | (a1 & 0xffff0000u);
          pk[1] = (a2 >> 16) | (a3 & 0xffff0000u);
        } else {
          pk[0] = (a0 & 0xffffu) | (a1 << 16);
          pk[1] = (a2 & 0xffffu) | (a3 << 16);
        }
        *reinterpret_cast<v2u*>(base + ((d0 + j) * VLD + 4 * kg) * 2) = pk;
      }
    }
  };

  // S^T tile 2c + hh (16 keys x 16 queries) row rho = 4 a + b holds key 32 c + 8 a + 4 hh + b, so
  // register i of lane group qq of tiles 2c, 2c+1 holds keys 32 c + 8 qq + {i, 4 + i}: the k-slot
  // order of the B operand of the O^T product.  This lane's A operand (row rho = qi) is key row
  // 32 c + 4 hh + krow, stored chunk (4 kk + qq) ^ qi (swz of that row is qi), i.e. at
  // kofs[kk % 4] + 256 (kk / 4) within the row.
  const int krow = 8 * (qi >> 2) + (qi & 3);
  uint32_t kofs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kofs[j] = uint32_t(krow * KCH * 16 + (((4 * j + qq) ^ qi) * 16));
  const uint32_t vofs = uint32_t((qi * VLD + 8 * qq) * 2);  // V^T row d = qi, keys 8 qq ..

  // ---- main loop -----------------------------------------------------------------------------
  v4f o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // Reference exponent of this lane's query, in log2 units: p = exp2(s * c - ms).  It follows the
  // running maximum of s * c lazily, moving only when a block's maximum exceeds it by more than 8
  // (so p <= 2^8: the same relative bf16 / fp32 rounding, far from any overflow), which keeps the
  // rescale of O to the few blocks where the maximum jumps; when it moves, O and l are rescaled
  // by exactly exp2(ms_old - ms_new), the ratio of the references the sums were taken against.
  float ms = -__builtin_inff();
  float l = 0.0f;  // this lane group's share of sum exp2(s * c - ms)
  const float c = p.c;
  const int win = p.window;
  const uint32_t wlim = attn_window_limit(win);
  const int Tk = p.Tk;

  // the first block's K and V loads go out before the Q loads, so their latencies overlap
  if (nblk > 0) {
    issue_k(kb0, 0);
    load_v(kb0);
  }
  // ---- Q fragments: B operand of v_mfma_f32_16x16x32_bf16, lane (qi, qq) holds
  // q[row qi][32 kk + 8 qq .. + 7] ---------------------------------------------------------------
  v8bf qf[NKK];
  {
    const uint16_t* qp = p.q + int64_t(h) * p.qhs + int64_t(qrow) * p.qrs + 8 * qq;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      v4i t = v4i{0, 0, 0, 0};
      if (valid) t = *reinterpret_cast<const v4i*>(qp + 32 * kk);
      qf[kk] = __builtin_bit_cast(v8bf, t);
    }
  }

  if (nblk > 0) store_vt(0);
  for (int n = 0; n < nblk; ++n) {
    const int kb = kb0 + n * BN;
    const int slot = n & 1;
    attn_wait_vmcnt<0>();
    __syncthreads();  // K and V^T of block n are in LDS; the other slots are free
    if (n + 1 < nblk) {
      issue_k(kb + BN, slot ^ 1);
      load_v(kb + BN);
    }

    // S^T = K Q^T: 2 NKC independent accumulators
    v4f s[2 * NKC];
    const char* kbase = lds + slot * K_SLOT;
#pragma unroll
    for (int t = 0; t < 2 * NKC; ++t) s[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
      for (int t = 0; t < 2 * NKC; ++t) {
        const int row0 = 32 * (t >> 1) + 4 * (t & 1);
        const v8bf a = *reinterpret_cast<const v8bf*>(kbase + kofs[kk % 4] + row0 * (KCH * 16) + (kk / 4) * 256);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[kk], s[t], 0, 0, 0);
      }

    // mask, block maximum, online softmax
    const bool edge = !valid || kb + BN - 1 > pmin || (win > 0 && kb < pmax - win + 1) || kb + BN > Tk;
    if (edge) {
#pragma unroll
      for (int t = 0; t < 2 * NKC; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb + 32 * (t >> 1) + 8 * qq + 4 * (t & 1) + i;
          s[t][i] = attn_mask(s[t][i], valid & attn_key_visible(key, pos, Tk, wlim));
        }
    }
    float bm = -__builtin_inff();
#pragma unroll
    for (int t = 0; t < 2 * NKC; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) bm = fmaxf(bm, s[t][i]);
    bm = lanes4_max(bm);
    const float bmc = bm * c;
    const bool grow = bmc > ms + 8.0f;  // false while every key so far is masked (bmc = -inf)
    const float alpha = !grow ? 1.0f : (ms == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(ms - bmc));
    if (grow) ms = bmc;
    const float mref = ms == -__builtin_inff() ? 0.0f : ms;
    float bs = 0.0f;
    v8bf pb[NKC];
#pragma unroll
    for (int ch = 0; ch < NKC; ++ch)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * ch + (j >> 2)][j & 3], c, -mref));
        bs += pe;
        pb[ch][j] = (__bf16)pe;
      }
    l = l * alpha + bs;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
    }

    // O^T += V^T P^T
    const char* vbase = lds + V_OFF + slot * V_SLOT + vofs;
#pragma unroll
    for (int ch = 0; ch < NKC; ++ch)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const v8bf a = *reinterpret_cast<const v8bf*>(vbase + (16 * dt * VLD + 32 * ch) * 2);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[ch], o[dt], 0, 0, 0);
      }

    if (n + 1 < nblk) store_vt(slot ^ 1);
  }

  // ---- output: o / l per row (bf16), and the logsumexp ms ln 2 + ln l -----------------------------
  auto row_sum = [&](float x) {  // the row's total over its four lane groups
    return lanes4_sum(x);
  };
  uint16_t* const op = p.o + int64_t(h) * p.ohs + int64_t(qrow) * p.ors + 4 * qq;
  // quantised output: the bf16 rows are staged in LDS (past the arrival word) for attn_quant_tokens
  constexpr int QROW = D * 2 + 16;
  static_assert(1024 + NW * 16 * QROW <= V_OFF + 2 * V_SLOT, "staged rows fit the LDS");
  char* const qst = lds + 1024;
  auto store_o = [&](int dt, v4f x, float inv) {
    if (!valid) return;
    v2u w;
    w[0] = pack_bf16x2(x[0] * inv, x[1] * inv);
    w[1] = pack_bf16x2(x[2] * inv, x[3] * inv);
    if (p.qpk)
      *reinterpret_cast<v2u*>(qst + r * QROW + (16 * dt + 4 * qq) * 2) = w;
    else
      *reinterpret_cast<v2u*>(op + 16 * dt) = w;
  };
  auto store_lse = [&](float m, float lt) {
    if (valid && p.lse && qq == 0)
      p.lse[int64_t(h) * p.Tq + qrow] = lt > 0.0f ? m * 0.69314718055994531f + __logf(lt) : -__builtin_inff();
  };

  // ---- split tiles: park this part; the last part to arrive merges them in part order ---------
  // The XCDs' L2 caches are not coherent with each other, so the parts go through system-scope
  // (sc0 sc1) buffer stores and loads and the arrival count is a system-scope atomic; each
  // thread's stores are complete (vmcnt 0) before the barrier that precedes the count.  A parked
  // part is slot-major (slot dt of every thread, then the next slot), so each store and load of a
  // wave covers 1 KiB of whole cache lines: these accesses bypass the caches, and a lane-major
  // layout (each lane's slots contiguous) made every one of them a partial-line write.
  if (split_tile) {
    constexpr uint32_t SLOT_BYTES = NT * 16;              // one 16-byte slot of every thread
    constexpr uint32_t PART_BYTES = (NDT + 1) * SLOT_BYTES;  // o[NDT] and (m, l)
    const int first_item = g * p.nsplit_items + (b - part);
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(p.part + size_t(first_item) * (PART_BYTES / 4), uint32_t(nparts) * PART_BYTES);
    const uint32_t lane_off = uint32_t(tid) * 16u;
    const uint32_t base = uint32_t(part) * PART_BYTES + lane_off;
    const v4f ml = v4f{ms, l, 0.0f, 0.0f};
    if (p.merge_mode) {
      // attn_merge_kernel merges the parts after this kernel, whose end writes the L2s back: plain
      // (write-back) stores suffice
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, o[dt]), rp, base + dt * SLOT_BYTES, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, ml), rp, base + NDT * SLOT_BYTES, 0, 0);
      return;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, o[dt]), rp, base + dt * SLOT_BYTES, 0, 0x11);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, ml), rp, base + NDT * SLOT_BYTES, 0, 0x11);
    __builtin_amdgcn_s_waitcnt(0);
    int* arrived = reinterpret_cast<int*>(lds);
    const int counter = g * p.nsplit_tiles + (p.ntiles - 1 - tile);
    __syncthreads();
    if (tid == 0)
      *arrived = __hip_atomic_fetch_add(p.counters + counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    if (*arrived != nparts - 1) return;
    // merge: M = max of the parts' references, w_s = exp2(ms_s - M), o = sum_s w_s o_s, l likewise,
    // each sum in part order.  NP (4, 8 or 16) >= nparts slots per sum are loaded unconditionally
    // -- those past the last part lie outside the buffer resource and read zero, and take weight
    // 0, so they add +0 to sums that are never -0 -- in batches of 16 loads per thread (DG d tiles
    // at a time), each summed and stored as soon as it arrives.
    auto merge = [&](auto np_tag) {
      constexpr int NP = decltype(np_tag)::value;
      constexpr int DG = 16 / NP;
      static_assert(NDT % DG == 0, "d tiles per batch");
      float wsp[NP], lsp[NP];
      float M = -__builtin_inff();
#pragma unroll
      for (int sp = 0; sp < NP; ++sp) {
        const v4f ml = __builtin_bit_cast(
            v4f, __builtin_amdgcn_raw_buffer_load_b128(rp, uint32_t(sp) * PART_BYTES + lane_off + NDT * SLOT_BYTES,
                                                       0, 0x11));
        wsp[sp] = sp < nparts ? ml[0] : -__builtin_inff();
        lsp[sp] = ml[1];
        M = fmaxf(M, wsp[sp]);
      }
      const float Ms = M == -__builtin_inff() ? 0.0f : M;
      float lm = 0.0f;
#pragma unroll
      for (int sp = 0; sp < NP; ++sp) {
        wsp[sp] = sp < nparts ? __builtin_amdgcn_exp2f(wsp[sp] - Ms) : 0.0f;
        lm = __builtin_fmaf(wsp[sp], lsp[sp], lm);
      }
      const float lt = row_sum(lm);
      const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
      for (int d0 = 0; d0 < NDT; d0 += DG) {
        v4f od[DG][NP];
#pragma unroll
        for (int j = 0; j < DG; ++j)
#pragma unroll
          for (int sp = 0; sp < NP; ++sp)
            od[j][sp] = __builtin_bit_cast(
                v4f, __builtin_amdgcn_raw_buffer_load_b128(
                         rp, uint32_t(sp) * PART_BYTES + lane_off + uint32_t(d0 + j) * SLOT_BYTES, 0, 0x11));
#pragma unroll
        for (int j = 0; j < DG; ++j) {
          v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int sp = 0; sp < NP; ++sp)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(wsp[sp], od[j][sp][i], acc[i]);
          store_o(d0 + j, acc, inv);
        }
      }
      store_lse(M, lt);
    };
    if (tid == 0) __hip_atomic_store(p.counters + counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (nparts <= 4)
      merge(std::integral_constant<int, 4>{});
    else if (nparts <= 8)
      merge(std::integral_constant<int, 8>{});
    else
      merge(std::integral_constant<int, 16>{});
    if (p.qpk) {
      __syncthreads();
      attn_quant_tokens<D, NT>(p, qst, QROW, i0, tile, tid);
    }
    return;
  }

  // ---- normalise and store --------------------------------------------------------------------
  const float lt = row_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (p.qpk) __syncthreads();  // every wave is done with the K / V slots the rows are staged over
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) store_o(dt, o[dt], inv);
  store_lse(ms, lt);
  if (p.qpk) {
    __syncthreads();
    attn_quant_tokens<D, NT>(p, qst, QROW, i0, tile, tid);
  }
}

// ---- prefill, head_dim split over the waves for P V -------------------------------------------
//
// attn_fwd2_kernel computes the same function as attn_fwd_kernel with the same work list and
// moves less data through LDS per key block.  NW waves (4 or 8) own the tile's 128 rows for the S
// phase, RT = 8 / NW row tiles of 16 each (Q of those rows in registers, K from LDS as the A
// operand: each K fragment feeds RT MFMAs).  The softmax writes the rows' P (bf16) and rescale
// factors to LDS, and the P V product is split over head_dim instead of rows: wave w computes O^T
// for columns [w D/NW, (w+1) D/NW) of all 128 rows, its V^T operand read from the row-major V rows
// (DMA'd like K, chunk x of row r stored at x ^ 2 (r & 3)) with ds_read_b64_tr_b16, its P^T operand
// from the P rows.  Per block the workgroup reads K NW times from LDS but V and P once each, and V
// needs no transposing pass through registers.  With 4 waves (one per SIMD, 512 registers each)
// the waves hold Q of 32 rows and a quarter of O^T and still have registers to keep several LDS
// reads in flight; with 8 (two per SIMD, 256 registers) head_dim 512 leaves room for one.
//
// Pipeline, one barrier per key block: iteration n computes P V of block n and the S phase and
// softmax of block n + 1, while the DMAs of K(n + 2) and V(n + 1) are in flight; K, V and P each
// have two slots (block n in slot n % 2).  Key masking is branch-free so the two phases share one
// basic block.  The O rescale for a grown row maximum (rare: the reference exponent trails the
// maximum lazily) is skipped unless some row of the workgroup grew past a finite maximum.
//
// Split tiles park O^T slot-major (slot (dt, rt) of every thread, then the next slot) followed by
// each row's (m, l, 0, 0); the merging workgroup first turns the parts' (m, l) into per-row
// weights in LDS, then sums each O^T slot over the parts in part order.
template <int D, int BN, int NW>
struct AttnFwd2Shape {
  static constexpr int NT = NW * 64;
  static constexpr int RT = 8 / NW;                  // 16-row tiles per wave in the S phase
  static constexpr int KCH = D / 8;                  // 16-byte chunks per K / V row
  static constexpr int ROW = D * 2;                  // bytes per K / V row
  static constexpr int KV_SLOT = BN * ROW;           // one K or V block
  static constexpr int PLD = BN + 8;                 // padded P row, elements
  static constexpr int P_SLOT = 128 * PLD * 2;       // the 128 rows' P of one block
  static constexpr int V_OFF = 2 * KV_SLOT, P_OFF = 4 * KV_SLOT, A_OFF = P_OFF + 2 * P_SLOT;
  static constexpr int A_BYTES = 2 * 128 * 4 + 2 * 16 * 4 + 128 * 4;  // alpha [2][128], flags [2][16], inv [128]
  static constexpr int LDS = A_OFF + A_BYTES;
  static constexpr int NDW = D / NW / 16;            // 16-wide d tiles of O^T per wave
  static constexpr int SLOTS = NDW * 8;              // O^T registers (v4f) per thread
  static constexpr uint32_t PART_O = uint32_t(SLOTS) * NT * 16;
  static constexpr uint32_t PART_BYTES = PART_O + 128 * 16;  // + each row's (m, l, 0, 0)
};

template <int D, int BN, int NW>
__global__ __launch_bounds__(NW * 64, 1) void attn_fwd2_kernel(AttnParams p) {
  using S = AttnFwd2Shape<D, BN, NW>;
  constexpr int NT = S::NT, RT = S::RT, KCH = S::KCH, ROW = S::ROW, PLD = S::PLD, NDW = S::NDW;
  constexpr int NKC = BN / 32;                       // 32-key chunks per block
  constexpr int KU = BN * KCH / NT;                  // DMA instructions per thread per K or V block
  constexpr int NKK = D / 32;                        // k-steps of S^T
  static_assert((NW == 4 || NW == 8) && KU * NT == BN * KCH && NDW >= 1, "tiling");
  static_assert(S::LDS <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char lds[S::LDS];
  float* const alpha_s = reinterpret_cast<float*>(lds + S::A_OFF);       // [2][128]
  int* const flag_s = reinterpret_cast<int*>(lds + S::A_OFF + 1024);     // [2][16]
  float* const inv_s = reinterpret_cast<float*>(lds + S::A_OFF + 1152);  // [128]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 15, qq = lane >> 4;

  // ---- which KV group and query rows (as attn_fwd_kernel) ----------------------------------
  int g, b, tile, part = 0, nparts = 1;
  if (p.window > 0 && p.nsplit_tiles == 0) {
    const int lb = attn_xcd_remap(blockIdx.x, p.KV * p.per_group);
    g = lb / p.per_group;
    b = tile = lb % p.per_group;
  } else {
    g = int(blockIdx.x) % p.KV;
    b = int(blockIdx.x) / p.KV;
    if (p.ordered) b = p.order[b];
    if (b >= p.per_group) return;  // (never: the order table is a permutation of the items)
    int s = 0;
    while (s + 1 < p.nseg && b >= p.seg_item[s + 1]) ++s;
    nparts = p.seg_k[s];
    const int off = b - p.seg_item[s];
    tile = p.seg_tile[s] - off / nparts;
    part = off % nparts;
    if (tile < 0 || (nparts > 1 && b >= p.nsplit_items)) return;  // (never, as above)
  }
  const bool split_tile = nparts > 1;
  // the lambdas below read these copies, never p itself: a reference to the kernel arguments
  // would make the compiler copy the whole argument block (launch-order table included) to scratch
  const int G = p.G, PB = p.PB, Tq = p.Tq;
  const uint32_t krs2 = uint32_t(p.krs) * 2u, vrs2 = uint32_t(p.vrs) * 2u;
  uint16_t* const out = p.o;
  const int64_t ohs = p.ohs, ors = p.ors;
  float* const lse = p.lse;
  const int i0 = tile * PB;
  // row r of the tile is (head r % G, position r / G); this lane's S-phase rows are
  // srow[j] = 16 (RT wave + j) + qi
  auto row_valid = [&](int r) __attribute__((always_inline)) { return r / G < PB && i0 + r / G < Tq; };
  int srow[RT], pos[RT];
  bool valid[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    srow[j] = 16 * (RT * wave + j) + qi;
    valid[j] = row_valid(srow[j]);
    pos[j] = p.q_start + i0 + srow[j] / G;
  }

  const int pmin = p.q_start + i0;
  const int pmax = p.q_start + min(i0 + PB, Tq) - 1;
  const int khi = min(pmax, p.Tk - 1);
  const int klo = p.window > 0 ? max(0, pmin - p.window + 1) : 0;
  const int kb_first = (klo / BN) * BN;
  const int nblk_tile = khi >= kb_first ? (khi - kb_first) / BN + 1 : 0;
  const int n_lo = part * nblk_tile / nparts;
  const int n_hi = (part + 1) * nblk_tile / nparts;
  const int kb0 = kb_first + n_lo * BN;
  const int nblk = n_hi - n_lo;

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + int64_t(g) * p.khs, p.k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + int64_t(g) * p.vhs, p.v_bytes);

  // ---- DMA offsets: chunk x = (u NW + wave) 64 + lane of a block is key row x / KCH, stored
  // chunk x % KCH; K holds source chunk (x % KCH) ^ swz(row), swz(row) = (row & 3) | ((row >> 1)
  // & 12), V holds source chunk (x % KCH) ^ 2 (row & 3).
  uint32_t koff[KU], voff[KU];
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    const int x = (u * NW + wave) * 64 + lane;
    const int row = x / KCH, cs = x % KCH;
    koff[u] = uint32_t(row) * krs2 + uint32_t(cs ^ ((row & 3) | ((row >> 1) & 12))) * 16u;
    voff[u] = uint32_t(row) * vrs2 + uint32_t(cs ^ (2 * (row & 3))) * 16u;
  }
  auto issue_k = [&](int kb, int slot) __attribute__((always_inline)) {
    char* base = lds + slot * S::KV_SLOT;
    const uint32_t rowoff = uint32_t(kb) * krs2;
#pragma unroll
    for (int u = 0; u < KU; ++u) attn_dma16(rk, base + (u * NW + wave) * 1024, rowoff + koff[u]);
  };
  auto issue_v = [&](int kb, int slot) __attribute__((always_inline)) {
    char* base = lds + S::V_OFF + slot * S::KV_SLOT;
    const uint32_t rowoff = uint32_t(kb) * vrs2;
#pragma unroll
    for (int u = 0; u < KU; ++u) attn_dma16(rv, base + (u * NW + wave) * 1024, rowoff + voff[u]);
  };

  // ---- first blocks' loads, then Q (B operand: lane (qi, qq) of row tile j holds
  // q[srow[j]][32 kk + 8 qq .. + 7]) ------------------------------------------------------------
  if (nblk > 0) {
    issue_k(kb0, 0);
    issue_v(kb0, 0);
  }
  v8bf qf[RT][NKK];
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const uint16_t* qp = p.q + int64_t(g * G + srow[j] % G) * p.qhs + int64_t(i0 + srow[j] / G) * p.qrs + 8 * qq;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      v4i t = v4i{0, 0, 0, 0};
      if (valid[j]) t = *reinterpret_cast<const v4i*>(qp + 32 * kk);
      qf[j][kk] = __builtin_bit_cast(v8bf, t);
    }
  }
  if (nblk > 1) issue_k(kb0 + BN, 1);

  // ---- S phase operand offsets (K rows of S^T tile 2c + hh, as attn_fwd_kernel) ------------
  const int krow = 8 * (qi >> 2) + (qi & 3);
  uint32_t kofs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kofs[j] = uint32_t(krow * KCH * 16 + (((4 * j + qq) ^ qi) * 16));

  // running softmax state of rows srow[j]: reference exponent ms (log2 units, trailing the maximum
  // by at most 8) and this lane group's share l of sum exp2(s c - ms)
  float ms[RT], l[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    ms[j] = -__builtin_inff();
    l[j] = 0.0f;
  }
  const float c = p.c;
  const int win = p.window;
  const uint32_t wlim = attn_window_limit(win);
  const int Tk = p.Tk;

  // S^T of block n (K slot n % 2), softmax, P rows and rescale factors into slot n % 2
  auto s_phase = [&](int n) __attribute__((always_inline)) {
    const int kb = kb0 + n * BN;
    const int slot = n & 1;
    v4f s[RT][2 * NKC];
    const char* kbase = lds + slot * S::KV_SLOT;
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int t = 0; t < 2 * NKC; ++t) s[j][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // K fragments through a ring of KR registers: fragment i + KR is read once fragment i has fed
    // its MFMAs, so KR reads are in flight while the MFMAs run
    constexpr int NR = NKK * 2 * NKC, KR = 3;
    auto kfrag = [&](int i) __attribute__((always_inline)) {
      const int kk = i / (2 * NKC), t = i % (2 * NKC);
      const int row0 = 32 * (t >> 1) + 4 * (t & 1);
      return *reinterpret_cast<const v8bf*>(kbase + kofs[kk % 4] + row0 * (KCH * 16) + (kk / 4) * 256);
    };
    v8bf kf[KR];
#pragma unroll
    for (int i = 0; i < KR; ++i) kf[i] = kfrag(i);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int kk = i / (2 * NKC), t = i % (2 * NKC);
#pragma unroll
      for (int j = 0; j < RT; ++j) s[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[i % KR], qf[j][kk], s[j][t], 0, 0, 0);
      if (i + KR < NR) kf[i % KR] = kfrag(i + KR);
    }
    bool any = false;
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      float bm = -__builtin_inff();
#pragma unroll
      for (int t = 0; t < 2 * NKC; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb + 32 * (t >> 1) + 8 * qq + 4 * (t & 1) + i;
          s[j][t][i] = attn_mask(s[j][t][i], valid[j] & attn_key_visible(key, pos[j], Tk, wlim));
          bm = fmaxf(bm, s[j][t][i]);
        }
      bm = lanes4_max(bm);
      const float bmc = bm * c;
      const bool grow = bmc > ms[j] + 8.0f;  // false while every key so far is masked (bmc = -inf)
      const bool had = ms[j] != -__builtin_inff();
      const float alpha = !grow ? 1.0f : (had ? __builtin_amdgcn_exp2f(ms[j] - bmc) : 0.0f);
      ms[j] = grow ? bmc : ms[j];
      const float mref = ms[j] == -__builtin_inff() ? 0.0f : ms[j];
      float bs = 0.0f;
      uint16_t* prow = reinterpret_cast<uint16_t*>(lds + S::P_OFF + slot * S::P_SLOT) + srow[j] * PLD + 8 * qq;
#pragma unroll
      for (int ch = 0; ch < NKC; ++ch) {
        v8bf pb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][2 * ch + (e >> 2)][e & 3], c, -mref));
          bs += pe;
          pb[e] = (__bf16)pe;
        }
        *reinterpret_cast<v8bf*>(prow + 32 * ch) = pb;
      }
      l[j] = l[j] * alpha + bs;
      if (qq == 0) alpha_s[slot * 128 + srow[j]] = alpha;
      any = any || (grow && had);
    }
    // a row whose maximum grew past a finite one needs its O rescaled (a row that had none has O = 0)
    const bool wave_any = __builtin_amdgcn_ballot_w64(any) != 0;
    if (lane == 0) flag_s[slot * 16 + wave] = wave_any ? 1 : 0;
  };

  // ---- O^T for columns [wave D/NW, (wave+1) D/NW) of all rows: o[dt][rt] register i of lane
  // (qi, qq) is d = wave D/NW + 16 dt + 4 qq + i, row 16 rt + qi -------------------------------
  v4f o[NDW][8];
#pragma unroll
  for (int dt = 0; dt < NDW; ++dt)
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) o[dt][rt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const int vsrc = qq * 8 + (qi >> 2);  // this lane's V source row within a 32-key chunk (+4)
  auto pv_phase = [&](int n) __attribute__((always_inline)) {
    const int slot = n & 1;
    const int* fl = flag_s + slot * 16;
    int f = 0;
#pragma unroll
    for (int w4 = 0; w4 < NW; w4 += 4) {
      const v4i fv = *reinterpret_cast<const v4i*>(fl + w4);
      f |= fv[0] | fv[1] | fv[2] | fv[3];
    }
    if (f != 0) {
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const float a = alpha_s[slot * 128 + rt * 16 + qi];
#pragma unroll
        for (int dt = 0; dt < NDW; ++dt) o[dt][rt] *= a;
      }
    }
    const char* vl = lds + S::V_OFF + slot * S::KV_SLOT;
    const uint16_t* pl = reinterpret_cast<const uint16_t*>(lds + S::P_OFF + slot * S::P_SLOT);
#pragma unroll
    for (int ch = 0; ch < NKC; ++ch) {
      v8bf va[NDW];
#pragma unroll
      for (int dt = 0; dt < NDW; ++dt) {
        const int d = wave * (D / NW) + 16 * dt + 4 * (qi & 3);  // this lane's 4 source columns
        const int r0 = 32 * ch + vsrc, r1 = r0 + 4;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(
            vl + r0 * ROW + (((d >> 3) ^ (2 * (r0 & 3))) * 16) + (d & 7) * 2));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(
            vl + r1 * ROW + (((d >> 3) ^ (2 * (r1 & 3))) * 16) + (d & 7) * 2));
        va[dt] = __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const v8bf pb = *reinterpret_cast<const v8bf*>(pl + (rt * 16 + qi) * PLD + 32 * ch + 8 * qq);
#pragma unroll
        for (int dt = 0; dt < NDW; ++dt) o[dt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pb, o[dt][rt], 0, 0, 0);
      }
    }
  };

  // ---- main loop --------------------------------------------------------------------------
  // iteration n: P V of block n and the S phase of block n + 1 (one basic block, so their MFMAs
  // and LDS reads interleave), with K(n + 2) and V(n + 1) loading into the slots freed by
  // iteration n - 1
  if (nblk > 0) {
    if (nblk > 1)
      attn_wait_vmcnt<KU>();  // K(0), V(0) and Q have landed; K(1) may be in flight
    else
      attn_wait_vmcnt<0>();
    __syncthreads();
    s_phase(0);
  }
  for (int n = 0; n + 1 < nblk; ++n) {
    attn_wait_vmcnt<0>();
    __syncthreads();  // P(n) of every row; K(n + 1) and V(n) in LDS; the other slots free
    if (n + 2 < nblk) issue_k(kb0 + (n + 2) * BN, n & 1);
    issue_v(kb0 + (n + 1) * BN, (n + 1) & 1);
    pv_phase(n);
    s_phase(n + 1);
  }
  if (nblk > 0) {
    attn_wait_vmcnt<0>();
    __syncthreads();
    pv_phase(nblk - 1);
  }

  // ---- output ---------------------------------------------------------------------------------
  const int d_lane = wave * (D / NW) + 4 * qq;  // + 16 dt + i
  auto out_row = [&](int r) __attribute__((always_inline)) {  // output row pointer of tile row r
    const int hl = r % G, pr = r / G;
    return out + int64_t(g * G + hl) * ohs + int64_t(i0 + pr) * ors;
  };
  // quantised output: the bf16 rows are staged in LDS past the merge weights and below the row
  // factors, for attn_quant_tokens
  constexpr int QOFF = 16 * 1024, QROW = D * 2;
  static_assert(QOFF + 128 * QROW <= S::A_OFF && ATTN_MAX_SEG * 128 * 4 + 1024 <= QOFF, "staged rows fit");
  auto store_slot = [&](int dt, int rt, v4f x, float inv) __attribute__((always_inline)) {
    const int r = rt * 16 + qi;
    if (!row_valid(r)) return;
    v2u w;
    w[0] = pack_bf16x2(x[0] * inv, x[1] * inv);
    w[1] = pack_bf16x2(x[2] * inv, x[3] * inv);
    if (p.qpk)
      *reinterpret_cast<v2u*>(lds + QOFF + r * QROW + (d_lane + 16 * dt) * 2) = w;
    else
      *reinterpret_cast<v2u*>(out_row(r) + d_lane + 16 * dt) = w;
  };
  auto store_lse = [&](int r, float m, float lt) __attribute__((always_inline)) {
    if (row_valid(r) && lse)
      lse[int64_t(g * G + r % G) * Tq + i0 + r / G] = lt > 0.0f ? m * 0.69314718055994531f + __logf(lt) : -__builtin_inff();
  };
  float lt[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    lt[j] = lanes4_sum(l[j]);
  }

  if (split_tile) {
    // park O^T slot-major and each row's (ms, l); the last part to arrive merges in part order
    const int first_item = g * p.nsplit_items + (b - part);
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(p.part + size_t(first_item) * (S::PART_BYTES / 4), uint32_t(nparts) * S::PART_BYTES);
    const uint32_t lane_off = uint32_t(tid) * 16u;
    // write-through (system-scope) stores when the last part merges in this kernel on another XCD;
    // plain stores when attn_merge_kernel merges after this kernel, whose end writes the L2s back
    auto park = [&](auto policy) __attribute__((always_inline)) {
      constexpr int POL = decltype(policy)::value;
      const uint32_t base = uint32_t(part) * S::PART_BYTES;
#pragma unroll
      for (int dt = 0; dt < NDW; ++dt)
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, o[dt][rt]), rp,
                                                 base + uint32_t(dt * 8 + rt) * (NT * 16) + lane_off, 0, POL);
      if (qq == 0) {
#pragma unroll
        for (int j = 0; j < RT; ++j) {
          const v4f ml = v4f{ms[j], lt[j], 0.0f, 0.0f};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, ml), rp,
                                                 base + S::PART_O + uint32_t(srow[j]) * 16u, 0, POL);
        }
      }
    };
    if (p.merge_mode) {
      park(std::integral_constant<int, 0>{});
      return;
    }
    park(std::integral_constant<int, 0x11>{});
    __builtin_amdgcn_s_waitcnt(0);
    int* arrived = reinterpret_cast<int*>(lds);
    const int counter = g * p.nsplit_tiles + (p.ntiles - 1 - tile);
    __syncthreads();
    if (tid == 0)
      *arrived = __hip_atomic_fetch_add(p.counters + counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    if (*arrived != nparts - 1) return;
    if (tid == 0) __hip_atomic_store(p.counters + counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    // per-row weights w_s = exp2(m_s - M) (0 past the last part) into LDS, 1 / sum_s w_s l_s too
    float* const wts = reinterpret_cast<float*>(lds + 1024);  // [ATTN_MAX_SEG][128], over the K slots
    if (tid < 128) {
      float M = -__builtin_inff();
      float mv[ATTN_MAX_SEG], lv[ATTN_MAX_SEG];
#pragma unroll
      for (int sp = 0; sp < ATTN_MAX_SEG; ++sp) {
        // (16-byte records: this compiler lowers __builtin_amdgcn_raw_buffer_load_b64 to a one-dword load)
        const v4f ml = sp < nparts ? __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                         rp, uint32_t(sp) * S::PART_BYTES + S::PART_O + uint32_t(tid) * 16u, 0, 0x11))
                                   : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        mv[sp] = sp < nparts ? ml[0] : -__builtin_inff();
        lv[sp] = ml[1];
        M = fmaxf(M, mv[sp]);
      }
      const float Ms = M == -__builtin_inff() ? 0.0f : M;
      float L = 0.0f;
#pragma unroll
      for (int sp = 0; sp < ATTN_MAX_SEG; ++sp) {
        const float w = sp < nparts ? __builtin_amdgcn_exp2f(mv[sp] - Ms) : 0.0f;
        wts[sp * 128 + tid] = w;
        L = __builtin_fmaf(w, lv[sp], L);
      }
      inv_s[tid] = L > 0.0f ? 1.0f / L : 0.0f;
      store_lse(tid, M, L);
    }
    __syncthreads();
    auto merge = [&](auto np_tag) __attribute__((always_inline)) {
      constexpr int NP = decltype(np_tag)::value;
      constexpr int DG = 16 / NP;  // O^T slots per batch of 16 loads
      static_assert((NDW * 8) % DG == 0, "slots per batch");
#pragma unroll
      for (int s0 = 0; s0 < NDW * 8; s0 += DG) {
        v4f od[DG][NP];
#pragma unroll
        for (int j = 0; j < DG; ++j)
#pragma unroll
          for (int sp = 0; sp < NP; ++sp)
            od[j][sp] = __builtin_bit_cast(
                v4f, __builtin_amdgcn_raw_buffer_load_b128(
                         rp, uint32_t(sp) * S::PART_BYTES + uint32_t(s0 + j) * (NT * 16) + lane_off, 0, 0x11));
#pragma unroll
        for (int j = 0; j < DG; ++j) {
          const int dt = (s0 + j) / 8, rt = (s0 + j) % 8;
          v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int sp = 0; sp < NP; ++sp) {
            const float w = wts[sp * 128 + rt * 16 + qi];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(w, od[j][sp][i], acc[i]);
          }
          store_slot(dt, rt, acc, inv_s[rt * 16 + qi]);
        }
      }
    };
    if (nparts <= 4)
      merge(std::integral_constant<int, 4>{});
    else if (nparts <= 8)
      merge(std::integral_constant<int, 8>{});
    else
      merge(std::integral_constant<int, 16>{});
    if (p.qpk) {
      __syncthreads();
      attn_quant_tokens<D, NT>(p, lds + QOFF, QROW, i0, tile, tid);
    }
    return;
  }

  // ---- normalise and store ------------------------------------------------------------------
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    if (qq == 0) {
      inv_s[srow[j]] = lt[j] > 0.0f ? 1.0f / lt[j] : 0.0f;
      store_lse(srow[j], ms[j], lt[j]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int dt = 0; dt < NDW; ++dt)
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) store_slot(dt, rt, o[dt][rt], inv_s[rt * 16 + qi]);
  if (p.qpk) {
    __syncthreads();
    attn_quant_tokens<D, NT>(p, lds + QOFF, QROW, i0, tile, tid);
  }
}

// ---- merge of parked parts (merge_mode 1) ------------------------------------------------------
//
// Where every part of a call would run in one round on the CUs, the last part of a tile to arrive
// would merge its tile's parts on one CU at the end (one tile at head_dim 512 parks ~256 KiB per
// part), so instead the parts are only parked and this kernel merges them, spread over one
// workgroup per (KV group, split tile, 16-byte slot of the parked O^T): 16 (head_dim 256) or 32
// (head_dim 512) workgroups per tile.  Thread t merges what thread t of the attention workgroup
// parked in that slot -- 4 output columns of one row -- with the arithmetic of the in-kernel merge
// (weights exp2(m_s - M) in part order, the row's l summed the same way), so both modes give the
// same bits.
//   FWD2 = false (attn_fwd_kernel): slot dt of thread t = (wave, qq, qi) holds row 16 wave + qi,
//     columns 16 dt + 4 qq ..; slot D/16 holds that thread's (m, lane-group share of l).
//   FWD2 = true (attn_fwd2_kernel): slot 8 dt + rt holds row 16 rt + qi, columns
//     wave D/8 + 4 qq + 16 dt ..; each row's (m, l) sits after the slots.
template <int D, bool FWD2>
__global__ __launch_bounds__(512) void attn_merge_kernel(AttnParams p) {
  using S2 = AttnFwd2Shape<D, 32, ATTN_FWD2_NW>;
  constexpr int NT = 512;
  constexpr uint32_t SLOT_BYTES = NT * 16;
  constexpr int NSLOT = FWD2 ? S2::SLOTS : D / 16;
  constexpr uint32_t PART_BYTES = FWD2 ? S2::PART_BYTES : uint32_t(D / 16 + 1) * SLOT_BYTES;
  static_assert(!FWD2 || (ATTN_FWD2_NW * 64 == NT && S2::NDW * 8 == NSLOT), "head_dim 512 layout");
  static_assert(FWD2 || ATTN_NW * 64 == NT, "attn_fwd_kernel layout");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, qi = lane & 15, qq = lane >> 4;
  // The NSLOT workgroups of a split tile each write a few columns of every row of the tile: dealt
  // to one XCD (consecutive logical workgroups), so each output line is assembled in one L2.
  const int lb = attn_xcd_remap(int(blockIdx.x), int(gridDim.x));
  const int slot = lb % NSLOT;
  const int st = (lb / NSLOT) % p.nsplit_tiles;
  const int g = lb / (NSLOT * p.nsplit_tiles);
  // split tile st is tile ntiles - 1 - st; its parts are consecutive items of its segment
  const int tile = p.ntiles - 1 - st;
  int s = 0;
  while (s + 1 < p.nseg && tile <= p.seg_tile[s + 1]) ++s;
  const int nparts = p.seg_k[s];
  const int first_item = g * p.nsplit_items + p.seg_item[s] + (p.seg_tile[s] - tile) * nparts;
  const __amdgpu_buffer_rsrc_t rp =
      make_rsrc(p.part + size_t(first_item) * (PART_BYTES / 4), uint32_t(nparts) * PART_BYTES);
  int r, d;
  uint32_t ml_off;
  if constexpr (FWD2) {
    r = (slot % 8) * 16 + qi;
    d = wave * (D / ATTN_FWD2_NW) + 4 * qq + 16 * (slot / 8);
    ml_off = S2::PART_O + uint32_t(r) * 16u;
  } else {
    r = wave * 16 + qi;
    d = 16 * slot + 4 * qq;
    ml_off = uint32_t(NSLOT) * SLOT_BYTES + uint32_t(tid) * 16u;
  }
  // NP >= nparts records per sum are loaded unconditionally, all before any is used: those past the
  // last part lie outside the buffer resource, read zero and take weight 0
  auto merge = [&](auto np_tag, float& M, float& lt, v4f& acc) __attribute__((always_inline)) {
    constexpr int NP = decltype(np_tag)::value;
    v4f mlv[NP], od[NP];
#pragma unroll
    for (int sp = 0; sp < NP; ++sp) {
      mlv[sp] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rp, uint32_t(sp) * PART_BYTES + ml_off, 0, 0));
      od[sp] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                             rp, uint32_t(sp) * PART_BYTES + uint32_t(slot) * SLOT_BYTES +
                                                     uint32_t(tid) * 16u, 0, 0));
    }
    float w[NP];
    M = -__builtin_inff();
#pragma unroll
    for (int sp = 0; sp < NP; ++sp) {
      w[sp] = sp < nparts ? mlv[sp][0] : -__builtin_inff();
      M = fmaxf(M, w[sp]);
    }
    const float Ms = M == -__builtin_inff() ? 0.0f : M;
    float lm = 0.0f;
#pragma unroll
    for (int sp = 0; sp < NP; ++sp) {
      w[sp] = sp < nparts ? __builtin_amdgcn_exp2f(w[sp] - Ms) : 0.0f;
      lm = __builtin_fmaf(w[sp], mlv[sp][1], lm);
    }
    lt = FWD2 ? lm : lanes4_sum(lm);
    acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int sp = 0; sp < NP; ++sp)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(w[sp], od[sp][i], acc[i]);
  };
  float M, lt;
  v4f acc;
  if (nparts <= 4)
    merge(std::integral_constant<int, 4>{}, M, lt, acc);
  else if (nparts <= 8)
    merge(std::integral_constant<int, 8>{}, M, lt, acc);
  else
    merge(std::integral_constant<int, 16>{}, M, lt, acc);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  const int i0 = tile * p.PB, pr = r / p.G, hl = r % p.G;
  if (pr >= p.PB || i0 + pr >= p.Tq) return;
  const int h = g * p.G + hl;
  v2u w;
  w[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  w[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<v2u*>(p.o + int64_t(h) * p.ohs + int64_t(i0 + pr) * p.ors + d) = w;
  if (d == 0 && p.lse)
    p.lse[int64_t(h) * p.Tq + i0 + pr] = lt > 0.0f ? M * 0.69314718055994531f + __logf(lt) : -__builtin_inff();
}

// ---- decode: one query per head, keys split into chunks --------------------------------------
//
// The reference's decode step (local_attn.py:44-68, _split_kv_decode; local_sdpa's decode branch,
// local_attn.py:74-83) attends one query per head to the cache (or its last W entries), splitting
// the keys into chunks whose partial results are merged by their logsumexp.  Here
// attn_decode_split_kernel computes, per (KV group, chunk of 32 or 64 keys), the G heads' chunk
// maximum M, sum L = sum_j exp2((s_j - M) c) and unnormalised o = sum_j bf16(exp2((s_j - M) c)) v_j;
// attn_decode_merge_kernel combines the chunks in chunk order (deterministic).
//
// Split kernel, 4 waves: the chunk's K and V rows are loaded into LDS at once by DMA.  Wave w
// computes the 16-key S^T tile w (16x16x32 bf16 MFMA, K rows from LDS as the A operand, the G <= 16
// query rows in registers as the B operand); the chunk's softmax goes through LDS; then wave w
// computes O^T for head_dim columns [w D/4, (w+1) D/4) as V^T P^T, its V^T operand read from the
// row-major V rows with ds_read_b64_tr_b16 (result lane i, slot j = lane 4j + i/4's element i%4 of a
// 16-lane group), its P^T operand from LDS.
// keys per chunk: 64 (32 at head_dim 512, so that two workgroups fit in a CU's LDS)

struct DecodeParams {
  const uint16_t* q; int64_t qhs;       // bf16 [H, D]
  const uint16_t* k; int64_t khs, krs;  // bf16 [KV, Tk, D]
  const uint16_t* v; int64_t vhs, vrs;
  uint16_t* o; int64_t ohs;             // bf16 [H, D]
  float* lse;                           // [H] or null
  float* part_o;                        // [KV][nchunk][G][D] unnormalised partial outputs
  float* part_ml;                       // [KV][nchunk][G][2] chunk maximum and sum
  uint32_t k_bytes, v_bytes;
  int H, KV, G, Tk, klo, pos, nchunk;
  float scale, c;
  // Position in device memory (a decode step replayed from a graph): the query position is
  // *pos_dev, the keys [klo, pos] with klo from `window`; the grid holds nchunk_grid chunks per KV
  // head, enough for any position the cache holds.  Null: pos / klo / nchunk / Tk above, and
  // nchunk_grid = nchunk.
  const int* pos_dev;
  int window, nchunk_grid;
  // k_qkv in the kernel (qkv_y non-null; with pos_dev, G <= 8): q is made from the token's qkv row
  // [H*D q | KV*D k | KV*D v] (bf16) -- per head RMS norm with qw (null: no weight) and RoPE with the
  // cos / sin rows [D] -- instead of read from q; with kv_write the workgroup holding the position
  // also makes the token's key (norm with kw, RoPE) and value (norm without weight) of its KV head,
  // writes them into k / v at the position (when it is inside the Tk rows) and attends to them there.
  const uint16_t* qkv_y; const uint16_t* rope_c; const uint16_t* rope_s;
  const uint16_t* qw; const uint16_t* kw;
  float qkv_eps; int kv_write; uint32_t qkv_bytes;  // bytes of the qkv row
  int rope_rows;  // rows of the cos / sin tables: row *pos_dev of them (1: that row whatever the position)
};

// The call's query position, first key, live chunks and key bound: the host's, or with pos_dev the
// position read from device memory, its chunks clamped to the launched grid (a position past the
// cache reads zero keys through the buffer bounds and never indexes past the grid's partials).
struct DecodeGeom {
  int pos, klo, nchunk, Tk;
};
template <int DEC_C>
__device__ __forceinline__ DecodeGeom decode_geom(const DecodeParams& p) {
  if (!p.pos_dev) return DecodeGeom{p.pos, p.klo, p.nchunk, p.Tk};
  const int pos = *p.pos_dev;
  const int klo = p.window > 0 ? max(0, pos - p.window + 1) : 0;
  const int nchunk = max(0, min((pos - klo) / DEC_C + 1, p.nchunk_grid));
  return DecodeGeom{pos, klo, nchunk, pos + 1};
}

// E bf16 values as the raw words they are loaded in (unpacked to fp32 when used); zero until loaded.
template <int E>
struct Bf16Words {
  uint32_t w[E == 4 ? 2 : 1] = {};
  // from byte offset off of the buffer r (past its end: zeros)
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (E == 4) {
      const v2u a = __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
      w[0] = a[0];
      w[1] = a[1];
    } else if constexpr (E == 2) {
      w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else {
      w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    }
  }
  __device__ __forceinline__ void unpack(float (&o)[E]) const {
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
  }
};

template <int D>
__global__ __launch_bounds__(256, 2) void attn_decode_split_kernel(DecodeParams p) {
  constexpr int DEC_C = dec_chunk(D);
  constexpr int KCH = D / 8;                 // 16-byte chunks per row
  constexpr int ROW = D * 2;                 // bytes per K / V row
  constexpr int KV_BYTES = DEC_C * ROW;      // one chunk of K (or V)
  constexpr int PLD = DEC_C + 8;             // padded P row, elements
  constexpr int NKK = D / 32;
  constexpr int NDT = D / 64;                // 16-wide d tiles per wave
  constexpr int DMA = DEC_C * KCH / 256;     // DMA instructions per thread per operand
  constexpr int QBYTES = 8 * D * 2;          // the made q rows of up to 8 heads (k_qkv in the kernel)
  __shared__ __attribute__((aligned(1024))) char lds[2 * KV_BYTES + 16 * PLD * 2 + 2 * 4 * 16 * 4 + QBYTES];
  char* const kl = lds;
  char* const vl = lds + KV_BYTES;
  uint16_t* const pl = reinterpret_cast<uint16_t*>(lds + 2 * KV_BYTES);
  float* const smax = reinterpret_cast<float*>(lds + 2 * KV_BYTES + 16 * PLD * 2);  // [4 waves][16]
  float* const ssum = smax + 64;
  uint16_t* const ql = reinterpret_cast<uint16_t*>(lds + 2 * KV_BYTES + 16 * PLD * 2 + 2 * 4 * 16 * 4);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 15, qq = lane >> 4;
  const DecodeGeom geo = decode_geom<DEC_C>(p);
  const int g = blockIdx.x / p.nchunk_grid, chunk = blockIdx.x % p.nchunk_grid;
  if (chunk >= geo.nchunk) return;           // (the whole workgroup, before any barrier)
  const int kc = geo.klo + chunk * DEC_C;    // first key of the chunk
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + int64_t(g) * p.khs, p.k_bytes);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + int64_t(g) * p.vhs, p.v_bytes);

  // k_qkv in the kernel: wave w makes q heads w and w + 4 of the group; in the workgroup holding the
  // position (with kv_write) wave 0 also makes the key and wave 1 the value.  Their operands are
  // fetched as raw bf16 words before the DMAs are issued and unpacked after, so the DMAs go out first.
  constexpr int E = D / 128, HALF = D / 2;
  const bool fused = p.qkv_y != nullptr;
  const bool make_kv = fused && p.kv_write && chunk == geo.nchunk - 1 && geo.pos >= 0 && geo.pos < p.Tk;
  const int p0 = lane * E;
  // operand o, half h: raw[o][h]; o = 0, 1: q heads wave, wave + 4; 2: key / value; 3: q weight;
  // 4: key weight; 5: cos; 6: sin
  // Every fetch is issued (an operand this wave does not use reads past its buffer's end as zeros),
  // so no branch stands between them and the DMAs.
  Bf16Words<E> raw[7][2];
  if (fused) {
    const uint32_t vec = uint32_t(D) * 2u;
    const uint32_t tab = uint32_t(p.rope_rows) * vec;  // a position past the tables reads zeros
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(p.qkv_y, p.qkv_bytes), rc = make_rsrc(p.rope_c, tab),
                                 rs = make_rsrc(p.rope_s, tab), rqw = make_rsrc(p.qw, p.qw ? vec : 0u),
                                 rkw = make_rsrc(p.kw, p.kw ? vec : 0u);
    auto fetch = [&](int o, __amdgpu_buffer_rsrc_t r, bool on, int row) __attribute__((always_inline)) {
      const uint32_t off = on ? (uint32_t(row) * uint32_t(D) + uint32_t(p0)) * 2u : 0x80000000u;
      raw[o][0].load(r, off);
      raw[o][1].load(r, off + uint32_t(HALF) * 2u);
    };
    const int rope_row = p.rope_rows > 1 ? max(geo.pos, 0) : 0;
    fetch(5, rc, p.rope_rows == 1 || geo.pos < p.rope_rows, rope_row);
    fetch(6, rs, p.rope_rows == 1 || geo.pos < p.rope_rows, rope_row);
    fetch(3, rqw, true, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) fetch(j, ry, wave + 4 * j < p.G, g * p.G + wave + 4 * j);
    fetch(2, ry, make_kv && wave < 2, p.H + (wave == 0 ? 0 : p.KV) + g);
    fetch(4, rkw, make_kv && wave == 0, 0);
  }

  // K chunk x of row r lands at stored chunk x ^ (r & 15); V chunk x of row r at x ^ 2 (r & 3).
#pragma unroll
  for (int u = 0; u < DMA; ++u) {
    const int x = (u * 4 + wave) * 64 + lane;
    const int r = x / KCH, cs = x % KCH;
    const uint32_t row = uint32_t(kc + r);
    attn_dma16(rk, kl + (u * 4 + wave) * 1024, row * uint32_t(p.krs) * 2u + uint32_t(cs ^ (r & 15)) * 16u);
    attn_dma16(rv, vl + (u * 4 + wave) * 1024, row * uint32_t(p.vrs) * 2u + uint32_t(cs ^ (2 * (r & 3))) * 16u);
  }
  // Q rows (B operand): lane (qi, qq) holds q[head g*G + qi][32 kk + 8 qq .. + 7], zero past G.
  v8bf qf[NKK];
  float xy1[E], xy2[E];
  if (fused) {
    // the q heads into LDS; the key / value into the cache (k_qkv_cache's stores)
    float rc1[E], rc2[E], rs1[E], rs2[E], w1[E], w2[E];
    raw[5][0].unpack(rc1);
    raw[5][1].unpack(rc2);
    raw[6][0].unpack(rs1);
    raw[6][1].unpack(rs2);
    raw[3][0].unpack(w1);
    raw[3][1].unpack(w2);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int hl = wave + 4 * j;
      if (hl < p.G) {
        float qy1[E], qy2[E];
        raw[j][0].unpack(qy1);
        raw[j][1].unpack(qy2);
        qkv_head_regs<E>(qy1, qy2, p.qkv_eps, p.qw != nullptr, w1, w2, true, rc1, rc2, rs1, rs2);
        store_bf16<E>(ql + hl * D + p0, qy1);
        store_bf16<E>(ql + hl * D + p0 + HALF, qy2);
      }
    }
    if (make_kv && wave < 2) {
      float xw1[E], xw2[E];
      raw[2][0].unpack(xy1);
      raw[2][1].unpack(xy2);
      raw[4][0].unpack(xw1);
      raw[4][1].unpack(xw2);
      qkv_head_regs<E>(xy1, xy2, p.qkv_eps, wave == 0 && p.kw != nullptr, xw1, xw2, wave == 0, rc1, rc2, rs1, rs2);
      uint16_t* dst = const_cast<uint16_t*>(wave == 0 ? p.k + int64_t(g) * p.khs + int64_t(geo.pos) * p.krs
                                                      : p.v + int64_t(g) * p.vhs + int64_t(geo.pos) * p.vrs);
      store_bf16<E>(dst + p0, xy1);
      store_bf16<E>(dst + p0 + HALF, xy2);
    }
  } else {
    const bool has = qi < p.G;
    const uint16_t* qp = p.q + int64_t(g * p.G + (has ? qi : 0)) * p.qhs + 8 * qq;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      v4i t = v4i{0, 0, 0, 0};
      if (has) t = *reinterpret_cast<const v4i*>(qp + 32 * kk);
      qf[kk] = __builtin_bit_cast(v8bf, t);
    }
  }
  attn_wait_vmcnt<0>();
  __syncthreads();
  if (make_kv) {
    // the token's row of the chunk (DMA'd from the cache before it was written) replaced by the made
    // key and value, in the chunk's swizzled layouts
    if (wave < 2) {
      const int r = geo.pos - kc;
      char* row = (wave == 0 ? kl : vl) + r * ROW;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int d = p0 + hh * HALF;
        const int cs = wave == 0 ? ((d >> 3) ^ (r & 15)) : ((d >> 3) ^ (2 * (r & 3)));
        store_bf16<E>(reinterpret_cast<uint16_t*>(row + cs * 16 + (d & 7) * 2), hh ? xy2 : xy1);
      }
    }
    __syncthreads();
  }
  if (fused) {
    const bool has = qi < p.G;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      v4i t = v4i{0, 0, 0, 0};
      if (has) t = *reinterpret_cast<const v4i*>(ql + qi * D + 32 * kk + 8 * qq);
      qf[kk] = __builtin_bit_cast(v8bf, t);
    }
  }

  // S^T tile: keys 16 wave + 4 qq + i (i = 0..3) of the chunk, query qi; two accumulators.
  const bool has_tile = 16 * wave < DEC_C;
  v4f s0 = v4f{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
  if (has_tile) {
    const int r = 16 * wave + qi;
    const char* kr = kl + r * ROW;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const v8bf a = *reinterpret_cast<const v8bf*>(kr + (((4 * kk + qq) ^ qi) * 16));
      if (kk & 1)
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[kk], s1, 0, 0, 0);
      else
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[kk], s0, 0, 0, 0);
    }
  }
  float sc[4];
  float bm = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = kc + 16 * wave + 4 * qq + i;
    sc[i] = attn_mask(s0[i] + s1[i], has_tile & attn_key_visible(key, geo.pos, geo.Tk, 0x80000000u));
    bm = fmaxf(bm, sc[i]);
  }
  bm = lanes4_max(bm);
  if (qq == 0) smax[wave * 16 + qi] = bm;
  __syncthreads();
  float M = fmaxf(fmaxf(smax[qi], smax[16 + qi]), fmaxf(smax[32 + qi], smax[48 + qi]));
  const float ms = M == -__builtin_inff() ? 0.0f : M * p.c;
  float ls = 0.0f;
  v4u pw;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], p.c, -ms));
    ls += pe;
    reinterpret_cast<uint16_t*>(&pw)[i] = f32_to_bf16(pe);
  }
  if (has_tile) *reinterpret_cast<v2u*>(pl + qi * PLD + 16 * wave + 4 * qq) = v2u{pw[0], pw[1]};
  ls = lanes4_sum(ls);
  if (qq == 0) ssum[wave * 16 + qi] = ls;
  __syncthreads();

  // O^T for d in [wave D/4, (wave+1) D/4): V^T operand by transposing reads of the V rows.
  v4f o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const int srow = qq * 8 + (qi >> 2);  // this lane's source row (+ 32 c, + 4 for slots 4..7)
#pragma unroll
  for (int c = 0; c < DEC_C / 32; ++c) {
    const v8bf b = *reinterpret_cast<const v8bf*>(pl + qi * PLD + 32 * c + 8 * qq);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = wave * (D / 4) + 16 * dt + 4 * (qi & 3);  // this lane's 4 source columns
      v4s lo, hi;
      {
        const int r = 32 * c + srow;
        const int cs = (d >> 3) ^ (2 * (r & 3));
        lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s*)(vl + r * ROW + cs * 16 + (d & 7) * 2));
      }
      {
        const int r = 32 * c + srow + 4;
        const int cs = (d >> 3) ^ (2 * (r & 3));
        hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s*)(vl + r * ROW + cs * 16 + (d & 7) * 2));
      }
      const v8s a8 = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a8), b, o[dt], 0, 0, 0);
    }
  }

  // partial results: O^T register i of lane (qi, qq) is d = wave D/4 + 16 dt + 4 qq + i, head qi
  if (qi < p.G) {
    const int64_t base = (int64_t(g) * p.nchunk_grid + chunk) * p.G + qi;
    float* po = p.part_o + base * D + wave * (D / 4) + 4 * qq;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<v4f*>(po + 16 * dt) = o[dt];
    if (wave == 0 && qq == 0) {
      const float L = ssum[qi] + ssum[16 + qi] + ssum[32 + qi] + ssum[48 + qi];
      p.part_ml[base * 2] = M;
      p.part_ml[base * 2 + 1] = L;
    }
  }
}

// Workgroups of 256 threads per (head, 64 output columns): M = max_c M_c, w_c = exp2((M_c - M) c),
// o = sum_c w_c o_c / sum_c w_c L_c.  The chunk statistics are read in parallel into LDS, the sums
// run in chunk order (deterministic); the two halves of the workgroup take alternate chunks of the
// output sum and are added in a fixed order.
constexpr int DEC_MAX_CHUNKS = 4096;
constexpr int DEC_MCOLS = 16;  // float4 output columns per merge workgroup

template <int D>
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(DecodeParams p) {
  __shared__ float wsh[DEC_MAX_CHUNKS];
  __shared__ float red[256];
  const int h = blockIdx.x, g = h / p.G, hl = h % p.G;
  const int t = threadIdx.x;
  const int nchunk = decode_geom<dec_chunk(D)>(p).nchunk;
  const float* ml = p.part_ml + (int64_t(g) * p.nchunk_grid * p.G + hl) * 2;  // chunk c at ml[c * G * 2]
  float mx = -__builtin_inff();
  for (int c = t; c < nchunk; c += 256) {
    const float m = ml[int64_t(c) * p.G * 2];
    wsh[c] = m;
    mx = fmaxf(mx, m);
  }
  red[t] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] = fmaxf(red[t], red[t + s]);
    __syncthreads();
  }
  const float M = red[0];
  __syncthreads();
  const float ms = M == -__builtin_inff() ? 0.0f : M * p.c;
  float lsum = 0.0f;
  for (int c = t; c < nchunk; c += 256) {
    const float w = __builtin_amdgcn_exp2f(__builtin_fmaf(wsh[c], p.c, -ms));
    wsh[c] = w;
    lsum = __builtin_fmaf(w, ml[int64_t(c) * p.G * 2 + 1], lsum);
  }
  red[t] = lsum;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] += red[t + s];
    __syncthreads();
  }
  const float L = red[0];
  // output columns: this workgroup's DEC_MCOLS float4 columns (blockIdx.y); thread t handles
  // column t % DEC_MCOLS of chunks t / DEC_MCOLS, + PARTS, ..., eight loads in flight at a time
  constexpr int COLS = DEC_MCOLS, PARTS = 256 / COLS;
  const int col = blockIdx.y * COLS + t % COLS, part = t / COLS;
  v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const float* po = p.part_o + (int64_t(g) * p.nchunk_grid * p.G + hl) * D + 4 * col;  // chunk c at po[c * G * D]
  for (int c0 = part; c0 < nchunk; c0 += 8 * PARTS) {
    v4f oc[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = c0 + u * PARTS;
      oc[u] = c < nchunk ? *reinterpret_cast<const v4f*>(po + int64_t(c) * p.G * D) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = c0 + u * PARTS;
      const float w = c < nchunk ? wsh[c] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(w, oc[u][i], acc[i]);
    }
  }
  // fold the PARTS partial sums in order 0, 1, ..
  __shared__ v4f parts[256];
  parts[t] = acc;
  __syncthreads();
  if (part != 0) return;
  for (int q = 1; q < PARTS; ++q) acc += parts[q * COLS + t % COLS];
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  v2u w2;
  w2[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  w2[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<v2u*>(p.o + int64_t(h) * p.ohs + 4 * col) = w2;
  if (p.lse && col == 0) p.lse[h] = L > 0.0f ? M * p.scale + __logf(L) : -__builtin_inff();
}

}  // namespace w8a8

using namespace w8a8;

static int attn_bn(int64_t D) { return D == 128 ? 128 : (D == 256 ? 64 : 32); }

// Bytes of one parked split part: attn_fwd2_kernel's (head_dim 512) or attn_fwd_kernel's.
static int64_t attn_part_bytes(int64_t D) {
  if (D == 512) return AttnFwd2Shape<512, 32, ATTN_FWD2_NW>::PART_BYTES;
  return int64_t(ATTN_NW) * 64 * (D / 16 + 1) * 16;
}

// Compute units of the current device (256 on MI355X), read once; the initialisation of a
// function-local static is thread-safe, so concurrent first calls from several host threads agree.
static int attn_cu_count() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

// ---- the causal work list ---------------------------------------------------------------------
//
// A causal call's query tiles differ in length (tile t sees the keys up to its last position), and
// a workgroup holds its CU alone (the kernel's LDS), so the split of long tiles and the launch
// order set the time.  The hardware hands workgroup i to XCD i % 8, there to the XCD's four
// shader engines (8 CUs each) in a fixed rotation, and there to the first CU that frees, in launch
// order: workgroup i waits in the queue of one of 32 engines (i % 32 on a 256-CU part) however
// idle the others are.  The plan splits each tile of n key blocks into k = ceil(n / L) parts (at
// most ATTN_MAX_SEG) for a target part length L and launches the items longest first (each
// engine's queue then runs longest-first too); it takes the L whose list finishes first on a
// model of that dispatch, in units of one key block: an item costs its blocks plus a fixed start
// and output cost, a split part the time to park its result, and a merge a fixed cost plus the
// time to read each part.  Measured per-block costs on the chip: ~3.3 us at head_dim 512 (32
// keys) and 256 (64 keys) with every CU busy.

// A split workspace starts with ATTN_COUNTER_BYTES of arrival counters at fixed offsets, whatever
// the plan: every call leaves its counters zero, and calls of different shapes share a workspace
// (one per stream), so no call's parked parts may overlap another plan's counters.
constexpr int64_t ATTN_COUNTER_BYTES = 65536;

struct AttnPlan {
  int ntiles = 0, per_group = 0, nseg = 1, nsplit_tiles = 0, nsplit_items = 0;
  int seg_tile[ATTN_MAX_SEG] = {}, seg_k[ATTN_MAX_SEG] = {}, seg_item[ATTN_MAX_SEG + 1] = {};
  int merge_mode = 0;           // 0: the last part merges in the kernel; 1: attn_merge_kernel after it
  std::vector<uint16_t> order;  // launch order of the items (empty: item order)
};

// Model constants fitted to per-workgroup timings of the full-attention layer (head_dim 512) at
// T = 3658 over seven part lengths, and of 256 queries at position 3402 over five.
constexpr double ATTN_ITEM_COST = 2.0;        // start (Q, first block in flight) and output, in blocks
constexpr double ATTN_PARK_COST = 1.5;        // parking a split part
constexpr double ATTN_MERGE_COST = 2.0;       // a merge: fixed part ...
constexpr double ATTN_MERGE_PART_COST = 0.5;  // ... and per part read

// Key blocks tile t of a causal call sees (keys 0 .. its last position).
static int attn_causal_blocks(int t, int PB, int BN, int64_t Tq, int64_t q_start) {
  const int64_t end = (int64_t(t) + 1) * PB < Tq ? (int64_t(t) + 1) * PB : Tq;
  return int((q_start + end - 1) / BN + 1);
}

// One-tile-per-workgroup list, longest tile first (sliding windows, calls without a workspace,
// calls the split does not speed up).
static void attn_plan_unsplit(AttnPlan& pl) {
  pl.per_group = pl.ntiles;
  pl.nseg = 1;
  pl.seg_tile[0] = pl.ntiles - 1;
  pl.seg_k[0] = 1;
  pl.seg_item[0] = 0;
  pl.seg_item[1] = pl.ntiles;
  pl.nsplit_tiles = pl.nsplit_items = 0;
  pl.merge_mode = 0;
  pl.order.clear();
}

// Segments of the list for target part length L (tiles from the longest down, k parts each).
static void attn_plan_segments(const std::vector<int>& nb, int L, AttnPlan& pl) {
  pl.nseg = 0;
  pl.nsplit_tiles = pl.nsplit_items = 0;
  int items = 0;
  for (int t = pl.ntiles - 1; t >= 0; --t) {
    int k = (nb[t] + L - 1) / L;
    k = k < 1 ? 1 : (k > ATTN_MAX_SEG ? ATTN_MAX_SEG : k);
    if (pl.nseg == 0 || pl.seg_k[pl.nseg - 1] != k) {
      pl.seg_tile[pl.nseg] = t;
      pl.seg_k[pl.nseg] = k;
      pl.seg_item[pl.nseg] = items;
      ++pl.nseg;
    }
    items += k;
    if (k > 1) {
      ++pl.nsplit_tiles;
      pl.nsplit_items += k;
    }
  }
  pl.seg_item[pl.nseg] = items;
  pl.per_group = items;
  pl.order.clear();
}

// Key blocks and modelled cost of every item, in item order.
static void attn_plan_items(const AttnPlan& pl, const std::vector<int>& nb, std::vector<int>& blocks,
                            std::vector<double>& cost) {
  blocks.resize(pl.per_group);
  cost.resize(pl.per_group);
  for (int s = 0; s < pl.nseg; ++s) {
    const int k = pl.seg_k[s];
    for (int item = pl.seg_item[s]; item < pl.seg_item[s + 1]; ++item) {
      const int off = item - pl.seg_item[s], t = pl.seg_tile[s] - off / k, part = off % k;
      blocks[item] = (part + 1) * nb[t] / k - part * nb[t] / k;
      double c = ATTN_ITEM_COST + blocks[item];
      if (k > 1) {
        c += ATTN_PARK_COST;
        if (pl.merge_mode == 0 && part == k - 1) c += ATTN_MERGE_COST + ATTN_MERGE_PART_COST * k;
      }
      cost[item] = c;
    }
  }
}

// The merge kernel of merge_mode 1, in block units: its launch, then the parked parts read once at
// the rate many CUs reach together (~5 TB/s, 16.5 MB per 3.3 us block).
constexpr double ATTN_MERGE_KERNEL_COST = 1.0;
constexpr double ATTN_MERGE_BYTES_PER_BLOCK = 16.5e6;
static double attn_merge_kernel_cost(const AttnPlan& pl, int64_t KV, int64_t D) {
  return ATTN_MERGE_KERNEL_COST + double(KV) * pl.nsplit_items * double(attn_part_bytes(D)) / ATTN_MERGE_BYTES_PER_BLOCK;
}

// Launch the items longest first (ties in item order), when the table fits the kernel arguments.
static void attn_plan_order(AttnPlan& pl, const std::vector<int>& blocks) {
  pl.order.clear();
  if (pl.per_group > ATTN_MAX_ORDER) return;
  pl.order.resize(pl.per_group);
  for (int i = 0; i < pl.per_group; ++i) pl.order[i] = uint16_t(i);
  std::stable_sort(pl.order.begin(), pl.order.end(), [&](uint16_t x, uint16_t y) { return blocks[x] > blocks[y]; });
}

// Modelled finishing time: workgroup w = j * KV + g (item order[j] of group g) joins the queue of
// engine w % (CUs / 8), whose 8 CUs take their queue's items in turn as they free.
static double attn_plan_makespan(const AttnPlan& pl, const std::vector<double>& cost, int KV, int cus) {
  const int ne = cus % 8 == 0 ? cus / 8 : 1, per_e = cus / ne;
  std::vector<std::priority_queue<double, std::vector<double>, std::greater<double>>> free_at(ne);
  for (auto& q : free_at)
    for (int c = 0; c < per_e; ++c) q.push(0.0);
  double end = 0.0;
  int64_t wg = 0;
  for (int j = 0; j < pl.per_group; ++j) {
    const double c = cost[pl.order.empty() ? j : pl.order[j]];
    for (int g = 0; g < KV; ++g, ++wg) {
      auto& q = free_at[wg % ne];
      const double t0 = q.top();
      q.pop();
      q.push(t0 + c);
      end = t0 + c > end ? t0 + c : end;
    }
  }
  return end;
}

static AttnPlan attn_plan_compute(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start,
                                  int64_t window) {
  AttnPlan pl;
  const int PB = int(ATTN_NW * 16 / (H / KV)), BN = attn_bn(D);
  pl.ntiles = int((Tq + PB - 1) / PB);
  attn_plan_unsplit(pl);
  if (pl.ntiles == 0) return pl;
  const int cus = attn_cu_count();
  std::vector<int> nb(pl.ntiles);
  int mx = 0;
  for (int t = 0; t < pl.ntiles; ++t) {
    if (window > 0) {  // the kernels' key range of a sliding-window tile
      const int64_t pmin = q_start + int64_t(t) * PB, pmax = q_start + std::min<int64_t>((int64_t(t) + 1) * PB, Tq) - 1;
      const int64_t khi = std::min<int64_t>(pmax, Tk - 1), klo = std::max<int64_t>(0, pmin - window + 1);
      const int64_t kb_first = klo / BN * BN;
      nb[t] = khi >= kb_first ? int((khi - kb_first) / BN + 1) : 0;
    } else {
      nb[t] = attn_causal_blocks(t, PB, BN, Tq, q_start);
    }
    mx = nb[t] > mx ? nb[t] : mx;
  }
  // the list would not fit the model's budget of simulated items: keep one item per tile
  if (mx < 2 || int64_t(pl.ntiles) * KV * ATTN_MAX_SEG > (int64_t(1) << 22)) return pl;
  std::vector<int> blocks;
  std::vector<double> cost;
  attn_plan_items(pl, nb, blocks, cost);
  const double unsplit = attn_plan_makespan(pl, cost, int(KV), cus);
  double best = 0.0;
  AttnPlan split;
  auto consider = [&](AttnPlan& c) {
    attn_plan_items(c, nb, blocks, cost);
    attn_plan_order(c, blocks);
    double ms = attn_plan_makespan(c, cost, int(KV), cus);
    if (c.merge_mode == 1) ms += attn_merge_kernel_cost(c, KV, D);
    if (split.ntiles == 0 || ms < best) {
      best = ms;
      split = c;
    }
  };
  if (window > 0) {
    // every tile's keys in the same number of parts k (a tile with fewer blocks parks empty parts),
    // merged by the merge kernel: taken where the tiles alone would leave most CUs idle
    if (KV * int64_t(pl.ntiles) < cus) {
      for (int k = 2; k <= ATTN_MAX_SEG && k <= mx; ++k) {
        AttnPlan c;
        c.ntiles = pl.ntiles;
        c.nseg = 1;
        c.seg_tile[0] = pl.ntiles - 1;
        c.seg_k[0] = k;
        c.seg_item[0] = 0;
        c.seg_item[1] = pl.ntiles * k;
        c.per_group = pl.ntiles * k;
        c.nsplit_tiles = pl.ntiles;
        c.nsplit_items = pl.ntiles * k;
        c.merge_mode = 1;
        consider(c);
      }
    }
  } else if (mx >= 8) {
    // part lengths from 4 blocks up to the longest tile, ~12% apart, with either merge
    int prev = 0;
    for (double Lf = 4.0; Lf < mx; Lf *= 1.125) {
      const int L = int(Lf);
      if (L == prev) continue;
      prev = L;
      for (int mode = 0; mode < 2; ++mode) {
        AttnPlan c;
        c.ntiles = pl.ntiles;
        attn_plan_segments(nb, L, c);
        if (mode == 0 && KV * c.nsplit_tiles * 4 > ATTN_COUNTER_BYTES) continue;  // one counter per split tile
        c.merge_mode = mode;
        consider(c);
      }
    }
  }
  // a split list is taken only when it beats one workgroup per tile by 2% on the model
  if (split.ntiles > 0 && split.nsplit_tiles > 0 && best < 0.98 * unsplit) pl = split;
  return pl;
}

// Plans are cached per call shape: the model runs once per (shape, position).
static AttnPlan attn_plan(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start, int64_t window) {
  static std::mutex mu;
  static std::map<std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t, int64_t>, AttnPlan> cache;
  const auto key = std::make_tuple(H, KV, Tq, D, q_start, window);
  {
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  const AttnPlan pl = attn_plan_compute(H, KV, Tq, Tk, D, q_start, window);
  std::lock_guard<std::mutex> g(mu);
  if (cache.size() >= 1024) cache.clear();
  cache.emplace(key, pl);
  return pl;
}

static int64_t attn_split_workspace(const AttnPlan& pl, int64_t KV, int64_t D) {
  if (pl.nsplit_tiles == 0) return 0;
  return ATTN_COUNTER_BYTES + KV * int64_t(pl.nsplit_items) * attn_part_bytes(D);
}

extern "C" int64_t w8a8_attention_workspace_bytes(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                                                  int64_t q_start, int64_t window) {
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 128 || (D != 128 && D != 256 && D != 512) || Tq < 0 ||
      q_start < 0 || window < 0 || Tk < q_start + Tq)
    return -1;
  return attn_split_workspace(attn_plan(H, KV, Tq, Tk, D, q_start, window), KV, D);
}

extern "C" int64_t w8a8_attention_plan_items(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                                             int64_t q_start, int64_t window, int* launch_order, int* merge_kernel) {
  if (w8a8_attention_workspace_bytes(H, KV, Tq, Tk, D, q_start, window) < 0) return -1;
  const AttnPlan pl = attn_plan(H, KV, Tq, Tk, D, q_start, window);
  if (launch_order) *launch_order = pl.order.empty() ? 0 : 1;
  if (merge_kernel) *merge_kernel = pl.nsplit_tiles > 0 ? pl.merge_mode : 0;
  return pl.per_group;
}

static int attention_launch(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* k,
                            int64_t k_head_stride, int64_t k_row_stride, const uint16_t* v, int64_t v_head_stride,
                            int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                            int64_t q_start, int64_t window, float scale, uint16_t* o, int64_t o_head_stride,
                            int64_t o_row_stride, float* lse, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream, int8_t* qpk = nullptr, float* qsx = nullptr) {
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 128)
    return fail(W8A8_EINVAL, "attention: H=%lld KV=%lld (H must be a multiple of KV, at most 128 heads per KV head)",
                (long long)H, (long long)KV);
  if (D != 128 && D != 256 && D != 512)
    return fail(W8A8_ENOTSUP, "attention: head_dim %lld (supported: 128, 256, 512)", (long long)D);
  if (Tq < 0 || q_start < 0 || window < 0 || Tk < q_start + Tq || Tk > INT32_MAX || H * KV > INT32_MAX)
    return fail(W8A8_EINVAL, "attention: Tq=%lld q_start=%lld Tk=%lld window=%lld (need Tk >= q_start + Tq)",
                (long long)Tq, (long long)q_start, (long long)Tk, (long long)window);
  if (!(scale > 0.0f) || scale == __builtin_inff()) return fail(W8A8_EINVAL, "attention: scale must be positive");
  if (Tq == 0) return W8A8_OK;
  if (!q || !k || !v || (!o && !qpk) || (qpk && !qsx)) return fail(W8A8_EINVAL, "attention: null pointer");
  if (q_row_stride < D || k_row_stride < D || v_row_stride < D || o_row_stride < 1 || o_head_stride < 1)
    return fail(W8A8_EINVAL, "attention: row strides smaller than head_dim");
  const int64_t strides[8] = {q_head_stride, q_row_stride, k_head_stride, k_row_stride,
                              v_head_stride, v_row_stride, o_head_stride, o_row_stride};
  for (int i = 0; i < 8; ++i)
    if (strides[i] % 8 != 0) return fail(W8A8_EALIGN, "attention: strides must be multiples of 8 elements");
  if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16 || (uintptr_t)o % 16)
    return fail(W8A8_EALIGN, "attention: q, k, v and o must be 16-byte aligned");
  const int64_t kb = ((Tk - 1) * k_row_stride + D) * 2, vb = ((Tk - 1) * v_row_stride + D) * 2;
  if (kb > INT32_MAX || vb > INT32_MAX) return fail(W8A8_ENOTSUP, "attention: one head's K or V above 2 GiB");
  AttnParams p;
  p.q = q; p.qhs = q_head_stride; p.qrs = q_row_stride;
  p.k = k; p.khs = k_head_stride; p.krs = k_row_stride;
  p.v = v; p.vhs = v_head_stride; p.vrs = v_row_stride;
  p.o = o; p.ohs = o_head_stride; p.ors = o_row_stride;
  p.lse = lse;
  p.k_bytes = uint32_t(kb); p.v_bytes = uint32_t(vb);
  p.H = int(H); p.KV = int(KV); p.G = int(H / KV); p.PB = ATTN_NW * 16 / p.G;
  p.Tq = int(Tq); p.Tk = int(Tk); p.q_start = int(q_start); p.window = int(window);
  AttnPlan pl = attn_plan(H, KV, Tq, Tk, D, q_start, window);
  p.part = nullptr;
  p.counters = nullptr;
  if (pl.nsplit_tiles > 0) {
    const int64_t need = attn_split_workspace(pl, KV, D);
    if (!workspace) {
      attn_plan_unsplit(pl);
    } else if (workspace_bytes < need) {
      return fail(W8A8_EINVAL, "attention: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                  (long long)need);
    } else if ((uintptr_t)workspace % 16) {
      return fail(W8A8_EALIGN, "attention: the workspace must be 16-byte aligned");
    } else {
      p.counters = static_cast<int*>(workspace);
      p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ATTN_COUNTER_BYTES);
    }
  }
  p.ntiles = pl.ntiles;
  p.per_group = pl.per_group;
  p.nseg = pl.nseg;
  p.nsplit_tiles = pl.nsplit_tiles;
  p.nsplit_items = pl.nsplit_items;
  for (int i = 0; i < ATTN_MAX_SEG; ++i) {
    p.seg_tile[i] = pl.seg_tile[i];
    p.seg_k[i] = pl.seg_k[i];
  }
  for (int i = 0; i <= ATTN_MAX_SEG; ++i) p.seg_item[i] = pl.seg_item[i];
  p.merge_mode = pl.nsplit_tiles > 0 ? pl.merge_mode : 0;
  p.ordered = pl.order.empty() ? 0 : 1;
  for (size_t i = 0; i < pl.order.size(); ++i) p.order[i] = pl.order[i];
  p.scale = scale; p.c = scale * 1.4426950408889634f;
  p.qpk = qpk;
  p.qsx = qsx;
  p.qKF = int(2 * ((H * D + 63) / 64));
  p.qMp = int((Tq + 31) / 32 * 32);
  if (qpk && p.nsplit_tiles > 0 && p.merge_mode == 1)
    return fail(W8A8_ENOTSUP, "attention_quant: this call merges its key parts in a second kernel, which does not "
                              "hold whole token rows");
  const int64_t nwg = KV * int64_t(p.per_group);
  if (nwg > INT32_MAX) return fail(W8A8_ENOTSUP, "attention: too many query tiles");
  const dim3 grid{unsigned(nwg), 1, 1};
  if (D == 128)
    attn_fwd_kernel<128, 128, ATTN_NW><<<grid, dim3{ATTN_NW * 64, 1, 1}, 0, stream>>>(p);
  else if (D == 256)
    attn_fwd_kernel<256, 64, ATTN_NW><<<grid, dim3{ATTN_NW * 64, 1, 1}, 0, stream>>>(p);
  else
    attn_fwd2_kernel<512, 32, ATTN_FWD2_NW><<<grid, dim3{ATTN_FWD2_NW * 64, 1, 1}, 0, stream>>>(p);
  int rc = check_launch("attention_bf16");
  if (rc || !p.merge_mode) return rc;
  // one workgroup per (KV group, split tile, parked O^T slot)
  const int nslot = D == 512 ? AttnFwd2Shape<512, 32, ATTN_FWD2_NW>::SLOTS : int(D / 16);
  const dim3 mgrid{unsigned(KV * int64_t(p.nsplit_tiles) * nslot), 1, 1};
  if (D == 128)
    attn_merge_kernel<128, false><<<mgrid, dim3{512, 1, 1}, 0, stream>>>(p);
  else if (D == 256)
    attn_merge_kernel<256, false><<<mgrid, dim3{512, 1, 1}, 0, stream>>>(p);
  else
    attn_merge_kernel<512, true><<<mgrid, dim3{512, 1, 1}, 0, stream>>>(p);
  return check_launch("attention_merge");
}

extern "C" int w8a8_attention_bf16(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* k,
                                   int64_t k_head_stride, int64_t k_row_stride, const uint16_t* v,
                                   int64_t v_head_stride, int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tq,
                                   int64_t Tk, int64_t D, int64_t q_start, int64_t window, float scale, uint16_t* o,
                                   int64_t o_head_stride, int64_t o_row_stride, float* lse, hipStream_t stream) {
  return attention_launch(q, q_head_stride, q_row_stride, k, k_head_stride, k_row_stride, v, v_head_stride,
                          v_row_stride, H, KV, Tq, Tk, D, q_start, window, scale, o, o_head_stride, o_row_stride, lse,
                          nullptr, 0, stream);
}

extern "C" int w8a8_attention_ws_bf16(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride,
                                      const uint16_t* k, int64_t k_head_stride, int64_t k_row_stride, const uint16_t* v,
                                      int64_t v_head_stride, int64_t v_row_stride, int64_t H, int64_t KV, int64_t Tq,
                                      int64_t Tk, int64_t D, int64_t q_start, int64_t window, float scale, uint16_t* o,
                                      int64_t o_head_stride, int64_t o_row_stride, float* lse, void* workspace,
                                      int64_t workspace_bytes, hipStream_t stream) {
  return attention_launch(q, q_head_stride, q_row_stride, k, k_head_stride, k_row_stride, v, v_head_stride,
                          v_row_stride, H, KV, Tq, Tk, D, q_start, window, scale, o, o_head_stride, o_row_stride, lse,
                          workspace, workspace_bytes, stream);
}

// The attention output quantised per token in the same launch (k_attn_out, pipeline.py:88-92): one
// KV group (every head of a token in one workgroup), at most 16 heads, a power of two; and a plan
// that merges split key parts in the kernel.
static bool attention_quant_fits(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start,
                                 int64_t window) {
  if (KV != 1 || H < 1 || H > 16 || (H & (H - 1)) != 0) return false;
  if (w8a8_attention_workspace_bytes(H, KV, Tq, Tk, D, q_start, window) < 0) return false;
  const AttnPlan pl = attn_plan(H, KV, Tq, Tk, D, q_start, window);
  return !(pl.nsplit_tiles > 0 && pl.merge_mode == 1);
}

extern "C" int w8a8_attention_quant_supported(int64_t H, int64_t KV, int64_t Tq, int64_t Tk, int64_t D,
                                              int64_t q_start, int64_t window) {
  return attention_quant_fits(H, KV, Tq, Tk, D, q_start, window) ? 1 : 0;
}

extern "C" int w8a8_attention_quant_bf16(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride,
                                         const uint16_t* k, int64_t k_head_stride, int64_t k_row_stride,
                                         const uint16_t* v, int64_t v_head_stride, int64_t v_row_stride, int64_t H,
                                         int64_t KV, int64_t Tq, int64_t Tk, int64_t D, int64_t q_start,
                                         int64_t window, float scale, int8_t* packed, float* sx, void* workspace,
                                         int64_t workspace_bytes, hipStream_t stream) {
  if (Tq > 0 && !attention_quant_fits(H, KV, Tq, Tk, D, q_start, window))
    return fail(W8A8_ENOTSUP, "attention_quant: H=%lld KV=%lld Tq=%lld q_start=%lld window=%lld: needs one KV group of "
                              "at most 16 heads (a power of two) and a plan without a separate merge",
                (long long)H, (long long)KV, (long long)Tq, (long long)q_start, (long long)window);
  if ((uintptr_t)packed % 16) return fail(W8A8_EALIGN, "attention_quant: the packed rows must be 16-byte aligned");
  if ((Tq + 31) / 32 * 2 * ((H * D + 63) / 64) * 1024 > INT32_MAX)
    return fail(W8A8_ENOTSUP, "attention_quant: packed output above 2 GiB");
  return attention_launch(q, q_head_stride, q_row_stride, k, k_head_stride, k_row_stride, v, v_head_stride,
                          v_row_stride, H, KV, Tq, Tk, D, q_start, window, scale, nullptr, 8, 8, nullptr, workspace,
                          workspace_bytes, stream, packed, sx);
}

// The split and merge launches of one decode call: nchunk_grid chunks per KV head, partials in the
// workspace (nchunk_grid per KV head and query head).
// The split kernel, then (merge) the merge kernel.  The chunk partials sit at the start of the
// workspace: part_o [KV][nchunk_grid][G][D] fp32, then part_ml [KV][nchunk_grid][G][2].
static void decode_launch(DecodeParams& p, int64_t D, void* workspace, hipStream_t stream, bool merge = true) {
  p.part_o = static_cast<float*>(workspace);
  p.part_ml = p.part_o + int64_t(p.KV) * p.nchunk_grid * p.G * D;
  const dim3 grid{unsigned(p.KV * p.nchunk_grid), 1, 1};
  const dim3 mgrid{unsigned(p.H), unsigned(D / 4 / DEC_MCOLS), 1};
  if (D == 128) {
    attn_decode_split_kernel<128><<<grid, dim3{256, 1, 1}, 0, stream>>>(p);
    if (merge) attn_decode_merge_kernel<128><<<mgrid, dim3{256, 1, 1}, 0, stream>>>(p);
  } else if (D == 256) {
    attn_decode_split_kernel<256><<<grid, dim3{256, 1, 1}, 0, stream>>>(p);
    if (merge) attn_decode_merge_kernel<256><<<mgrid, dim3{256, 1, 1}, 0, stream>>>(p);
  } else {
    attn_decode_split_kernel<512><<<grid, dim3{256, 1, 1}, 0, stream>>>(p);
    if (merge) attn_decode_merge_kernel<512><<<mgrid, dim3{256, 1, 1}, 0, stream>>>(p);
  }
}

static void decode_geometry(int64_t D, int64_t q_pos, int64_t window, int& klo, int& nchunk) {
  klo = window > 0 ? int(q_pos - window + 1 > 0 ? q_pos - window + 1 : 0) : 0;
  nchunk = int((q_pos - klo) / dec_chunk(int(D)) + 1);
}

extern "C" int64_t w8a8_attention_decode_workspace_bytes(int64_t H, int64_t KV, int64_t Tk, int64_t D, int64_t q_pos,
                                                         int64_t window) {
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 16 || (D != 128 && D != 256 && D != 512) || Tk < 1 || q_pos < 0 ||
      q_pos >= Tk || window < 0)
    return -1;
  int klo, nchunk;
  decode_geometry(D, q_pos, window, klo, nchunk);
  return int64_t(KV) * nchunk * (H / KV) * (D + 2) * 4;
}

extern "C" int w8a8_attention_decode_bf16(const uint16_t* q, int64_t q_head_stride, const uint16_t* k,
                                          int64_t k_head_stride, int64_t k_row_stride, const uint16_t* v,
                                          int64_t v_head_stride, int64_t v_row_stride, int64_t H, int64_t KV,
                                          int64_t Tk, int64_t D, int64_t q_pos, int64_t window, float scale,
                                          uint16_t* o, int64_t o_head_stride, float* lse, void* workspace,
                                          int64_t workspace_bytes, hipStream_t stream) {
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 16)
    return fail(W8A8_EINVAL, "attention_decode: H=%lld KV=%lld (H must be a multiple of KV, at most 16 heads per KV head)",
                (long long)H, (long long)KV);
  if (D != 128 && D != 256 && D != 512)
    return fail(W8A8_ENOTSUP, "attention_decode: head_dim %lld (supported: 128, 256, 512)", (long long)D);
  if (Tk < 1 || Tk > INT32_MAX || q_pos < 0 || q_pos >= Tk || window < 0)
    return fail(W8A8_EINVAL, "attention_decode: Tk=%lld q_pos=%lld window=%lld (need 0 <= q_pos < Tk)", (long long)Tk,
                (long long)q_pos, (long long)window);
  {
    int klo, nchunk;
    decode_geometry(D, q_pos, window, klo, nchunk);
    if (nchunk > DEC_MAX_CHUNKS)
      return fail(W8A8_ENOTSUP, "attention_decode: %d key chunks of %d (at most %d)", nchunk, dec_chunk(int(D)),
                  DEC_MAX_CHUNKS);
  }
  if (!(scale > 0.0f) || scale == __builtin_inff()) return fail(W8A8_EINVAL, "attention_decode: scale must be positive");
  if (!q || !k || !v || !o || !workspace) return fail(W8A8_EINVAL, "attention_decode: null pointer");
  const int64_t need = w8a8_attention_decode_workspace_bytes(H, KV, Tk, D, q_pos, window);
  if (workspace_bytes < need)
    return fail(W8A8_EINVAL, "attention_decode: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                (long long)need);
  if (k_row_stride < D || v_row_stride < D || (H > 1 && (q_head_stride < D || o_head_stride < D)))
    return fail(W8A8_EINVAL, "attention_decode: strides smaller than head_dim");
  const int64_t strides[6] = {q_head_stride, k_head_stride, k_row_stride, v_head_stride, v_row_stride, o_head_stride};
  for (int i = 0; i < 6; ++i)
    if (strides[i] % 8 != 0) return fail(W8A8_EALIGN, "attention_decode: strides must be multiples of 8 elements");
  if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16 || (uintptr_t)o % 16 || (uintptr_t)workspace % 16)
    return fail(W8A8_EALIGN, "attention_decode: q, k, v, o and the workspace must be 16-byte aligned");
  const int64_t kb = ((Tk - 1) * k_row_stride + D) * 2, vb = ((Tk - 1) * v_row_stride + D) * 2;
  if (kb > INT32_MAX || vb > INT32_MAX) return fail(W8A8_ENOTSUP, "attention_decode: one head's K or V above 2 GiB");
  DecodeParams p{};
  p.q = q; p.qhs = q_head_stride; p.k = k; p.khs = k_head_stride; p.krs = k_row_stride;
  p.v = v; p.vhs = v_head_stride; p.vrs = v_row_stride; p.o = o; p.ohs = o_head_stride; p.lse = lse;
  p.k_bytes = uint32_t(kb); p.v_bytes = uint32_t(vb);
  p.H = int(H); p.KV = int(KV); p.G = int(H / KV); p.Tk = int(Tk); p.pos = int(q_pos);
  decode_geometry(D, q_pos, window, p.klo, p.nchunk);
  p.pos_dev = nullptr;
  p.window = int(window);
  p.nchunk_grid = p.nchunk;
  p.scale = scale; p.c = scale * 1.4426950408889634f;
  decode_launch(p, D, workspace, stream);
  return check_launch("attention_decode_bf16");
}

// Chunks per KV head the device-position launch holds: enough for every position below Tk.

extern "C" int64_t w8a8_attention_decode_dev_workspace_bytes(int64_t H, int64_t KV, int64_t Tk, int64_t D,
                                                             int64_t window) {
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 16 || (D != 128 && D != 256 && D != 512) || Tk < 1 ||
      Tk > INT32_MAX || window < 0)
    return -1;
  return int64_t(KV) * decode_grid_chunks(D, Tk, window) * (H / KV) * (D + 2) * 4;
}

extern "C" int w8a8_attention_decode_dev_bf16(const uint16_t* q, int64_t q_head_stride, const uint16_t* k,
                                              int64_t k_head_stride, int64_t k_row_stride, const uint16_t* v,
                                              int64_t v_head_stride, int64_t v_row_stride, int64_t H, int64_t KV,
                                              int64_t Tk, int64_t D, const int32_t* q_pos, int64_t window, float scale,
                                              uint16_t* o, int64_t o_head_stride, void* workspace,
                                              int64_t workspace_bytes, hipStream_t stream) {
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 16)
    return fail(W8A8_EINVAL, "attention_decode_dev: H=%lld KV=%lld (H must be a multiple of KV, at most 16 heads per "
                "KV head)", (long long)H, (long long)KV);
  if (D != 128 && D != 256 && D != 512)
    return fail(W8A8_ENOTSUP, "attention_decode_dev: head_dim %lld (supported: 128, 256, 512)", (long long)D);
  if (Tk < 1 || Tk > INT32_MAX || window < 0 || window > INT32_MAX)
    return fail(W8A8_EINVAL, "attention_decode_dev: Tk=%lld window=%lld", (long long)Tk, (long long)window);
  if (decode_grid_chunks(D, Tk, window) > DEC_MAX_CHUNKS)
    return fail(W8A8_ENOTSUP, "attention_decode_dev: %d key chunks of %d (at most %d)", decode_grid_chunks(D, Tk, window),
                dec_chunk(int(D)), DEC_MAX_CHUNKS);
  if (!(scale > 0.0f) || scale == __builtin_inff())
    return fail(W8A8_EINVAL, "attention_decode_dev: scale must be positive");
  if (!q || !k || !v || !o || !q_pos || !workspace) return fail(W8A8_EINVAL, "attention_decode_dev: null pointer");
  const int64_t need = w8a8_attention_decode_dev_workspace_bytes(H, KV, Tk, D, window);
  if (workspace_bytes < need)
    return fail(W8A8_EINVAL, "attention_decode_dev: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                (long long)need);
  if (k_row_stride < D || v_row_stride < D || (H > 1 && (q_head_stride < D || o_head_stride < D)))
    return fail(W8A8_EINVAL, "attention_decode_dev: strides smaller than head_dim");
  const int64_t strides[6] = {q_head_stride, k_head_stride, k_row_stride, v_head_stride, v_row_stride, o_head_stride};
  for (int i = 0; i < 6; ++i)
    if (strides[i] % 8 != 0) return fail(W8A8_EALIGN, "attention_decode_dev: strides must be multiples of 8 elements");
  if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16 || (uintptr_t)o % 16 || (uintptr_t)workspace % 16 ||
      (uintptr_t)q_pos % 4)
    return fail(W8A8_EALIGN, "attention_decode_dev: q, k, v, o and the workspace 16-byte, q_pos 4-byte aligned");
  const int64_t kb = ((Tk - 1) * k_row_stride + D) * 2, vb = ((Tk - 1) * v_row_stride + D) * 2;
  if (kb > INT32_MAX || vb > INT32_MAX) return fail(W8A8_ENOTSUP, "attention_decode_dev: one head's K or V above 2 GiB");
  DecodeParams p{};
  p.q = q; p.qhs = q_head_stride; p.k = k; p.khs = k_head_stride; p.krs = k_row_stride;
  p.v = v; p.vhs = v_head_stride; p.vrs = v_row_stride; p.o = o; p.ohs = o_head_stride; p.lse = nullptr;
  p.k_bytes = uint32_t(kb); p.v_bytes = uint32_t(vb);
  p.H = int(H); p.KV = int(KV); p.G = int(H / KV); p.Tk = int(Tk);
  p.pos_dev = q_pos;
  p.window = int(window);
  p.nchunk_grid = decode_grid_chunks(D, Tk, window);
  p.scale = scale; p.c = scale * 1.4426950408889634f;
  decode_launch(p, D, workspace, stream);
  return check_launch("attention_decode_dev_bf16");
}

extern "C" int w8a8_attention_decode_qkv_dev_bf16(const uint16_t* y, const uint16_t* cos_, const uint16_t* sin_,
                                                  int64_t rope_rows, const uint16_t* qw, const uint16_t* kw, float eps,
                                                  uint16_t* k,
                                                  int64_t k_head_stride, int64_t k_row_stride, uint16_t* v,
                                                  int64_t v_head_stride, int64_t v_row_stride, int64_t H, int64_t KV,
                                                  int64_t Tk, int64_t D, int kv_write, const int32_t* q_pos,
                                                  int64_t window, float scale, uint16_t* o, int64_t o_head_stride,
                                                  void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  const char* what = "attention_decode_qkv_dev";
  if (H < 1 || KV < 1 || H % KV != 0 || H / KV > 8)
    return fail(W8A8_EINVAL, "%s: H=%lld KV=%lld (H must be a multiple of KV, at most 8 heads per KV head)", what,
                (long long)H, (long long)KV);
  if (D != 128 && D != 256 && D != 512)
    return fail(W8A8_ENOTSUP, "%s: head_dim %lld (supported: 128, 256, 512)", what, (long long)D);
  if (Tk < 1 || Tk > INT32_MAX || window < 0 || window > INT32_MAX)
    return fail(W8A8_EINVAL, "%s: Tk=%lld window=%lld", what, (long long)Tk, (long long)window);
  if (decode_grid_chunks(D, Tk, window) > DEC_MAX_CHUNKS)
    return fail(W8A8_ENOTSUP, "%s: %d key chunks of %d (at most %d)", what, decode_grid_chunks(D, Tk, window),
                dec_chunk(int(D)), DEC_MAX_CHUNKS);
  if (!(scale > 0.0f) || scale == __builtin_inff()) return fail(W8A8_EINVAL, "%s: scale must be positive", what);
  if (!y || !cos_ || !sin_ || !k || !v || !q_pos || !workspace) return fail(W8A8_EINVAL, "%s: null pointer", what);
  if (rope_rows < 1 || rope_rows * D * 2 > INT32_MAX) return fail(W8A8_EINVAL, "%s: rope_rows=%lld", what, (long long)rope_rows);
  if (!o && decode_grid_chunks(D, Tk, window) > DEC_MERGE_IN_GEMV_CHUNKS)
    return fail(W8A8_ENOTSUP, "%s: without o the chunks (%d) are merged by w8a8_gemv_packed_attn_merge_bf16, which "
                "takes at most %d", what, decode_grid_chunks(D, Tk, window), DEC_MERGE_IN_GEMV_CHUNKS);
  const int64_t need = w8a8_attention_decode_dev_workspace_bytes(H, KV, Tk, D, window);
  if (workspace_bytes < need)
    return fail(W8A8_EINVAL, "%s: workspace of %lld bytes, %lld needed", what, (long long)workspace_bytes,
                (long long)need);
  if (k_row_stride < D || v_row_stride < D || (H > 1 && o_head_stride < D))
    return fail(W8A8_EINVAL, "%s: strides smaller than head_dim", what);
  const int64_t strides[5] = {k_head_stride, k_row_stride, v_head_stride, v_row_stride, o_head_stride};
  for (int i = 0; i < 5; ++i)
    if (strides[i] % 8 != 0) return fail(W8A8_EALIGN, "%s: strides must be multiples of 8 elements", what);
  for (const void* q : {static_cast<const void*>(y), static_cast<const void*>(cos_), static_cast<const void*>(sin_),
                        static_cast<const void*>(qw), static_cast<const void*>(kw), static_cast<const void*>(k),
                        static_cast<const void*>(v), static_cast<const void*>(o), static_cast<const void*>(workspace)})
    if (reinterpret_cast<uintptr_t>(q) % 16) return fail(W8A8_EALIGN, "%s: pointers must be 16-byte aligned", what);
  if ((uintptr_t)q_pos % 4) return fail(W8A8_EALIGN, "%s: q_pos must be 4-byte aligned", what);
  const int64_t kb = ((Tk - 1) * k_row_stride + D) * 2, vb = ((Tk - 1) * v_row_stride + D) * 2;
  if (kb > INT32_MAX || vb > INT32_MAX) return fail(W8A8_ENOTSUP, "%s: one head's K or V above 2 GiB", what);
  DecodeParams p{};
  p.q = nullptr; p.qhs = D; p.k = k; p.khs = k_head_stride; p.krs = k_row_stride;
  p.v = v; p.vhs = v_head_stride; p.vrs = v_row_stride; p.o = o; p.ohs = o_head_stride; p.lse = nullptr;
  p.k_bytes = uint32_t(kb); p.v_bytes = uint32_t(vb);
  p.H = int(H); p.KV = int(KV); p.G = int(H / KV); p.Tk = int(Tk);
  p.pos_dev = q_pos;
  p.window = int(window);
  p.nchunk_grid = decode_grid_chunks(D, Tk, window);
  p.scale = scale; p.c = scale * 1.4426950408889634f;
  p.qkv_y = y; p.rope_c = cos_; p.rope_s = sin_; p.qw = qw; p.kw = kw; p.qkv_eps = eps; p.kv_write = kv_write ? 1 : 0;
  p.qkv_bytes = uint32_t((H + (kv_write ? 2 * KV : 0)) * D * 2);
  p.rope_rows = int(rope_rows);
  decode_launch(p, D, workspace, stream, o != nullptr);
  return check_launch("attention_decode_qkv_dev_bf16");
}
