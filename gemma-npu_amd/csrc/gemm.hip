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

__device__ __forceinline__ float gelu_tanh_f32(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), the approximate="tanh" form.
  const float kBeta = 0.7978845608028654f;
  const float kKappa = 0.044715f;
  const float inner = kBeta * (x + kKappa * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in bits
// [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Buffer cache policy sc0 | sc1: system scope, coherent across the XCDs' caches.
static constexpr int kSysCoherent = 0x11;

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Logical tile of block b: each of the 8 XCDs gets a contiguous run.
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
  const int full = nblocks & ~7;
  if (b >= full) return b;
  const int per = full >> 3;
  return (b & 7) * per + (b >> 3);
}

// Epilogue for one 32x32 accumulator tile.  Lane l holds row m and, for register group
// g = 0..3, packed columns t*32 + 8g + lcol + r (r = 0..3, lcol = 4*(l/32)).
template <int EPI>
__device__ __forceinline__ void store_tile(const GemmParams& p, const v16i& acc, const v16i* acc_up, int m, int t,
                                           int lcol) {
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
    const float sxm = p.sx[m];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = t * 32 + 8 * g + lcol;
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float swn = (n + r < p.N) ? p.sw[n + r] : 0.0f;
        y[r] = bf16_to_f32(f32_to_bf16((float(acc[4 * g + r]) * sxm) * swn));
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
    // t is an even (gate) tile u = t/2; acc_up is the matching up tile t+1.
    const float sxm = p.sx[m];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = (t >> 1) * 32 + 8 * g + lcol;  // logical gate column
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = c + r < p.I;
        const float swg = ok ? p.sw[c + r] : 0.0f;
        const float swu = ok ? p.sw[p.I + c + r] : 0.0f;
        const float gate = bf16_to_f32(f32_to_bf16((float(acc[4 * g + r]) * sxm) * swg));
        const float up = bf16_to_f32(f32_to_bf16((float((*acc_up)[4 * g + r]) * sxm) * swu));
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

template <int BM, int BN, int WGM, int WGN, int NS, int EPI, bool A_PACKED, bool SPLIT, int MINB>
__global__ __launch_bounds__(WGM * WGN * 64, MINB) void gemm_kernel(GemmParams p) {
  constexpr int NW = WGM * WGN;
  constexpr int MT = BM / 32;         // A row-tiles per block
  constexpr int NTB = BN / 32;        // W column-tiles per block
  constexpr int F = 2 * (MT + NTB);   // fragments per k-tile of 64 (one ring slot)
  static_assert((2 * MT) % NW == 0 && (2 * NTB) % NW == 0, "each wave moves whole A and W fragments");
  constexpr int FA = 2 * MT / NW, FB = 2 * NTB / NW;  // fragments per wave per k-tile
  constexpr int WTM = MT / WGM;       // 32-row tiles per wave
  constexpr int WTN = NTB / WGN;      // 32-column tiles per wave
  static_assert(WTM * WGM == MT && WTN * WGN == NTB, "wave grid must divide the block tile");
  static_assert(EPI != EPI_GELU || (WTN % 2 == 0), "GELU pairs need an even tile count per wave");
  static_assert(NS >= 3, "the ring needs three slots: one read, one landing, one in flight");
  constexpr int NQ = WTM * WTN;                   // MFMAs per k-step
  constexpr int EARLY = NQ >= 8 ? NQ / 4 : 1;     // MFMAs issued before the next fragment reads

  // Slot layout: A fragments (s, mt) at (s*MT + mt) KiB, then W fragments (s, nt) at
  // (2*MT + s*NTB + nt) KiB, s = 0, 1 the two 32-wide k-steps of the k-tile.
  __shared__ __attribute__((aligned(1024))) char lds[NS][F * 1024];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT + NTB - 1) / NTB;
  // With split-K, the p.splits blocks of one output tile are consecutive logical blocks and
  // each multiplies k-tiles [k_lo, k_hi).
  const int lb = xcd_remap(blockIdx.x, ntm * ntn * p.splits);
  const int tile = lb / p.splits;
  const int split = lb % p.splits;
  int tm, tn;
  tile_coords(tile, ntm, ntn, p.gm, tm, tn);
  const int m0 = tm * BM;
  const int t0 = tn * NTB;
  const int k_lo = split * p.kt_per_split;
  const int k_hi = min(p.KF >> 1, k_lo + p.kt_per_split);

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.wp, p.w_bytes);

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
  constexpr uint32_t A_STEP = A_PACKED ? 2048u : 64u;  // bytes per k-tile

  auto issue = [&](int kt) {
    char* slot = lds[kt % NS];
#pragma unroll
    for (int i = 0; i < FA; ++i) dma16(ra, slot + (i * NW + wave) * 1024, offa[i] + uint32_t(kt) * A_STEP);
#pragma unroll
    for (int i = 0; i < FB; ++i) dma16(rw, slot + (2 * MT + i * NW + wave) * 1024, offb[i] + uint32_t(kt) * 2048u);
  };
  // This wave's operand fragments of k-step s of k-tile kt.
  auto read = [&](int kt, int s, v4i (&a)[WTM], v4i (&b)[WTN]) {
    const char* slot = lds[kt % NS];
#pragma unroll
    for (int j = 0; j < WTN; ++j)
      b[j] = *reinterpret_cast<const v4i*>(slot + (2 * MT + s * NTB + wn * WTN + j) * 1024 + lane * 16);
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

  // Pipeline.  DMA runs NS-1 k-tiles ahead of the multiply.  Fragments are read from LDS one
  // k-step ahead of their MFMAs, and the reads that refill a register set are issued only
  // after EARLY MFMAs of the other set, so they never wait on MFMAs still reading the set
  // they overwrite; sched_barrier keeps the compiler from reordering the phases.  The barrier
  // that publishes the next k-tile sits in the middle of the current one.
  const int KT = k_hi - k_lo;  // k-tiles of 64 this block multiplies
  auto issue_local = [&](int t) { issue(k_lo + t); };
  auto read_local = [&](int t, int s, v4i (&a)[WTM], v4i (&b)[WTN]) { read(k_lo + t, s, a, b); };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < KT) issue_local(s);
  if (NS - 2 < KT)
    wait_vmcnt<(FA + FB) * (NS - 2)>();
  else
    wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();

  v4i a0[WTM], b0[WTN], a1[WTM], b1[WTN];
  if (KT > 0) read_local(0, 0, a0, b0);
  for (int kt = 0; kt < KT; ++kt) {
    mma(a0, b0, 0, EARLY);
    __builtin_amdgcn_sched_barrier(0);
    read_local(kt, 1, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    mma(a0, b0, EARLY, NQ);
    mma(a1, b1, 0, EARLY);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < KT) {
      // k-tile kt+1 has landed once at most the NS-3 k-tiles issued after it are in flight.
      if (kt + NS - 2 < KT)
        wait_vmcnt<(FA + FB) * (NS - 3)>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      // Every wave has consumed k-tile kt-1 (its MFMAs waited on those reads), so its slot,
      // (kt-1) % NS = (kt+NS-1) % NS, can be refilled.
      if (kt + NS - 1 < KT) issue_local(kt + NS - 1);
      read_local(kt + 1, 0, a0, b0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma(a1, b1, EARLY, NQ);
  }

  // ---- split-K: park partial sums; the last block of the tile adds them up -------------------
  // The XCDs' L2 caches are not coherent with each other, so the partials go through with
  // system-scope (sc0 sc1) buffer stores and loads, which are coherent by themselves, and the
  // arrival count is a system-scope atomic.  Each thread's stores are complete (vmcnt 0)
  // before the barrier that precedes the count, so a block that sees itself last reads every
  // other block's finished partials.  No cache-wide writeback or invalidate is needed.
  if constexpr (SPLIT) {
    constexpr uint32_t kPartialBytes = uint32_t(NW) * NQ * 64 * 64;  // one split's tile, lane-native
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.ws + size_t(tile) * p.splits * (kPartialBytes / 4),
                                                uint32_t(p.splits) * kPartialBytes);
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t off =
              uint32_t(split) * kPartialBytes + ((wave * NQ + i * WTN + j) * 64 + lane) * 64 + g * 16;
          const v4u v = {uint32_t(acc[i][j][4 * g]), uint32_t(acc[i][j][4 * g + 1]), uint32_t(acc[i][j][4 * g + 2]),
                         uint32_t(acc[i][j][4 * g + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, rp, off, 0, kSysCoherent);
        }
    __builtin_amdgcn_s_waitcnt(0);
    // The ring is idle now (every wave's reads completed before its last MFMAs), so its first
    // word carries the arrival count to the whole block.
    int* arrived = reinterpret_cast<int*>(&lds[0][0]);
    __syncthreads();
    if (threadIdx.x == 0)
      *arrived = __hip_atomic_fetch_add(p.counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    if (*arrived != p.splits - 1) return;
    for (int o = 0; o < p.splits; ++o) {
      if (o == split) continue;
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const uint32_t off = uint32_t(o) * kPartialBytes + ((wave * NQ + i * WTN + j) * 64 + lane) * 64 + g * 16;
            const v4i v = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, kSysCoherent));
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][4 * g + r] += v[r];
          }
    }
    if (threadIdx.x == 0) __hip_atomic_store(p.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }

  // ---- epilogue ---------------------------------------------------------------------------
  const int lrow = lane & 31;
  const int lcol = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < WTM; ++i) {
    const int m = m0 + (wm * WTM + i) * 32 + lrow;
    if (m >= p.M) continue;
    if constexpr (EPI == EPI_GELU) {
#pragma unroll
      for (int j = 0; j < WTN; j += 2) store_tile<EPI>(p, acc[i][j], &acc[i][j + 1], m, t0 + wn * WTN + j, lcol);
    } else {
#pragma unroll
      for (int j = 0; j < WTN; ++j) store_tile<EPI>(p, acc[i][j], nullptr, m, t0 + wn * WTN + j, lcol);
    }
  }
}

// ---- host-side launch ----------------------------------------------------------------------

static const int kBM[8] = {256, 256, 128, 256, 128, 128, 256, 128};
static constexpr int64_t kCounterBytes = 4096;
static const int kBN[8] = {256, 256, 256, 128, 128, 128, 128, 256};

// Split-K: blocks per output tile so the grid covers the 256 CUs when there are few tiles.
// Every split keeps at least 4 k-tiles of 64; `kps` is the number of k-tiles per split.
// Measured on MI355X the partial-sum exchange costs more than the extra CUs gain on the E2B
// shapes, so automatic selection keeps K whole (kAutoSplit = false); the machinery stays
// available behind the workspace argument.
static constexpr bool kAutoSplit = false;
// req: 0 = automatic, n >= 1 = at most n splits.
static int pick_splits(int tiles, int KT, int req, int& kps) {
  int s = 1;
  if (tiles < 200 && (req > 1 || (req == 0 && kAutoSplit))) s = 256 / tiles;  // and so tiles < kCounterBytes / 4
  if (req > 0) s = min(s, req);
  s = max(1, min(s, min(8, KT / 4)));
  kps = (KT + s - 1) / s;
  return (KT + kps - 1) / kps;
}

// Split-K workspace: kCounterBytes of arrival counters (one int per output tile; zero before
// and after every call) followed by the partial sums (scratch).
int64_t gemm_workspace_bytes(int M, int NP, int KF, int cfg, int split_k) {
  if (cfg <= 1) return 0;  // the 256x256 tiles run without split-K
  const int ntm = (M + kBM[cfg] - 1) / kBM[cfg], ntn = (NP + kBN[cfg] - 1) / kBN[cfg];
  int kps;
  const int s = pick_splits(ntm * ntn, KF / 2, split_k, kps);
  if (s <= 1) return 0;
  return kCounterBytes + int64_t(ntm) * ntn * s * kBM[cfg] * kBN[cfg] * 4;
}

// Blocks per CU the tile is built for: two when two rings fit in the 160 KiB of LDS.
template <int BM, int BN, int NS>
constexpr int blocks_per_cu() { return 2 * NS * 2 * (BM / 32 + BN / 32) * 1024 <= 160 * 1024 ? 2 : 1; }

template <int BM, int BN, int WGM, int WGN, int NS, bool AP, bool SPLIT>
static void launch_kernel(const GemmParams& p, int epi, dim3 grid, hipStream_t stream) {
  const int threads = WGM * WGN * 64;
  constexpr int B = blocks_per_cu<BM, BN, NS>();
  switch (epi) {
    case EPI_I32: gemm_kernel<BM, BN, WGM, WGN, NS, EPI_I32, AP, SPLIT, B><<<grid, threads, 0, stream>>>(p); break;
    case EPI_BF16: gemm_kernel<BM, BN, WGM, WGN, NS, EPI_BF16, AP, SPLIT, B><<<grid, threads, 0, stream>>>(p); break;
    case EPI_GELU: gemm_kernel<BM, BN, WGM, WGN, NS, EPI_GELU, AP, SPLIT, B><<<grid, threads, 0, stream>>>(p); break;
    case EPI_RESID: gemm_kernel<BM, BN, WGM, WGN, NS, EPI_RESID, AP, SPLIT, B><<<grid, threads, 0, stream>>>(p); break;
  }
}

// CAN_SPLIT: this tile shape has a split-K instantiation (the 256x256 tiles, used only when
// there are enough tiles to fill the GPU, do not).
template <int BM, int BN, int WGM, int WGN, int NS, bool AP, bool CAN_SPLIT>
static void launch_epi(GemmParams p, int epi, void* ws, int64_t ws_bytes, hipStream_t stream) {
  const int ntm = (p.M + BM - 1) / BM;
  const int ntn = (p.NT * 32 + BN - 1) / BN;
  p.gm = min(ntm, BM >= BN ? 4 : 8);
  const int KT = p.KF / 2;
  p.splits = 1;
  p.kt_per_split = KT;
  if (CAN_SPLIT && ws) {
    int kps;
    const int s = pick_splits(ntm * ntn, KT, p.split_req, kps);
    const int64_t need = kCounterBytes + int64_t(ntm) * ntn * s * BM * BN * 4;
    if (s > 1 && ws_bytes >= need && ntm * ntn * 4 <= kCounterBytes) {
      p.splits = s;
      p.kt_per_split = kps;
      p.counters = static_cast<int*>(ws);
      p.ws = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + kCounterBytes);
    }
  }
  dim3 grid(unsigned(ntm * ntn * p.splits));
  if (CAN_SPLIT && p.splits > 1)
    launch_kernel<BM, BN, WGM, WGN, NS, AP, CAN_SPLIT>(p, epi, grid, stream);
  else
    launch_kernel<BM, BN, WGM, WGN, NS, AP, false>(p, epi, grid, stream);
}

template <int BM, int BN, int WGM, int WGN, int NS, bool CAN_SPLIT>
static void launch(const GemmParams& p, int epi, bool a_packed, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (a_packed)
    launch_epi<BM, BN, WGM, WGN, NS, true, CAN_SPLIT>(p, epi, ws, ws_bytes, stream);
  else
    launch_epi<BM, BN, WGM, WGN, NS, false, CAN_SPLIT>(p, epi, ws, ws_bytes, stream);
}

// Tile configurations (block tile, 4 waves in 2 x 2, LDS ring depth):
//   0: 256x256, waves of 128x128, 4 slots (128 KiB)
//   1: 256x256, waves of 128x128, 5 slots (160 KiB)
//   2: 128x256, waves of 64x128,  6 slots (144 KiB)
//   3: 256x128, waves of 128x64,  6 slots (144 KiB)
//   4: 128x128, waves of 64x64,   8 slots (128 KiB)
//   5: 128x128, waves of 64x64,   4 slots (64 KiB, two blocks per CU)
//   6: 256x128, waves of 128x64,  3 slots (72 KiB, two blocks per CU)
//   7: 128x256, waves of 64x128,  3 slots (72 KiB, two blocks per CU)
int gemm_config_count() { return 8; }

// Tile choice, from timing every configuration on the E2B prefill shapes (M = 512, 3658,
// 16384): 256x256 when there are enough of them (>= 4 waves of blocks), else the two-blocks-
// per-CU tiles, 256 wide along the longer of M and N when that still gives >= 384 tiles.
int gemm_pick_config(int M, int NP, int K) {
  (void)K;
  auto tiles = [&](int c) { return long((M + kBM[c] - 1) / kBM[c]) * ((NP + kBN[c] - 1) / kBN[c]); };
  if (tiles(0) >= 1024) return 0;
  const int wide = M >= NP ? 6 : 7;
  if (tiles(wide) >= 384) return wide;
  return 5;
}

int gemm_launch(const GemmParams& p, int epi, int cfg, bool a_packed, void* ws, int64_t ws_bytes,
                hipStream_t stream) {
  if (cfg < 0) cfg = gemm_pick_config(p.M, p.NT * 32, p.KF * 32);
  switch (cfg) {
    case 0: launch<256, 256, 2, 2, 4, false>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 1: launch<256, 256, 2, 2, 5, false>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 2: launch<128, 256, 2, 2, 6, true>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 3: launch<256, 128, 2, 2, 6, true>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 4: launch<128, 128, 2, 2, 8, true>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 5: launch<128, 128, 2, 2, 4, true>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 6: launch<256, 128, 2, 2, 3, true>(p, epi, a_packed, ws, ws_bytes, stream); break;
    case 7: launch<128, 256, 2, 2, 3, true>(p, epi, a_packed, ws, ws_bytes, stream); break;
    default: return fail(W8A8_EINVAL, "gemm: unknown tile config %d", cfg);
  }
  return check_launch("gemm");
}

}  // namespace w8a8
