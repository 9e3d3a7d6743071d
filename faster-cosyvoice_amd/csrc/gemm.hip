// f16 MFMA GEMM for gfx950 with fused epilogues.
//
// C[M,N] = A[M,K] . W[N,K]^T, both operands K-contiguous (PyTorch Linear layout), fp32
// accumulation on v_mfma_f32_32x32x16_f16 (on this part the 32x32x16 form sustains ~93% of
// the f16 peak in a register loop, the 16x16x32 form ~54%).
//
// Main loop.  A workgroup of WM x WN waves owns a BM x BN tile (256x256, 192x256, 128x256 and
// 256x128 with 8 waves, 160x256, 128x128, 96x128 and 32x128 with 4 waves, several workgroups
// per CU);
// each wave a sub-tile of 32x32 MFMA tiles.  Operands go straight from global memory into LDS
// with global_load_lds_dwordx4 (no register staging, no ds_write; scalar base and LDS address,
// per-lane 32-bit offset) through a ring of slices (two stages of K = 64, three for the small
// 32x128 tile, whose few workgroups per CU leave the copy latency exposed: FF2 at ~1k rows
// 19.6 -> 17.3 us; and where a launch's tiles fit one round of CUs, so each holds a CU alone,
// three for 96x128 and 128x128 and four for 32x128; one wave-level copy fills 1 KB of LDS =
// 8 rows x 128 B, so every L2 request is a full 128-byte line).  The 16-byte chunks of a row
// sit at a row-rotated position, so 16 consecutive rows read at one chunk index hit 16 distinct
// 16-byte bank groups.  Inside a slice the fragments of
// k-step ks+1 are read while the MFMAs of k-step ks run, and the loop is rotated so that a
// slice's last k-step runs after the barrier that publishes the next slice.  The tile shape is
// chosen per call from the tile rounds over the 256 CUs and per-shape rates.

// Operand roles are swapped: the MFMA computes D = W_tile . A_tile^T, so the accumulator of a
// 32x32 tile holds, in lane l, output row m = l % 32 and four consecutive output columns per
// register group.  Every epilogue therefore reads and writes 4 consecutive columns of one row
// at a time (16-byte fp32 / 8-byte f16 vector accesses), and the interleaved RoPE pairs
// (2i, 2i+1) sit in the same lane.
//
// Rasterization: blocks are dealt round-robin over the 8 XCDs, so block ids are first remapped
// to give each XCD a contiguous range of tiles; inside that range tiles are visited in groups of
// GROUP_M M-tiles x all N-tiles (M fastest), keeping the group's A rows and W columns inside
// one XCD's 4 MB L2.
#include <cstdlib>
#include <type_traits>

#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int kXcds = 8;

// Tile shape.  WM x WN waves; each wave owns (BM/WM) x (BN/WN) outputs as TM x TN MFMA tiles of
// 32x32.  A ring of STAGES LDS slices of (BM + BN) x BK f16; one wave-level copy fills 1 KB =
// ROWS_PER_COPY rows of one slice.
template <int BM_, int BN_, int WM_, int WN_, int BK_ = 64, int STAGES_ = 2>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_, STAGES = STAGES_;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static constexpr int ROW_CHUNKS = BK / 8;            // 16-byte chunks per slice row
  static constexpr int ROWS_PER_COPY = 64 / ROW_CHUNKS;
  static constexpr int A_INSTR = BM / ROWS_PER_COPY / kWaves;  // copies per wave per slice
  static constexpr int B_INSTR = BN / ROWS_PER_COPY / kWaves;
  static constexpr int LOADS = A_INSTR + B_INSTR;
  static constexpr int kLds = STAGES * (BM + BN) * BK * 2;
  static constexpr int kOcc = (160 * 1024) / kLds >= 2 ? 2 : 1;  // workgroups per CU
  static constexpr int kGroupM = 1024 / BM > 0 ? 1024 / BM : 1;  // ~1024 A rows per L2 group
  static_assert(BK == 32 || BK == 64, "slice depth");
  static_assert(STAGES >= 2 && (STAGES - 2) * LOADS < 64, "ring depth");
  static_assert(BM % (ROWS_PER_COPY * kWaves) == 0 && BN % (ROWS_PER_COPY * kWaves) == 0,
                "copy split");
  static_assert(TM * WM * 32 == BM && TN * WN * 32 == BN, "wave tiling");
};

// Block bid -> tile (tm, tn) of `total` tiles; false for a block past them (a grid sized for a
// larger capacity than the live rows need).  Each XCD's blocks take a contiguous tile range.
__device__ __forceinline__ bool tile_coords(int bid, int total, int tiles_m, int tiles_n,
                                            int group_m, int& tm, int& tn) {
  const int xcd = bid % kXcds, idx = bid / kXcds;
  const int base = total / kXcds, extra = total % kXcds;
  if (idx >= base + (xcd < extra ? 1 : 0)) return false;
  const int t = xcd * base + min(xcd, extra) + idx;
  const int per_group = group_m * tiles_n;
  const int g = t / per_group;
  const int first_m = g * group_m;
  const int gm = min(group_m, tiles_m - first_m);
  const int r = t - g * per_group;
  tm = first_m + r % gm;
  tn = r / gm;
  return true;
}

// position of 16-byte chunk `chunk` in LDS row `row`: rows of 8 chunks (BK 64) rotate by row/2,
// rows of 4 chunks (BK 32) by row/4, so 16 consecutive rows read at one chunk index hit 16
// distinct 16-byte bank groups
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  return BK == 64 ? chunk ^ ((row >> 1) & 7) : chunk ^ ((row >> 2) & 3);
}

// Lane-strided 16-byte global -> LDS copy: lane l copies the 16 bytes at base + voff (its own
// 32-bit byte offset from a wave-uniform 64-bit base held in SGPRs) to bytes [16 l, 16 l + 16)
// from the wave-uniform LDS address `lds`.  With the base and the LDS address scalar, a copy
// costs one m0 write and one load instruction; the K advance is a scalar add on the base.
// Issued as inline asm so the compiler does not treat every later LDS read as dependent on it
// (it would wait for vmcnt(0) before each one); the K loop orders these copies with explicit
// vmcnt waits and barriers instead.  (m0 is named as a clobber on purpose: the copy's LDS base
// lives there.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(n) (n < 64: bits [3:0] and [15:14]), leaving expcnt / lgkmcnt unconstrained
#define FCV_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define FCV_WAIT_VMCNT0() FCV_WAIT_VMCNT(0)

// vmcnt(ahead * L) for a wave-uniform ahead in [0, A]
template <int L, int A>
__device__ __forceinline__ void wait_loads_ahead(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      FCV_WAIT_VMCNT(A * L);
      return;
    }
    wait_loads_ahead<L, A - 1>(ahead);
  } else {
    FCV_WAIT_VMCNT0();
  }
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Whether an epilogue's per-row loads are issued one 32-row block ahead (the default); an
// epilogue sets kPipelineRows = false when two blocks of its row context do not fit in registers.
template <class E, class = void>
struct pipeline_rows : std::true_type {};
template <class E>
struct pipeline_rows<E, std::void_t<decltype(E::kPipelineRows)>>
    : std::bool_constant<E::kPipelineRows> {};

// Whether an epilogue writes some tiles in the accumulator's own lane layout (finish_direct).
template <class E, class = void>
struct direct_layout : std::false_type {};
template <class E>
struct direct_layout<E, std::void_t<decltype(&E::finish_direct)>> : std::true_type {};

// workgroups per CU with the epilogue's row_info array in LDS as well
template <class C, class Epi>
constexpr int occupancy() {
  return (160 * 1024) / (C::kLds + (Epi::kRowInfo ? C::BM * 4 : 0)) >= 2 ? C::kOcc : 1;
}

template <class C, class Epi>
__global__ __launch_bounds__(C::kThreads, (occupancy<C, Epi>())) void gemm_kernel(
    const f16* __restrict__ A, int lda, const f16* __restrict__ W, int ldw, int M, int N, int K,
    Epi epi, const int32_t* __restrict__ m_live) {
  constexpr int BM = C::BM, BN = C::BN, TM = C::TM, TN = C::TN, BK = C::BK, S = C::STAGES;
  // operand ring; after the K loop the same bytes stage the epilogue
  __shared__ __attribute__((aligned(1024))) f16 smem[S * (BM + BN) * BK];
  f16 (*sA)[BM * BK] = reinterpret_cast<f16 (*)[BM * BK]>(smem);
  f16 (*sB)[BN * BK] = reinterpret_cast<f16 (*)[BN * BK]>(smem + S * BM * BK);

  if (m_live) M = *m_live;  // live rows of a capacity-sized grid
  const int tiles_n = N / BN;
  const int tiles_m = (M + BM - 1) / BM;
  int tmi, tni;
  if (!tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, C::kGroupM, tmi, tni)) return;
  const int m0 = tmi * BM;
  const int n0 = tni * BN;
  const int lane = threadIdx.x & 63;
  // per-row epilogue inputs (row_info) of the tile's rows, fetched ahead of the operand copies
  // (so the wait for the first slice covers them) and parked in LDS with the first slice
  static_assert(BM <= C::kThreads, "one thread per tile row");
  __shared__ int32_t rinfo[Epi::kRowInfo ? BM : 1];
  int rin = -1;
  if constexpr (Epi::kRowInfo) {
    if ((int)threadIdx.x < BM && m0 + (int)threadIdx.x < M) rin = epi.row_info(m0 + threadIdx.x);
  }
  // wave index as a scalar, so the copies' LDS destinations are computed in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm0 = (wave / C::WN) * (BM / C::WM);
  const int wn0 = (wave % C::WN) * (BN / C::WN);

  // per-lane source of each copy: row r0 + lane / ROW_CHUNKS, and the chunk that belongs at LDS
  // position lane % ROW_CHUNKS of that row (A rows clamped to M - 1), as a byte offset from the
  // operand's base (A spans < 4 GB: rows x lda x 2 bytes).  The destinations are scalar: the
  // stage's base + this wave's first copy row + i copies.
  const int lrow = lane / C::ROW_CHUNKS;
  const int lpos = lane % C::ROW_CHUNKS;
  uint32_t a_off[C::A_INSTR], w_off[C::B_INSTR];
#pragma unroll
  for (int i = 0; i < C::A_INSTR; ++i) {
    const int row = (wave * C::A_INSTR + i) * C::ROWS_PER_COPY + lrow;
    a_off[i] = (uint32_t)(((long)min(m0 + row, M - 1) * lda + swz<BK>(row, lpos) * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < C::B_INSTR; ++i) {
    const int row = (wave * C::B_INSTR + i) * C::ROWS_PER_COPY + lrow;
    w_off[i] = (uint32_t)(((long)(n0 + row) * ldw + swz<BK>(row, lpos) * 8) * 2);
  }
  constexpr uint32_t kCopyBytes = C::ROWS_PER_COPY * BK * 2;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem;
  const uint32_t lds_a = lds_base + (uint32_t)wave * C::A_INSTR * kCopyBytes;
  const uint32_t lds_b = lds_base + S * BM * BK * 2 + (uint32_t)wave * C::B_INSTR * kCopyBytes;
  auto issue = [&](int kt, int stage) {
    const f16* a_k = A + kt * BK;
    const f16* w_k = W + kt * BK;
#pragma unroll
    for (int i = 0; i < C::A_INSTR; ++i)
      lds_dma16(a_k, a_off[i], lds_a + stage * (BM * BK * 2) + i * kCopyBytes);
#pragma unroll
    for (int i = 0; i < C::B_INSTR; ++i)
      lds_dma16(w_k, w_off[i], lds_b + stage * (BN * BK * 2) + i * kCopyBytes);
  };

  // Column-only epilogue inputs (bias; gates shared by all rows) are loaded here, before the K
  // loop: issued after the epilogue's first stores they would wait for those stores to drain
  // (loads and stores share one counter).  Staged layout: lanes 16r .. 16r + 15 cover the
  // wave's TN x 32 columns, 4 per lane; direct layout: register group g of MFMA tile j holds
  // columns 32 j + 8 g + 4 (lane / 32) + 0..3.
  using Col = typename Epi::Col;
  constexpr int WCOLS = TN * 32;
  constexpr int LANES_PER_ROW = WCOLS / 4;
  const int col_base = n0 + wn0;
  bool direct = false;
  if constexpr (direct_layout<Epi>::value) direct = epi.direct(col_base);
  const int rc = (lane % LANES_PER_ROW) * 4;
  Col scol{};
  Col dcol[TN][4];
  if (direct) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) dcol[j][g] = epi.column(col_base + j * 32 + g * 8 + (lane >> 5) * 4);
  } else {
    scol = epi.column(col_base + rc);
  }

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int fr = lane & 31, fh = lane >> 5;
  // Ring of S stages, K loop rotated by one k-step.  Slice j is published by a wait for this
  // wave's copies of slice j (the copies of the up to S-2 later slices already issued may still
  // be in flight; loads complete in order) and a barrier (all copies of slice j landed; every
  // wave has its last fragments of slice j-1 in registers, so the stage slice j-1 used is free).
  // The barrier sits between k-steps KS-2 and KS-1 of slice j-1: after it the wave starts slice
  // j+S-1 into that free stage, reads slice j's k-step 0 fragments, and runs slice j-1's last
  // k-step from registers while those reads are in flight, so the matrix pipe does not wait on
  // a fresh LDS read after a barrier.  Inside a slice the fragments of k-step ks+1 are read
  // while the MFMAs of k-step ks run.  Every accumulator sees its k-steps in the same order as
  // an unrotated loop.
  const int KT = K / BK;
  constexpr int KS = BK / 16;
  static_assert(KS % 2 == 0, "k-step 0 of a slice uses fragment buffer 0");
  f16x8 fa[2][TM], fb[2][TN];
  auto load = [&](int buf, int ks, int st) {
    const f16* a_st = sA[st];
    const f16* b_st = sB[st];
    const int chunk = ks * 2 + fh;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = wm0 + i * 32 + fr;
      fa[buf][i] = *reinterpret_cast<const f16x8*>(a_st + row * BK + swz<BK>(row, chunk) * 8);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int row = wn0 + j * 32 + fr;
      fb[buf][j] = *reinterpret_cast<const f16x8*>(b_st + row * BK + swz<BK>(row, chunk) * 8);
    }
  };
  // scheduling fences keep each k-step's LDS reads ahead of the previous k-step's MFMAs (left
  // alone, the scheduler sinks each read next to its first use and waits on it)
  auto mma = [&](int buf) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(fb[buf][j], fa[buf][i], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
  };
  // k-steps 0 .. KS-2 of the slice in stage st (k-step 0's fragments already in buffer 0);
  // leaves k-step KS-1's fragments in buffer 1
  auto slice_head = [&](int st) {
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      load((ks + 1) & 1, ks + 1, st);
      mma(ks & 1);
    }
  };
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < KT) issue(st, st);
  wait_loads_ahead<C::LOADS, S - 2>(KT - 1);  // slice 0
  if constexpr (Epi::kRowInfo) {
    if ((int)threadIdx.x < BM) rinfo[threadIdx.x] = rin;
  }
  __syncthreads();
  if (S - 1 < KT) issue(S - 1, S - 1);
  load(0, 0, 0);
  slice_head(0);
  int stage = 0;
  for (int kt = 1; kt < KT; ++kt) {
    const int next = stage == S - 1 ? 0 : stage + 1;
    wait_loads_ahead<C::LOADS, S - 2>(KT - 1 - kt);  // slice kt
    __syncthreads();
    if (kt + S - 1 < KT) issue(kt + S - 1, stage);  // into the stage slice kt-1 used
    load(0, 0, next);
    mma(1);  // slice kt-1, last k-step
    slice_head(next);
    stage = next;
  }
  mma(1);  // last slice, last k-step

  // Nothing is in flight here; the explicit wait tells the compiler's counter tracking that the
  // column loads issued before the loop are complete on every path (with a zero-trip loop path
  // it would otherwise wait again, for every store, inside each row-guarded store block).
  FCV_WAIT_VMCNT0();

  // Epilogue.  Accumulator lane l holds output row m0 + wm0 + 32 i + l % 32 and, in register
  // group g, columns n0 + wn0 + 32 j + 8 g + 4 (l / 32) + 0..3: stored directly, every store
  // instruction would touch 32 rows.  Instead each wave stages one 32-row block at a time
  // through its own LDS region (row pitch padded by 16 bytes) and reads it back row-major:
  // lanes 16 r .. 16 r + 15 then cover TN x 32 consecutive columns of one row, so the epilogue's
  // stores are contiguous runs of 16 x 16 B (fp32) or 16 x 8 B (f16).  Epilogues that write a
  // transposed layout (V^T) keep the direct lane layout, where 32 lanes cover 32 rows.
  // Row-dependent loads of a block (residual, row indices, rotary tables) are issued together
  // by prepare before the block's stores in finish; finish computes its values unconditionally
  // and guards only the stores, so a block waits for its loads once, not once per store.
  using Ctx = typename Epi::Ctx;
  constexpr int PITCH = WCOLS + 4;  // floats
  static_assert(C::kWaves * 32 * PITCH * 4 <= (int)sizeof(smem), "epilogue staging");
  if constexpr (direct_layout<Epi>::value) {
  if (direct) {
    // direct-layout tiles (V^T) read nothing per row
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = m0 + wm0 + i * 32 + fr;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                           acc[i][j][4 * g + 3]};
          const int c = col_base + j * 32 + g * 8 + fh * 4;
          epi.finish_direct(v, dcol[j][g], row, c, M);
        }
      }
    }
    return;
  }
  }
  __syncthreads();  // every wave is done reading the operand ring
  float* stg = reinterpret_cast<float*>(smem) + wave * 32 * PITCH;
  constexpr int ROWS_PER_PASS = 64 / LANES_PER_ROW;
  constexpr int PASSES = 32 / ROWS_PER_PASS;
  const int rr = lane / LANES_PER_ROW;
  const int col = col_base + rc;
  // Two instantiations: tiles whose epilogue reads per-row data (the residual, rotary angles)
  // issue each 32-row block's loads one block ahead, before the previous block's stores, so a
  // block's wait covers loads that have been in flight for a whole block and not the stores
  // just issued (loads and stores share one counter and complete in order); the rows' row_info
  // comes from LDS, so no load waits on another.  Tiles without row data never wait.
  auto prepare_block = [&](int i, Ctx (&cx)[PASSES]) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int tr = wm0 + i * 32 + p * ROWS_PER_PASS + rr;
      int info = -1;
      if constexpr (Epi::kRowInfo) info = rinfo[tr];
      cx[p] = epi.prepare(m0 + tr, col, M, scol, info);
    }
  };
  auto staged = [&](auto loads_c) {
    constexpr bool kLoads = decltype(loads_c)::value;
    constexpr bool kAhead = pipeline_rows<Epi>::value;
    Ctx cx[PASSES];
    if constexpr (kLoads && kAhead) prepare_block(0, cx);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(stg + fr * PITCH + j * 32 + g * 8 + fh * 4) =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                    acc[i][j][4 * g + 3]};
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      f32x4 v[PASSES];
#pragma unroll
      for (int p = 0; p < PASSES; ++p)
        v[p] = *reinterpret_cast<const f32x4*>(stg + (p * ROWS_PER_PASS + rr) * PITCH + rc);
      // the next block's row loads go out before this block's stores (or, for epilogues whose
      // row context is too large to hold twice, this block's, waited for here)
      Ctx cn[PASSES];
      if constexpr (kLoads && kAhead) {
        if (i + 1 < TM) prepare_block(i + 1, cn);
      } else if constexpr (kLoads) {
        prepare_block(i, cx);
        FCV_WAIT_VMCNT0();
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int r = p * ROWS_PER_PASS + rr;
        const Ctx x = kLoads ? cx[p] : epi.blank(scol);
        epi.template finish<kLoads>(v[p], x, scol, m0 + wm0 + i * 32 + r, col, M);
      }
      if constexpr (kLoads && kAhead) {
        if (i + 1 < TM) {
#pragma unroll
          for (int p = 0; p < PASSES; ++p) cx[p] = cn[p];
        }
      }
    }
  };
  if (epi.row_loads(col_base, WCOLS))
    staged(std::true_type{});
  else
    staged(std::false_type{});
}

// ---- epilogues: v = C[row][col .. col+3] (col % 4 == 0) -------------------------------------
// column(col): loads that depend on the column only (issued before the K loop);
// row_loads(col0, n): whether columns [col0, col0 + n) need per-row data;
// kRowInfo / row_info(row): one int per row (a position, a document, a destination row), loaded
// for the tile's rows before the K loop and kept in LDS;
// prepare(row, col, M, col_ctx, info): the row-dependent loads (info = the row's row_info, or -1
// past M); blank(col_ctx): the context when there are none; finish(v, ctx, col_ctx, row, col,
// M): the arithmetic and the stores.

__device__ __forceinline__ float4 add4(const f32x4& v, const float4& b) {
  return float4{v[0] + b.x, v[1] + b.y, v[2] + b.z, v[3] + b.w};
}
struct NoCtx {};
struct BiasCol { float4 b; };

// Raw buffer accesses (stride 0) over [base, base + bytes): a load past `bytes` reads zeros and a
// store past it is dropped, so row guards (row >= M) cost no branch, and the offsets are 32-bit
// (the callers check that M x ld x element size stays below 2 GB, the range being an int).
// Descriptor word 3 = 0x00020000: DATA_FORMAT 32 bits (bits 15-18 = 4), no swizzle, the
// setting raw (untyped) buffer accesses use on this GPU family.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 buffer_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return float4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                __uint_as_float(v.w)};
}
__device__ __forceinline__ void buffer_st4(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 x) {
  const u32x4 v = {__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z),
                   __float_as_uint(x.w)};
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}
__device__ __forceinline__ void buffer_st_f16x4(__amdgpu_buffer_rsrc_t r, uint32_t off, f16x4 x) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, x), r, off, 0, 0);
}

struct EpiBiasF32F16 {
  const float* bias;
  float* out_f32;
  f16* out_f16;
  int ldo;
  using Col = BiasCol;
  using Ctx = NoCtx;
  __device__ bool row_loads(int, int) const { return false; }
  __device__ Ctx blank(const Col&) const { return {}; }
  __device__ bool direct(int) const { return false; }
  __device__ Col column(int col) const { return {ld4(bias + col)}; }
  static constexpr bool kRowInfo = false;
  __device__ Ctx prepare(int, int, int, const Col&, int) const { return {}; }
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx&, const Col& c, int row, int col, int M) const {
    const float4 y = add4(v, c.b);
    const f16x4 yb = f2h4(y.x, y.y, y.z, y.w);
    if (row >= M) return;
    *reinterpret_cast<float4*>(out_f32 + (long)row * ldo + col) = y;
    *reinterpret_cast<f16x4*>(out_f16 + (long)row * ldo + col) = yb;
  }
};

struct EpiBiasF32 {
  const float* bias;
  float* out;
  int ldo;
  int n_valid;  // multiple of 4
  using Col = BiasCol;
  using Ctx = NoCtx;
  __device__ bool row_loads(int, int) const { return false; }
  __device__ Ctx blank(const Col&) const { return {}; }
  __device__ bool direct(int) const { return false; }
  __device__ Col column(int col) const {
    return {col < n_valid ? ld4(bias + col) : float4{0.f, 0.f, 0.f, 0.f}};
  }
  static constexpr bool kRowInfo = false;
  __device__ Ctx prepare(int, int, int, const Col&, int) const { return {}; }
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx&, const Col& c, int row, int col, int M) const {
    const float4 y = add4(v, c.b);
    if (row >= M || col >= n_valid) return;
    *reinterpret_cast<float4*>(out + (long)row * ldo + col) = y;
  }
};

struct EpiBiasF32RowMap {
  const float* bias;
  float* out;
  int ldo;
  int n_valid;  // multiple of 4
  const int32_t* row_map;
  using Col = BiasCol;
  struct Ctx { int dst; };
  __device__ bool row_loads(int, int) const { return true; }
  __device__ Ctx blank(const Col&) const { return {-1}; }
  __device__ bool direct(int) const { return false; }
  __device__ Col column(int col) const {
    return {col < n_valid ? ld4(bias + col) : float4{0.f, 0.f, 0.f, 0.f}};
  }
  static constexpr bool kRowInfo = true;
  __device__ int row_info(int row) const { return row_map[row]; }
  __device__ Ctx prepare(int row, int, int M, const Col&, int info) const {
    return {row < M ? info : -1};
  }
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx& x, const Col& c, int, int col, int) const {
    const float4 y = add4(v, c.b);
    if (x.dst < 0 || col >= n_valid) return;
    *reinterpret_cast<float4*>(out + (long)x.dst * ldo + col) = y;
  }
};

struct EpiBiasSiluF16 {
  const float* bias;
  f16* out;
  int ldo;
  using Col = BiasCol;
  using Ctx = NoCtx;
  __device__ bool row_loads(int, int) const { return false; }
  __device__ Ctx blank(const Col&) const { return {}; }
  __device__ bool direct(int) const { return false; }
  __device__ Col column(int col) const { return {ld4(bias + col)}; }
  static constexpr bool kRowInfo = false;
  __device__ Ctx prepare(int, int, int, const Col&, int) const { return {}; }
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx&, const Col& c, int row, int col, int M) const {
    const float4 y = add4(v, c.b);
    const f16x4 yb = f2h4(silu(y.x), silu(y.y), silu(y.z), silu(y.w));
    if (row >= M) return;
    *reinterpret_cast<f16x4*>(out + (long)row * ldo + col) = yb;
  }
};

struct EpiBiasGeluF16 {
  const float* bias;
  f16* out;
  int ldo;
  using Col = BiasCol;
  using Ctx = NoCtx;
  __device__ bool row_loads(int, int) const { return false; }
  __device__ Ctx blank(const Col&) const { return {}; }
  __device__ bool direct(int) const { return false; }
  __device__ Col column(int col) const { return {ld4(bias + col)}; }
  static constexpr bool kRowInfo = false;
  __device__ Ctx prepare(int, int, int, const Col&, int) const { return {}; }
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx&, const Col& c, int row, int col, int M) const {
    const float4 y = add4(v, c.b);
    const f16x4 yb = f2h4(gelu_tanh(y.x), gelu_tanh(y.y), gelu_tanh(y.z), gelu_tanh(y.w));
    buffer_st_f16x4(buffer_over(out, (uint32_t)M * ldo * 2), (uint32_t)(row * ldo + col) * 2, yb);
  }
};

// h += gate * (acc + bias).  kPerDoc: each document has its own gate row (gate + d * mod_stride,
// d = docid[row]); otherwise one gate row is shared by every document and is loaded with the
// bias, before the K loop.  h is read and written through raw buffer accesses over its M rows.
template <bool kPerDoc>
struct EpiGatedResidual {
  const float* bias;
  float* h;
  int ldh;
  const float* gate;  // mod + gate offset
  long mod_stride;
  const int32_t* docid;
  struct Col { float4 b, g; };
  struct Ctx { float4 g, x; };
  __device__ bool row_loads(int, int) const { return true; }
  __device__ Ctx blank(const Col& c) const { return {c.g, float4{0.f, 0.f, 0.f, 0.f}}; }
  __device__ bool direct(int) const { return false; }
  __device__ Col column(int col) const {
    Col c;
    c.b = ld4(bias + col);
    c.g = kPerDoc ? float4{0.f, 0.f, 0.f, 0.f} : ld4(gate + col);
    return c;
  }
  static constexpr bool kRowInfo = kPerDoc;  // the row's document
  // a per-document gate row doubles the row context: one block of it at a time
  static constexpr bool kPipelineRows = !kPerDoc;
  __device__ int row_info(int row) const { return docid[row]; }
  __device__ Ctx prepare(int row, int col, int M, const Col& c, int info) const {
    Ctx x;
    x.g = c.g;
    if constexpr (kPerDoc) {
      if (row < M) x.g = ld4(gate + (long)info * mod_stride + col);
    }
    x.x = buffer_ld4(buffer_over(h, (uint32_t)M * ldh * 4), (uint32_t)(row * ldh + col) * 4);
    return x;
  }
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx& x, const Col& c, int row, int col, int M) const {
    const float4 y = add4(v, c.b);
    const float4 r = {fmaf(x.g.x, y.x, x.x.x), fmaf(x.g.y, y.y, x.x.y), fmaf(x.g.z, y.z, x.x.z),
                      fmaf(x.g.w, y.w, x.x.w)};
    buffer_st4(buffer_over(h, (uint32_t)M * ldh * 4), (uint32_t)(row * ldh + col) * 4, r);
  }
};

struct EpiQkvRope {
  const float* bias;
  int dim;        // heads * 64
  int rows;       // q / k row pitch per head (rp)
  const int32_t* pos;
  const float* rope_cos;
  const float* rope_sin;
  int rope_dim;
  int max_pos;
  f16* q;
  f16* k;
  f16* vt;
  int rp;
  using Col = BiasCol;
  struct Ctx { float2 cs, sn; };
  // V^T columns keep the accumulator lane layout (32 lanes = 32 consecutive rows of vt)
  // only the rotated columns (q and k columns < rope_dim) read per-row angles
  __device__ bool row_loads(int col0, int n) const {
    return col0 < 2 * dim && col0 % dim < rope_dim && n > 0;
  }
  __device__ Ctx blank(const Col&) const { return {{1.0f, 1.0f}, {0.0f, 0.0f}}; }
  __device__ bool direct(int col) const { return col >= 2 * dim; }
  __device__ Col column(int col) const { return {ld4(bias + col)}; }
  // the row's position, clamped to the tables (pad rows run past the document)
  static constexpr bool kRowInfo = true;
  __device__ int row_info(int row) const { return min(pos[row], max_pos - 1); }
  __device__ Ctx prepare(int row, int col, int M, const Col&, int info) const {
    Ctx c = {{1.0f, 1.0f}, {0.0f, 0.0f}};  // identity rotation where no angle is loaded
    const int cc = col >= dim ? col - dim : col;  // column in q or k (used when col < 2 dim)
    if (col < 2 * dim && row < M && cc < rope_dim) {
      // angles of the interleaved pairs (cc, cc+1), (cc+2, cc+3)
      const long t = (long)info * (rope_dim >> 1) + (cc >> 1);
      c.cs = *reinterpret_cast<const float2*>(rope_cos + t);
      c.sn = *reinterpret_cast<const float2*>(rope_sin + t);
    }
    return c;
  }
  // V^T tiles (columns >= 2 dim) keep the accumulator lane layout: vt[head][d + e][row], 32
  // lanes = 32 consecutive rows; rows in [M, rp) get finite copies of row M-1
  __device__ void finish_direct(const f32x4& v, const Col& cb, int row, int col, int) const {
    const float4 y = add4(v, cb.b);
    const int c = col - 2 * dim;
    const int head = c >> 6, d = c & 63;
    const f16x4 v4 = f2h4(y.x, y.y, y.z, y.w);
    if (row >= rp) return;
    f16* dst = vt + ((long)head * 64 + d) * rp + row;
    dst[0] = v4[0];
    dst[rp] = v4[1];
    dst[2 * rp] = v4[2];
    dst[3 * rp] = v4[3];
  }
  // q and k tiles (staged row-major): a wave's columns (at most 64, aligned) lie in one head, so
  // which, head and d are the same in every call of a lane.  kRowCtx: the tile's columns read
  // rotary angles (row_loads); without them no column of the tile rotates.
  template <bool kRowCtx>
  __device__ void finish(const f32x4& v, const Ctx& cx, const Col& cb, int row, int col,
                         int M) const {
    float4 y = add4(v, cb.b);
    // 0 q, 1 k; the same for every lane of a wave (its columns lie in one head), made scalar so
    // the store's buffer descriptor is built once in scalar registers
    const int which = __builtin_amdgcn_readfirstlane(col >= dim ? 1 : 0);
    const int c = col - which * dim;
    const int head = c >> 6, d = c & 63;
    if constexpr (kRowCtx) {
      // (a, b) -> (a cos - b sin, b cos + a sin) on the rotated columns (c < rope_dim)
      const float a0 = y.x, b0 = y.y, a1 = y.z, b1 = y.w;
      const float4 yr = {a0 * cx.cs.x - b0 * cx.sn.x, b0 * cx.cs.x + a0 * cx.sn.x,
                         a1 * cx.cs.y - b1 * cx.sn.y, b1 * cx.cs.y + a1 * cx.sn.y};
      if (c < rope_dim) y = yr;
    }
    const f16x4 yb = f2h4(y.x, y.y, y.z, y.w);
    if (row >= M) return;
    // q / k: [heads][rows][64], addressed by 32-bit byte offsets (the launcher checks the range)
    buffer_st_f16x4(buffer_over(which ? k : q, (uint32_t)dim * rows * 2),
                    (uint32_t)((head * rows + row) * 64 + d) * 2, yb);
  }
};

using Tile256x256 = TileCfg<256, 256, 2, 4>;
using Tile192x256 = TileCfg<192, 256, 2, 4>;
using Tile160x256 = TileCfg<160, 256, 1, 4>;
using Tile128x256 = TileCfg<128, 256, 2, 4>;
using Tile256x128 = TileCfg<256, 128, 4, 2>;
using Tile128x128 = TileCfg<128, 128, 2, 2>;
using Tile32x128 = TileCfg<32, 128, 1, 4, 64, 3>;
using Tile96x128 = TileCfg<96, 128, 1, 4>;
using Tile96x128x3 = TileCfg<96, 128, 1, 4, 64, 3>;  // one workgroup per CU
using Tile128x128x3 = TileCfg<128, 128, 2, 2, 64, 3>;  // one workgroup per CU
using Tile32x128x4 = TileCfg<32, 128, 1, 4, 64, 4>;
using Tile64x64x3 = TileCfg<64, 64, 2, 2, 64, 3>;    // three workgroups per CU
using Tile64x64x5 = TileCfg<64, 64, 2, 2, 64, 5>;    // two workgroups per CU
using Tile128x64x3 = TileCfg<128, 64, 2, 2, 64, 3>;  // two workgroups per CU
using Tile128x64x4 = TileCfg<128, 64, 2, 2, 64, 4>;  // one workgroup per CU
using Tile64x128x3 = TileCfg<64, 128, 2, 2, 64, 3>;  // two workgroups per CU

template <class C, class Epi>
hipError_t launch_tile(const f16* A, int lda, const f16* W, int ldw, int M, int N, int K,
                       const Epi& epi, hipStream_t stream, const int32_t* m_live) {
  if (N % C::BN != 0 || K % C::BK != 0) return hipErrorInvalidValue;
  const int tiles = ((M + C::BM - 1) / C::BM) * (N / C::BN);
  hipLaunchKernelGGL((gemm_kernel<C, Epi>), dim3(tiles), dim3(C::kThreads), 0, stream, A, lda, W,
                     ldw, M, N, K, epi, m_live);
  return hipGetLastError();
}

// Tile choice for larger launches: estimated time = (tiles per CU, rounded up) x tile area /
// per-CU rate.  The rates are fitted so the estimate picks the fastest shape measured for the
// block GEMMs (N = 1024, 2048, 3072 at ~4.6k and ~9.2k rows, production epilogues): 128x128
// runs two workgroups per CU, which its rate includes; 160x256 runs one wave per SIMD, so it
// rates low although it fills more CUs; 32x128 is rated low so it only wins when the larger
// shapes leave most CUs idle.  96x128 (four 96x32 waves, two workgroups per CU) sits below
// 192x256: it wins for the 1024-column GEMMs from ~2.5k to ~6k rows (a request group's share
// of a batch) and for FF1 and QKV at ~1.3k-3k rows; a sweep of the four block GEMMs over
// 1.1k-9.3k rows with every shape forced found the estimate's pick within 1 % of the fastest
// shape, except at 6.2k rows (QKV, 4 %).
//
// Small launches (one or two requests, up to ~3k rows) follow a measured table instead.  A K
// loop there is bound by the copies' latency, so what counts is how many slices are in flight
// per CU: 64x64 tiles with five ring stages (two per CU) while two per CU hold every tile and
// three stages (three per CU) above, 128x64 with four stages (one per CU) up to ~one round and
// three (two per CU) above, and 64x128 with three.  The larger tiles take over where they fill
// one round of CUs with their three-stage form.  The table is the fastest shape per output
// width measured in eager 22-block solves (weights streamed from HBM as in production) at the
// capacities one request plans into (340-3090 rows) with every shape and ring depth forced;
// its pick is within 3 % of the fastest at every measured size, and the four GEMMs of a block
// take 12-20 % less time at 340-1170 rows than the estimate's pick.  The choice only changes
// which rows and columns share a workgroup: every output element still accumulates its K
// slices in the same order, so results are bitwise identical for every tile shape (batch
// invariance holds).
constexpr int kCus = 256;
constexpr int kTileShapes = 11;
constexpr int kTileShape[kTileShapes][2] = {{256, 256}, {192, 256}, {128, 256}, {256, 128},
                                            {128, 128}, {32, 128},  {160, 256}, {96, 128},
                                            {64, 64},   {128, 64},  {64, 128}};
// 0: chosen from the small-launch table only
constexpr float kTileRate[kTileShapes] = {1.0f, 0.97f, 0.80f, 0.78f, 0.85f, 0.45f, 0.75f, 0.66f,
                                          0.0f, 0.0f,  0.0f};
constexpr int kTile128x128 = 4, kTile96x128 = 7, kTile64x64 = 8, kTile128x64 = 9, kTile64x128 = 10;

inline long tile_count(int M, int N, int bm, int bn) { return (long)((M + bm - 1) / bm) * (N / bn); }

// (largest M, shape) steps of the small-launch table for one output width
struct SmallStep {
  int max_m, shape;
};
constexpr SmallStep kSmall1024[] = {  // output projection and FF2 (K 1024 and 2048)
    {1024, kTile64x64}, {2100, kTile128x64}, {3072, kTile96x128}};
constexpr SmallStep kSmall2048[] = {  // FF1
    {600, kTile64x64}, {1000, kTile128x64}, {1536, kTile96x128}, {2048, kTile128x128},
    {2200, kTile128x64}};
constexpr SmallStep kSmall3072[] = {  // QKV
    {400, kTile64x64}, {850, kTile128x64}, {1000, kTile64x128}, {1200, kTile128x64},
    {1440, kTile64x128}, {2100, kTile96x128}};

template <int L>
inline int small_step(const SmallStep (&steps)[L], int M) {
  for (const SmallStep& s : steps)
    if (M <= s.max_m) return s.shape;
  return -1;
}

inline int choose_tile(int M, int N) {
  int small = -1;
  if (N == 1024) small = small_step(kSmall1024, M);
  else if (N == 2048) small = small_step(kSmall2048, M);
  else if (N == 3072) small = small_step(kSmall3072, M);
  else if (N < 1024 && M <= 3072) small = kTile64x64;  // output projection (128 columns)
  if (small >= 0) return small;
  int best = 4;
  float best_t = 3.0e38f;
  for (int c = 0; c < kTileShapes; ++c) {
    const int bm = kTileShape[c][0], bn = kTileShape[c][1];
    if (N % bn != 0 || kTileRate[c] <= 0.0f) continue;
    const long tiles = (long)((M + bm - 1) / bm) * (N / bn);
    const long per_cu = (tiles + kCus - 1) / kCus;
    const float t = (float)per_cu * bm * bn / kTileRate[c];
    if (t < best_t) { best_t = t; best = c; }
  }
  return best;
}

// FCV_GEMM_TILE=<shape index> forces one tile shape wherever it divides N: a test hook, since
// every shape must give the same bits (the tile choice never changes an element's K order).
inline int forced_tile(int N) {
  const char* e = std::getenv("FCV_GEMM_TILE");
  if (e == nullptr || *e == '\0') return -1;
  const int c = std::atoi(e);
  if (c < 0 || c >= kTileShapes || N % kTileShape[c][1] != 0) return -1;
  return c;
}

// M: the rows the grid covers (a capacity when m_live holds the live count, which must not
// exceed it).  The tile shape is chosen from M; it never changes an element's K summation
// order, so a layout's results are the same under any capacity.
template <class Epi>
hipError_t launch(const f16* A, int lda, const f16* W, int ldw, int M, int N, int K,
                  const Epi& epi, hipStream_t stream, const int32_t* m_live = nullptr) {
  if (M <= 0) return hipSuccess;
  if (N % 128 != 0 || K % 64 != 0 || lda % 8 != 0 || ldw % 8 != 0) return hipErrorInvalidValue;
  // the copies address A and W by 32-bit byte offsets from their bases
  if ((long)M * lda * 2 >= (1L << 32) || (long)N * ldw * 2 >= (1L << 32)) return hipErrorInvalidValue;
  const int forced = forced_tile(N);
  switch (forced >= 0 ? forced : choose_tile(M, N)) {
    case 0: return launch_tile<Tile256x256>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case 1: return launch_tile<Tile192x256>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case 2: return launch_tile<Tile128x256>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case 3: return launch_tile<Tile256x128>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case 5:
      if ((long)((M + 31) / 32) * (N / 128) <= kCus)
        return launch_tile<Tile32x128x4>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
      return launch_tile<Tile32x128>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case 6: return launch_tile<Tile160x256>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case kTile64x64:
      // five ring stages while two per CU hold every tile, three (three per CU) above
      if (tile_count(M, N, 64, 64) <= 2 * kCus)
        return launch_tile<Tile64x64x5>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
      return launch_tile<Tile64x64x3>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case kTile128x64:
      // four stages (one per CU) up to ~one round, three (two per CU) above
      if (tile_count(M, N, 128, 64) <= 288)
        return launch_tile<Tile128x64x4>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
      return launch_tile<Tile128x64x3>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case kTile64x128:
      return launch_tile<Tile64x128x3>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    case 7:
      // where the tiles fit one round of CUs, a third ring stage gives each copy more lead (the
      // tile then holds a CU alone); with more tiles the two-stage form's two per CU win
      if ((long)((M + 95) / 96) * (N / 128) <= kCus)
        return launch_tile<Tile96x128x3>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
      return launch_tile<Tile96x128>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
    default:
      if ((long)((M + 127) / 128) * (N / 128) <= kCus)
        return launch_tile<Tile128x128x3>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
      return launch_tile<Tile128x128>(A, lda, W, ldw, M, N, K, epi, stream, m_live);
  }
}

}  // namespace

hipError_t gemm_bias_f32_f16(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                              int M, int N, int K, float* out_f32, f16* out_f16, int ldo,
                              hipStream_t stream, const int32_t* m_live) {
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32F16{bias, out_f32, out_f16, ldo}, stream,
                m_live);
}

hipError_t gemm_bias_f32(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                         int M, int N, int K, float* out, int ldo, int n_valid,
                         hipStream_t stream) {
  if (n_valid % 4 != 0) return hipErrorInvalidValue;
  // the AdaLN projection and the time MLP (one row per distinct t): reading W is all the work,
  // and the skinny product sums a row the same way whatever the row count, so a document's
  // modulation does not depend on how many t rows the call carries
  if (n_valid == N && gemv_supported(M, K, lda, ldw))
    return gemv_bias_f32(A, lda, W, ldw, bias, M, N, K, out, ldo, stream);
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32{bias, out, ldo, n_valid}, stream);
}

hipError_t gemm_bias_f32_rowmap(const f16* A, int lda, const f16* W, int ldw,
                                const float* bias, int M, int N, int K, float* out, int ldo,
                                int n_valid, const int32_t* row_map, hipStream_t stream,
                                const int32_t* m_live) {
  if (n_valid % 4 != 0) return hipErrorInvalidValue;
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32RowMap{bias, out, ldo, n_valid, row_map},
                stream, m_live);
}

hipError_t gemm_bias_silu_f16(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                               int M, int N, int K, f16* out, int ldo, hipStream_t stream) {
  if (gemv_supported(M, K, lda, ldw))
    return gemv_bias_silu_f16(A, lda, W, ldw, bias, M, N, K, out, ldo, stream);
  return launch(A, lda, W, ldw, M, N, K, EpiBiasSiluF16{bias, out, ldo}, stream);
}

hipError_t gemm_bias_gelu_f16(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                              int M, int N, int K, f16* out, int ldo, hipStream_t stream,
                              const int32_t* m_live) {
  if ((long)M * ldo * 2 >= (1L << 31)) return hipErrorInvalidValue;  // buffer range is an int
  return launch(A, lda, W, ldw, M, N, K, EpiBiasGeluF16{bias, out, ldo}, stream, m_live);
}

hipError_t gemm_gated_residual(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                               int M, int N, int K, float* h, int ldh, const float* gate,
                               long mod_stride, const int32_t* docid, hipStream_t stream,
                               const int32_t* m_live) {
  if ((long)M * ldh * 4 >= (1L << 31)) return hipErrorInvalidValue;  // buffer range is an int
  if (mod_stride == 0)
    return launch(A, lda, W, ldw, M, N, K,
                  EpiGatedResidual<false>{bias, h, ldh, gate, 0, docid}, stream, m_live);
  return launch(A, lda, W, ldw, M, N, K,
                EpiGatedResidual<true>{bias, h, ldh, gate, mod_stride, docid}, stream, m_live);
}

hipError_t gemm_qkv_rope(const f16* A, int lda, const f16* W, int ldw, const float* bias, int M,
                         int dim, int heads, const int32_t* pos, const float* rope_cos,
                         const float* rope_sin, int rope_dim, int max_pos, f16* q, f16* k,
                         f16* vt, int rp, hipStream_t stream, const int32_t* m_live) {
  (void)heads;
  if (rp < M) return hipErrorInvalidValue;
  if ((long)dim * rp * 2 >= (1L << 31)) return hipErrorInvalidValue;  // q / k buffer offsets
  return launch(A, lda, W, ldw, M, 3 * dim, dim,
                EpiQkvRope{bias, dim, rp, pos, rope_cos, rope_sin, rope_dim, max_pos, q, k, vt, rp},
                stream, m_live);
}

}  // namespace fcv
