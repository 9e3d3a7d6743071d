// bf16 MFMA GEMM for gfx950 with fused epilogues.
//
// C[M,N] = A[M,K] . W[N,K]^T, both operands K-contiguous (PyTorch Linear layout), fp32
// accumulation on v_mfma_f32_32x32x16_bf16 (on this part the 32x32x16 form sustains ~93% of
// the bf16 peak in a register loop, the 16x16x32 form ~54%).
//
// Main loop.  A workgroup of 2x2 waves owns a 128x128 tile; each wave a 64x64 sub-tile of
// 2x2 MFMA tiles.  Operands go straight from global memory into LDS with
// global_load_lds_dwordx4 (no register staging, no ds_write) through a ring of STAGES slices of
// K = 32: while slice k feeds the MFMAs, slices k+1..k+STAGES-1 are in flight.  One wave-level
// load fills 1 KB of LDS = 16 rows x 64 B; the 16-byte chunks of a row sit at position
// chunk ^ ((row >> 2) & 3), so the 16-row fragment reads hit 16 distinct 16-byte bank groups.
// Default 3 stages = 48 KB of LDS per workgroup, three workgroups per CU (measured slightly
// ahead of 4 stages x 2 workgroups: tile epilogues of co-resident workgroups overlap more).
//
// Operand roles are swapped: the MFMA computes D = W_tile . A_tile^T, so the accumulator of a
// 32x32 tile holds, in lane l, output row m = l % 32 and four consecutive output columns per
// register group.  Every epilogue therefore reads and writes 4 consecutive columns of one row
// at a time (16-byte fp32 / 8-byte bf16 vector accesses), and the interleaved RoPE pairs
// (2i, 2i+1) sit in the same lane.
//
// Rasterization: blocks are dealt round-robin over the 8 XCDs, so block ids are first remapped
// to give each XCD a contiguous range of tiles; inside that range tiles are visited in groups of
// GROUP_M M-tiles x all N-tiles (M fastest), keeping the group's A rows and W columns inside
// one XCD's 4 MB L2.
#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int BM = 128, BN = 128, BK = 32;
#ifndef FCV_GEMM_STAGES
#define FCV_GEMM_STAGES 3
#endif
constexpr int STAGES = FCV_GEMM_STAGES;
constexpr int WG_PER_CU = STAGES == 4 ? 2 : 3;
constexpr int kThreads = 256;
constexpr int TM = 2, TN = 2;          // 32x32 MFMA tiles per wave (wave tile 64x64)
constexpr int A_INSTR = BM / 16 / 4;   // 1 KB DMA instructions per wave per slice
constexpr int B_INSTR = BN / 16 / 4;
constexpr int LOADS = A_INSTR + B_INSTR;
constexpr int kXcds = 8;
constexpr int GROUP_M = 8;

__device__ __forceinline__ void tile_coords(int bid, int total, int tiles_m, int tiles_n,
                                            int& tm, int& tn) {
  const int xcd = bid % kXcds, idx = bid / kXcds;
  const int base = total / kXcds, extra = total % kXcds;
  const int t = xcd * base + min(xcd, extra) + idx;
  const int per_group = GROUP_M * tiles_n;
  const int g = t / per_group;
  const int first_m = g * GROUP_M;
  const int gm = min(GROUP_M, tiles_m - first_m);
  const int r = t - g * per_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

// Lane-strided 16-byte global -> LDS copy: lane l writes bytes [16 l, 16 l + 16) of `dst`
// (dst wave-uniform).  Issued as inline asm so the compiler does not treat every later LDS read
// as dependent on it (it would wait for vmcnt(0) before each one); the K loop orders these copies
// with explicit vmcnt waits and barriers instead.
__device__ __forceinline__ void lds_dma16(const bf16* src, bf16* dst) {
  const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)dst;
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(src)
               : "memory", "m0");
}

// s_waitcnt vmcnt(n) (n < 64: bits [3:0] and [15:14]) leaving expcnt / lgkmcnt unconstrained
#define FCV_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

template <class Epi>
__global__ __launch_bounds__(kThreads, WG_PER_CU) void gemm_kernel(const bf16* __restrict__ A, int lda,
                                                           const bf16* __restrict__ W, int ldw,
                                                           int M, int N, int K, Epi epi) {
  __shared__ __attribute__((aligned(1024))) bf16 sA[STAGES][BM * BK];
  __shared__ __attribute__((aligned(1024))) bf16 sB[STAGES][BN * BK];

  const int tiles_n = N / BN;
  const int tiles_m = (M + BM - 1) / BM;
  int tmi, tni;
  tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * BM;
  const int n0 = tni * BN;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave >> 1) * 64;
  const int wn0 = (wave & 1) * 64;

  // per-lane source of each DMA instruction: row r0 + lane/4, swizzled chunk (A rows clamped)
  const int lrow = lane >> 2;
  const bf16* a_src[A_INSTR];
  const bf16* w_src[B_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int row = (wave * A_INSTR + i) * 16 + lrow;
    a_src[i] = A + (long)min(m0 + row, M - 1) * lda + swz(row, lane & 3) * 8;
  }
#pragma unroll
  for (int i = 0; i < B_INSTR; ++i) {
    const int row = (wave * B_INSTR + i) * 16 + lrow;
    w_src[i] = W + (long)(n0 + row) * ldw + swz(row, lane & 3) * 8;
  }
  const int KT = K / BK;
  auto issue = [&](int kt, int stage) {
    const int koff = min(kt, KT - 1) * BK;  // clamped tail copies keep the vmcnt count fixed
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i)
      lds_dma16(a_src[i] + koff, &sA[stage][(wave * A_INSTR + i) * 16 * BK]);
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i)
      lds_dma16(w_src[i] + koff, &sB[stage][(wave * B_INSTR + i) * 16 * BK]);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(s, s);
  const int fr = lane & 31, fh = lane >> 5;
  int stage = 0;
  for (int kt = 0; kt < KT; ++kt) {
    FCV_WAIT_VMCNT((STAGES - 2) * LOADS);  // this wave's copies of slice kt have landed
    __syncthreads();  // ... and every other wave's; slice kt-1 is no longer read
    issue(kt + STAGES - 1, stage == 0 ? STAGES - 1 : stage - 1);
    const bf16* a_st = sA[stage];
    const bf16* b_st = sB[stage];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = ks * 2 + fh;
      bf16x8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm0 + i * 32 + fr;
        fa[i] = *reinterpret_cast<const bf16x8*>(a_st + row * BK + swz(row, chunk) * 8);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn0 + j * 32 + fr;
        fb[j] = *reinterpret_cast<const bf16x8*>(b_st + row * BK + swz(row, chunk) * 8);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(fb[j], fa[i], acc[i][j]);
    }
    stage = stage == STAGES - 1 ? 0 : stage + 1;
  }
  FCV_WAIT_VMCNT(0);  // the clamped tail copies land before the workgroup retires

  // lane: output row m0 + wm0 + 32 i + lane % 32; register group g: columns
  // n0 + wn0 + 32 j + 8 g + 4 (lane / 32) + 0..3
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + wm0 + i * 32 + fr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                         acc[i][j][4 * g + 3]};
        epi(v, row, n0 + wn0 + j * 32 + g * 8 + fh * 4, M);
      }
    }
  }
}

// ---- epilogues: v = C[row][col0 .. col0+3] (col0 % 4 == 0) ----------------------------------

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

struct EpiBiasF32Bf16 {
  const float* bias;
  float* out_f32;
  bf16* out_bf16;
  int ldo;
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    if (row >= M) return;
    const float4 b = ld4(bias + col);
    const float4 y = {v[0] + b.x, v[1] + b.y, v[2] + b.z, v[3] + b.w};
    *reinterpret_cast<float4*>(out_f32 + (long)row * ldo + col) = y;
    *reinterpret_cast<bf16x4*>(out_bf16 + (long)row * ldo + col) =
        bf16x4{f2bf(y.x), f2bf(y.y), f2bf(y.z), f2bf(y.w)};
  }
};

struct EpiBiasF32 {
  const float* bias;
  float* out;
  int ldo;
  int n_valid;  // multiple of 4
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    if (row >= M || col >= n_valid) return;
    const float4 b = ld4(bias + col);
    *reinterpret_cast<float4*>(out + (long)row * ldo + col) =
        float4{v[0] + b.x, v[1] + b.y, v[2] + b.z, v[3] + b.w};
  }
};

struct EpiBiasF32RowMap {
  const float* bias;
  float* out;
  int ldo;
  int n_valid;  // multiple of 4
  const int32_t* row_map;
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    if (row >= M || col >= n_valid) return;
    const int dst = row_map[row];
    if (dst < 0) return;
    const float4 b = ld4(bias + col);
    *reinterpret_cast<float4*>(out + (long)dst * ldo + col) =
        float4{v[0] + b.x, v[1] + b.y, v[2] + b.z, v[3] + b.w};
  }
};

struct EpiBiasSiluBf16 {
  const float* bias;
  bf16* out;
  int ldo;
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    if (row >= M) return;
    const float4 b = ld4(bias + col);
    *reinterpret_cast<bf16x4*>(out + (long)row * ldo + col) =
        bf16x4{f2bf(silu(v[0] + b.x)), f2bf(silu(v[1] + b.y)), f2bf(silu(v[2] + b.z)),
               f2bf(silu(v[3] + b.w))};
  }
};

struct EpiBiasGeluBf16 {
  const float* bias;
  bf16* out;
  int ldo;
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    if (row >= M) return;
    const float4 b = ld4(bias + col);
    *reinterpret_cast<bf16x4*>(out + (long)row * ldo + col) =
        bf16x4{f2bf(gelu_tanh(v[0] + b.x)), f2bf(gelu_tanh(v[1] + b.y)),
               f2bf(gelu_tanh(v[2] + b.z)), f2bf(gelu_tanh(v[3] + b.w))};
  }
};

struct EpiGatedResidual {
  const float* bias;
  float* h;
  int ldh;
  const float* gate;  // mod + gate offset
  long mod_stride;
  const int32_t* docid;
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    if (row >= M) return;
    const float4 b = ld4(bias + col);
    const float4 g = ld4(gate + (long)docid[row] * mod_stride + col);
    float4* dst = reinterpret_cast<float4*>(h + (long)row * ldh + col);
    const float4 x = *dst;
    *dst = float4{x.x + g.x * (v[0] + b.x), x.y + g.y * (v[1] + b.y), x.z + g.z * (v[2] + b.z),
                  x.w + g.w * (v[3] + b.w)};
  }
};

struct EpiQkvRope {
  const float* bias;
  int dim;        // heads * 64
  int rows;       // M (q / k row pitch per head)
  const int32_t* pos;
  const float* rope_cos;
  const float* rope_sin;
  int rope_dim;
  int max_pos;
  bf16* q;
  bf16* k;
  bf16* vt;
  int rp;
  __device__ void operator()(const f32x4& v, int row, int col, int M) const {
    const int which = col / dim;  // 0 q, 1 k, 2 v
    const int c = col - which * dim;
    const int head = c >> 6, d = c & 63;
    const float4 b = ld4(bias + col);
    float y[4] = {v[0] + b.x, v[1] + b.y, v[2] + b.z, v[3] + b.w};
    if (which == 2) {
      // V transposed: vt[head][d + e][row]; rows < rp always (rp covers every M tile)
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[((long)head * 64 + d + e) * rp + row] = f2bf(y[e]);
      return;
    }
    if (row >= M) return;
    if (c < rope_dim) {
      // interleaved pairs (d, d+1), (d+2, d+3): (a, b) -> (a cos - b sin, b cos + a sin)
      const int p = min(pos[row], max_pos - 1);  // pad rows run past the document
      const int half = rope_dim >> 1;
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const float cs = rope_cos[p * half + ((c + e) >> 1)];
        const float sn = rope_sin[p * half + ((c + e) >> 1)];
        const float a = y[e], bb = y[e + 1];
        y[e] = a * cs - bb * sn;
        y[e + 1] = bb * cs + a * sn;
      }
    }
    bf16* dst = (which == 0 ? q : k) + ((long)head * rows + row) * 64 + d;
    *reinterpret_cast<bf16x4*>(dst) = bf16x4{f2bf(y[0]), f2bf(y[1]), f2bf(y[2]), f2bf(y[3])};
  }
};

template <class Epi>
hipError_t launch(const bf16* A, int lda, const bf16* W, int ldw, int M, int N, int K,
                  const Epi& epi, hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  if (N % BN != 0 || K % BK != 0 || lda % 8 != 0 || ldw % 8 != 0) return hipErrorInvalidValue;
  const int tiles = ((M + BM - 1) / BM) * (N / BN);
  hipLaunchKernelGGL((gemm_kernel<Epi>), dim3(tiles), dim3(kThreads), 0, stream, A, lda, W, ldw,
                     M, N, K, epi);
  return hipGetLastError();
}

}  // namespace

hipError_t gemm_bias_f32_bf16(const bf16* A, int lda, const bf16* W, int ldw, const float* bias,
                              int M, int N, int K, float* out_f32, bf16* out_bf16, int ldo,
                              hipStream_t stream) {
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32Bf16{bias, out_f32, out_bf16, ldo}, stream);
}

hipError_t gemm_bias_f32(const bf16* A, int lda, const bf16* W, int ldw, const float* bias,
                         int M, int N, int K, float* out, int ldo, int n_valid,
                         hipStream_t stream) {
  if (n_valid % 4 != 0) return hipErrorInvalidValue;
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32{bias, out, ldo, n_valid}, stream);
}

hipError_t gemm_bias_f32_rowmap(const bf16* A, int lda, const bf16* W, int ldw,
                                const float* bias, int M, int N, int K, float* out, int ldo,
                                int n_valid, const int32_t* row_map, hipStream_t stream) {
  if (n_valid % 4 != 0) return hipErrorInvalidValue;
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32RowMap{bias, out, ldo, n_valid, row_map},
                stream);
}

hipError_t gemm_bias_silu_bf16(const bf16* A, int lda, const bf16* W, int ldw, const float* bias,
                               int M, int N, int K, bf16* out, int ldo, hipStream_t stream) {
  return launch(A, lda, W, ldw, M, N, K, EpiBiasSiluBf16{bias, out, ldo}, stream);
}

hipError_t gemm_bias_gelu_bf16(const bf16* A, int lda, const bf16* W, int ldw, const float* bias,
                               int M, int N, int K, bf16* out, int ldo, hipStream_t stream) {
  return launch(A, lda, W, ldw, M, N, K, EpiBiasGeluBf16{bias, out, ldo}, stream);
}

hipError_t gemm_gated_residual(const bf16* A, int lda, const bf16* W, int ldw, const float* bias,
                               int M, int N, int K, float* h, int ldh, const float* gate,
                               long mod_stride, const int32_t* docid, hipStream_t stream) {
  return launch(A, lda, W, ldw, M, N, K,
                EpiGatedResidual{bias, h, ldh, gate, mod_stride, docid}, stream);
}

hipError_t gemm_qkv_rope(const bf16* A, int lda, const bf16* W, int ldw, const float* bias, int M,
                         int dim, int heads, const int32_t* pos, const float* rope_cos,
                         const float* rope_sin, int rope_dim, int max_pos, bf16* q, bf16* k,
                         bf16* vt, int rp, hipStream_t stream) {
  (void)heads;
  return launch(A, lda, W, ldw, M, 3 * dim, dim,
                EpiQkvRope{bias, dim, M, pos, rope_cos, rope_sin, rope_dim, max_pos, q, k, vt, rp},
                stream);
}

}  // namespace fcv
