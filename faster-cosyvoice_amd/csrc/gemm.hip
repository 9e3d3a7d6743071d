// bf16 MFMA GEMM for gfx950 with fused epilogues.
//
// C[M,N] = A[M,K] . W[N,K]^T, both operands K-contiguous (PyTorch Linear layout), fp32
// accumulation on v_mfma_f32_16x16x32_bf16.  Block tile 128x128x64, 256 threads as a 2x2
// grid of waves, each wave owning a 64x64 sub-tile (4x4 MFMA tiles, 64 accumulator VGPRs).
// Global -> register -> LDS staging with two LDS buffers: the next K tile is fetched into
// registers while the current one feeds the MFMAs, so there is one barrier per K tile.
// LDS rows are padded by 16 bytes so the 16-byte fragment reads of 16 consecutive rows hit
// distinct banks.  Block indices are remapped so that each XCD (blocks are dealt round-robin
// over the 8 XCDs) works on a contiguous range of tiles, N-fastest, which keeps the A rows
// of one M tile inside a single XCD's L2.
#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDSK = BK + 8;
constexpr int kThreads = 256;
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_remap(int bid, int total) {
  int xcd = bid % kXcds, idx = bid / kXcds;
  int base = total / kXcds, extra = total % kXcds;
  return xcd * base + min(xcd, extra) + idx;
}

template <class Epi>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(const bf16* __restrict__ A, int lda,
                                                           const bf16* __restrict__ W, int ldw,
                                                           int M, int N, int K, Epi epi) {
  __shared__ __attribute__((aligned(16))) bf16 sA[2][BM][LDSK];
  __shared__ __attribute__((aligned(16))) bf16 sB[2][BN][LDSK];

  const int n_tiles_n = N / BN;
  const int total = ((M + BM - 1) / BM) * n_tiles_n;
  const int tile = xcd_remap(blockIdx.x, total);
  const int m0 = (tile / n_tiles_n) * BM;
  const int n0 = (tile % n_tiles_n) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave >> 1) * 64;
  const int wn0 = (wave & 1) * 64;

  // global load assignment: 4 chunks of 16 bytes per operand per thread
  const int ld_row = tid >> 3;        // 0..31
  const int ld_k = (tid & 7) * 8;     // element offset inside the K tile
  const bf16* a_src[4];
  const bf16* w_src[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int ar = min(m0 + ld_row + 32 * i, M - 1);
    a_src[i] = A + (long)ar * lda + ld_k;
    w_src[i] = W + (long)(n0 + ld_row + 32 * i) * ldw + ld_k;
  }

  bf16x8 ra[4], rb[4];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = *reinterpret_cast<const bf16x8*>(a_src[i] + kt * BK);
      rb[i] = *reinterpret_cast<const bf16x8*>(w_src[i] + kt * BK);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<bf16x8*>(&sA[buf][ld_row + 32 * i][ld_k]) = ra[i];
      *reinterpret_cast<bf16x8*>(&sB[buf][ld_row + 32 * i][ld_k]) = rb[i];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK;
  fetch(0);
  stash(0);
  __syncthreads();

  const int frag_r = lane & 15;
  const int frag_k = (lane >> 4) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) fetch(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fa[i] = *reinterpret_cast<const bf16x8*>(&sA[cur][wm0 + i * 16 + frag_r][ks * 32 + frag_k]);
        fb[i] = *reinterpret_cast<const bf16x8*>(&sB[cur][wn0 + i * 16 + frag_r][ks * 32 + frag_k]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < KT) stash(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds rows row0 + 0..3 of column col for each 16x16 tile
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row0 = m0 + wm0 + i * 16 + (lane >> 4) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn0 + j * 16 + (lane & 15);
      epi(acc[i][j], row0, col, M);
    }
  }
}

// ---- epilogues ------------------------------------------------------------------------------

struct EpiBiasF32Bf16 {
  const float* bias;
  float* out_f32;
  bf16* out_bf16;
  int ldo;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    const float b = bias[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int row = row0 + r;
      if (row < M) {
        float y = v[r] + b;
        out_f32[(long)row * ldo + col] = y;
        out_bf16[(long)row * ldo + col] = f2bf(y);
      }
    }
  }
};

struct EpiBiasF32 {
  const float* bias;
  float* out;
  int ldo;
  int n_valid;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    if (col >= n_valid) return;
    const float b = bias[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int row = row0 + r;
      if (row < M) out[(long)row * ldo + col] = v[r] + b;
    }
  }
};

struct EpiBiasF32RowMap {
  const float* bias;
  float* out;
  int ldo;
  int n_valid;
  const int32_t* row_map;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    if (col >= n_valid) return;
    const float b = bias[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int row = row0 + r;
      if (row < M) {
        int dst = row_map[row];
        if (dst >= 0) out[(long)dst * ldo + col] = v[r] + b;
      }
    }
  }
};

struct EpiBiasSiluBf16 {
  const float* bias;
  bf16* out;
  int ldo;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    const float b = bias[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int row = row0 + r;
      if (row < M) out[(long)row * ldo + col] = f2bf(silu(v[r] + b));
    }
  }
};

struct EpiBiasGeluBf16 {
  const float* bias;
  bf16* out;
  int ldo;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    const float b = bias[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int row = row0 + r;
      if (row < M) out[(long)row * ldo + col] = f2bf(gelu_tanh(v[r] + b));
    }
  }
};

struct EpiGatedResidual {
  const float* bias;
  float* h;
  int ldh;
  const float* gate;  // mod + gate offset
  long mod_stride;
  const int32_t* docid;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    const float b = bias[col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int row = row0 + r;
      if (row < M) {
        float g = gate[(long)docid[row] * mod_stride + col];
        float* dst = h + (long)row * ldh + col;
        *dst = *dst + g * (v[r] + b);
      }
    }
  }
};

struct EpiQkvRope {
  const float* bias;
  int dim;        // heads * 64
  int rows;       // M (for the q/k row-major stores)
  const int32_t* pos;
  const float* rope_cos;
  const float* rope_sin;
  int rope_dim;
  int max_pos;
  bf16* q;
  bf16* k;
  bf16* vt;
  int rp;
  __device__ void operator()(const f32x4& v, int row0, int col, int M) const {
    const float b = bias[col];
    const int which = col / dim;        // 0 q, 1 k, 2 v (uniform per 16-column tile)
    const int c = col - which * dim;
    const int head = c >> 6, d = c & 63;
    float y[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = v[r] + b;
    // interleaved RoPE: pair (2i, 2i+1) lives in lanes (l, l^1); all lanes shuffle.
    float partner[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) partner[r] = __shfl_xor(y[r], 1, kWave);
    if (which < 2 && c < rope_dim) {
      const int half = rope_dim >> 1;
      const float sign = (c & 1) ? 1.0f : -1.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row = min(row0 + r, M - 1);
        int p = min(pos[row], max_pos - 1);  // pad rows run past the document
        float cs = rope_cos[p * half + (c >> 1)];
        float sn = rope_sin[p * half + (c >> 1)];
        y[r] = y[r] * cs + sign * partner[r] * sn;
      }
    }
    if (which == 2) {
      // V transposed: vt[head][d][row0 .. row0+3] as one 8-byte store (rows < rp always)
      bf16x4 pk = {f2bf(y[0]), f2bf(y[1]), f2bf(y[2]), f2bf(y[3])};
      *reinterpret_cast<bf16x4*>(vt + ((long)head * 64 + d) * rp + row0) = pk;
    } else {
      bf16* dst = (which == 0 ? q : k) + (long)head * rows * 64 + d;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row = row0 + r;
        if (row < M) dst[(long)row * 64] = f2bf(y[r]);
      }
    }
  }
};

template <class Epi>
hipError_t launch(const bf16* A, int lda, const bf16* W, int ldw, int M, int N, int K,
                  const Epi& epi, hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  const int tiles = ((M + BM - 1) / BM) * (N / BN);
  hipLaunchKernelGGL(gemm_kernel<Epi>, dim3(tiles), dim3(kThreads), 0, stream, A, lda, W, ldw, M,
                     N, K, epi);
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
  return launch(A, lda, W, ldw, M, N, K, EpiBiasF32{bias, out, ldo, n_valid}, stream);
}

hipError_t gemm_bias_f32_rowmap(const bf16* A, int lda, const bf16* W, int ldw,
                                const float* bias, int M, int N, int K, float* out, int ldo,
                                int n_valid, const int32_t* row_map, hipStream_t stream) {
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
