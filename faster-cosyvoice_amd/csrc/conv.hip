// Causal grouped conv1d + Mish (CausalConvPositionEmbedding) as an implicit GEMM on MFMA.
//
// Per (row tile of 128 frames, group g of 64 channels):
//   y[r, co] = mish(bias[co] + sum_{j<taps} sum_{ci<64} W[g][j][co][ci] * x[r - (taps-1) + j, ci])
// The 128 + taps - 1 input rows of the group's 64 channels are staged in LDS once; every tap
// j reads the same window shifted by j rows, so no im2col buffer exists.  Each tap's 64x64
// weight slice streams through an LDS double buffer.  Packed documents are handled per row:
// the A fragment of output row r at tap j is zeroed when the input row lies before r's
// document start, i.e. when pos[r] + j < taps - 1 (the per-document left zero padding of
// the reference's F.pad).  4 waves x 32 rows x 64 output channels, MFMA 16x16x32 bf16.
#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int TM = 128;       // output rows per workgroup
constexpr int CG = 64;        // channels per group
constexpr int LDP = CG + 8;   // padded LDS row
constexpr int MAX_TAPS = 31;
constexpr int WIN = TM + MAX_TAPS - 1;

__global__ __launch_bounds__(256, 2) void conv_kernel(const bf16* __restrict__ x, int C,
                                                      const bf16* __restrict__ w,
                                                      const float* __restrict__ bias, int taps,
                                                      const int32_t* __restrict__ pos, int rows,
                                                      bf16* __restrict__ out_bf16,
                                                      float* __restrict__ h) {
  __shared__ __attribute__((aligned(16))) bf16 sX[WIN][LDP];
  __shared__ __attribute__((aligned(16))) bf16 sW[2][CG][LDP];

  const int m0 = blockIdx.x * TM;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int halo = taps - 1;

  // stage the input window rows [m0 - halo, m0 + TM) of group g
  const int chunk_c = (tid & 7) * 8;
  for (int r = tid >> 3; r < TM + halo; r += 32) {
    int src = min(max(m0 - halo + r, 0), rows - 1);
    *reinterpret_cast<bf16x8*>(&sX[r][chunk_c]) =
        *reinterpret_cast<const bf16x8*>(x + (long)src * C + g * CG + chunk_c);
  }

  const bf16* wg = w + (long)g * taps * CG * CG;
  const int lw_r = tid >> 3;  // 0..31
  bf16x8 rw[2];
  auto fetch = [&](int j) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      rw[i] = *reinterpret_cast<const bf16x8*>(wg + ((long)j * CG + lw_r + 32 * i) * CG + chunk_c);
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<bf16x8*>(&sW[buf][lw_r + 32 * i][chunk_c]) = rw[i];
  };

  // rows owned by this lane in its two 16-row MFMA tiles
  const int fr = lane & 15;
  const int fk = (lane >> 4) * 8;
  int lrow[2], lpos[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    lrow[mt] = wave * 32 + mt * 16 + fr;  // row inside the tile
    lpos[mt] = pos[min(m0 + lrow[mt], rows - 1)];
  }

  f32x4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  fetch(0);
  stash(0);
  __syncthreads();
  const bf16x8 zero8 = {};
  for (int j = 0; j < taps; ++j) {
    const int cur = j & 1;
    if (j + 1 < taps) fetch(j + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 fa[2], fb[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        bf16x8 v = *reinterpret_cast<const bf16x8*>(&sX[lrow[mt] + j][ks * 32 + fk]);
        fa[mt] = (lpos[mt] + j >= halo) ? v : zero8;
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        fb[nt] = *reinterpret_cast<const bf16x8*>(&sW[cur][nt * 16 + fr][ks * 32 + fk]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mfma16(fa[mt], fb[nt], acc[mt][nt]);
    }
    if (j + 1 < taps) stash(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int row0 = m0 + wave * 32 + mt * 16 + (lane >> 4) * 4;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = g * CG + nt * 16 + fr;
      const float b = bias[col];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + r;
        if (row >= rows) continue;
        const float y = mish(acc[mt][nt][r] + b);
        if (out_bf16) out_bf16[(long)row * C + col] = f2bf(y);
        if (h) h[(long)row * C + col] += y;
      }
    }
  }
}

}  // namespace

hipError_t conv_causal_mish(const bf16* x, int C, const bf16* w, const float* bias, int taps,
                            const int32_t* pos, int rows, bf16* out_bf16, float* h,
                            hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (taps < 1 || taps > MAX_TAPS || C % CG != 0) return hipErrorInvalidValue;
  dim3 grid((rows + TM - 1) / TM, C / CG);
  hipLaunchKernelGGL(conv_kernel, grid, dim3(256), 0, stream, x, C, w, bias, taps, pos, rows,
                     out_bf16, h);
  return hipGetLastError();
}

}  // namespace fcv
