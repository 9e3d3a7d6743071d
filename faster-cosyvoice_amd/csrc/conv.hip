// Causal grouped conv1d + Mish (CausalConvPositionEmbedding) as an implicit GEMM on MFMA.
//
// Per (row tile of 128 frames, group g of 64 channels):
//   y[r, co] = mish(bias[co] + sum_{j<taps} sum_{ci<64} W[g][j][co][ci] * x[r - (taps-1) + j, ci])
// The 128 + taps - 1 input rows of the group's 64 channels are staged in LDS once; every tap
// j reads the same window shifted by j rows, so no im2col buffer exists.  Each tap's 64x64
// weight slice streams through an LDS double buffer.  Packed documents are handled per row:
// the input fragment of output row r at tap j is zeroed when the input row lies before r's
// document start, i.e. when pos[r] + j < taps - 1 (the per-document left zero padding of
// the reference's F.pad).
#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int TM = 128;       // output rows per workgroup
constexpr int CG = 64;        // channels per group
constexpr int LDP = CG + 8;   // padded LDS row (f16): 16 consecutive rows hit distinct banks
constexpr int MAX_TAPS = 31;
constexpr int WIN = TM + MAX_TAPS - 1;
constexpr int SPITCH = CG + 4;  // fp32 staging row
constexpr int X_BYTES = WIN * LDP * 2;
constexpr int W_BYTES = 2 * CG * LDP * 2;
constexpr int STAGE_BYTES = 4 * 32 * SPITCH * 4;
constexpr int SMEM_BYTES = X_BYTES + W_BYTES > STAGE_BYTES ? X_BYTES + W_BYTES : STAGE_BYTES;

// 4 waves x 32 output rows x 64 output channels; MFMA 32x32x16 with the weights as the A
// operand, so lane l accumulates output row l % 32 and, in register group g of channel tile t,
// channels 32 t + 8 g + 4 (l / 32) + 0..3.  The epilogue stages each wave's 32 x 64 block
// through LDS and reads it back row-major (16 lanes per row), so stores are contiguous runs of
// 128 B (f16 out) or 256 B (fp32 residual); the residual form issues all its h loads before
// its first store.
__global__ __launch_bounds__(256, 2) void conv_kernel(const f16* __restrict__ x, int C,
                                                      const f16* __restrict__ w,
                                                      const float* __restrict__ bias, int taps,
                                                      const int32_t* __restrict__ pos, int rows,
                                                      f16* __restrict__ out_f16,
                                                      float* __restrict__ h,
                                                      const int32_t* __restrict__ rows_live) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM_BYTES];
  f16 (*sX)[LDP] = reinterpret_cast<f16 (*)[LDP]>(smem);
  f16 (*sW)[CG][LDP] = reinterpret_cast<f16 (*)[CG][LDP]>(smem + X_BYTES);

  if (rows_live) rows = *rows_live;  // live rows of a capacity-sized grid
  const int m0 = blockIdx.x * TM;
  if (m0 >= rows) return;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int halo = taps - 1;

  // stage the input window rows [m0 - halo, m0 + TM) of group g
  const int chunk_c = (tid & 7) * 8;
  for (int r = tid >> 3; r < TM + halo; r += 32) {
    int src = min(max(m0 - halo + r, 0), rows - 1);
    *reinterpret_cast<f16x8*>(&sX[r][chunk_c]) =
        *reinterpret_cast<const f16x8*>(x + (long)src * C + g * CG + chunk_c);
  }

  const f16* wg = w + (long)g * taps * CG * CG;
  const int lw_r = tid >> 3;  // 0..31
  auto fetch = [&](f16x8 (&rw)[2], int j) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      rw[i] = *reinterpret_cast<const f16x8*>(wg + ((long)j * CG + lw_r + 32 * i) * CG + chunk_c);
  };
  auto stash = [&](const f16x8 (&rw)[2], int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<f16x8*>(&sW[buf][lw_r + 32 * i][chunk_c]) = rw[i];
  };

  // output row of this lane (B operand row) and its document position
  const int fr = lane & 31, fh = lane >> 5;
  const int lrow = wave * 32 + fr;
  const int lpos = pos[min(m0 + lrow, rows - 1)];
  const int col_lane = (lane & 15) * 4;  // epilogue: 4 channels of one row per lane
  const float4 bias4 = *reinterpret_cast<const float4*>(bias + g * CG + col_lane);

  f32x16 acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;

  const f16x8 zero8 = {};
  auto tap = [&](int j, int buf) {
    // rows before the row's document start read as zero (per-document causal padding)
    const bool live = lpos + j >= halo;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(&sX[lrow + j][ks * 16 + fh * 8]);
      const f16x8 xb = live ? v : zero8;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f16x8 wa = *reinterpret_cast<const f16x8*>(&sW[buf][t * 32 + fr][ks * 16 + fh * 8]);
        acc[t] = mfma32(wa, xb, acc[t]);
      }
    }
  };
  // Weights run two taps ahead of the MFMAs: tap j+1's slice (loaded during tap j-1) is stashed
  // while tap j+2's loads are in flight, so a stash never waits on loads issued in its own tap
  // (a workgroup alone on its CU would otherwise wait out a load round trip every tap).  Taps
  // past the last re-read the last slice, so every path issues the same loads.
  f16x8 ra[2], rb[2];
  fetch(ra, 0);
  stash(ra, 0);
  fetch(ra, min(1, taps - 1));
  __syncthreads();
  for (int j = 0; j < taps; j += 2) {
    fetch(rb, min(j + 2, taps - 1));
    __builtin_amdgcn_sched_barrier(0);
    tap(j, 0);
    stash(ra, 1);
    __syncthreads();
    if (j + 1 < taps) {
      fetch(ra, min(j + 3, taps - 1));
      __builtin_amdgcn_sched_barrier(0);
      tap(j + 1, 1);
      stash(rb, 0);
      __syncthreads();
    }
  }

  // epilogue (the loop's last barrier freed the window and weight buffers)
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * SPITCH;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f32x4*>(stage + fr * SPITCH + t * 32 + q * 8 + fh * 4) =
          f32x4{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int col = g * CG + col_lane;
  f32x4 v[8];
  float4 hv[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int r = p * 4 + (lane >> 4);
    v[p] = *reinterpret_cast<const f32x4*>(stage + r * SPITCH + col_lane);
    const int row = min(m0 + wave * 32 + r, rows - 1);
    if (h) hv[p] = *reinterpret_cast<const float4*>(h + (long)row * C + col);
  }
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int row = m0 + wave * 32 + p * 4 + (lane >> 4);
    const float4 y = {mish(v[p][0] + bias4.x), mish(v[p][1] + bias4.y), mish(v[p][2] + bias4.z),
                      mish(v[p][3] + bias4.w)};
    if (h) {
      const float4 r4 = {hv[p].x + y.x, hv[p].y + y.y, hv[p].z + y.z, hv[p].w + y.w};
      if (row < rows) *reinterpret_cast<float4*>(h + (long)row * C + col) = r4;
    } else {
      const f16x4 yb = f2h4(y.x, y.y, y.z, y.w);
      if (row < rows) *reinterpret_cast<f16x4*>(out_f16 + (long)row * C + col) = yb;
    }
  }
}

}  // namespace

hipError_t conv_causal_mish(const f16* x, int C, const f16* w, const float* bias, int taps,
                            const int32_t* pos, int rows, f16* out_f16, float* h,
                            hipStream_t stream, const int32_t* rows_live) {
  if (rows <= 0) return hipSuccess;
  if (taps < 1 || taps > MAX_TAPS || C % CG != 0) return hipErrorInvalidValue;
  dim3 grid((rows + TM - 1) / TM, C / CG);
  hipLaunchKernelGGL(conv_kernel, grid, dim3(256), 0, stream, x, C, w, bias, taps, pos, rows,
                     out_f16, h, rows_live);
  return hipGetLastError();
}

}  // namespace fcv
