// Skinny products out[m, n] = f(sum_k W[n, k] a[m, k] + bias[n]) for rows of a that share
// one W: the timestep MLP and the AdaLN projection, whose time is reading W (the concatenated
// AdaLN weights are 137216 x 1024 bf16 = 281 MB per evaluation).  Bandwidth-bound, so no MFMA:
// one wave owns 4 rows of W; lane l reads k in [8l, 8l + 8) of every 512-wide k block, so each
// load instruction covers 1 KB of one W row contiguously.  A launch takes up to 16 rows of a,
// in chunks of up to 4 against the W rows held in registers; each chunk's 4 x 4 partial sums
// are reduced with cross-lane shuffles and written by lane 0.  More rows take more launches of
// 16.  Every output element is summed in the same order whatever M is, so a row's result does
// not depend on how many rows share the call (one shared t, one t per document, or the t
// values of a solver's steps all give a t the same modulation row, bit for bit).
#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int kGemvRows = 4;   // W rows per wave
constexpr int kGemvMaxM = 16;  // rows of a per launch (in chunks of up to 4)

struct GemvF32 {
  const float* bias;
  float* out;
  int ldo;
  __device__ void operator()(int m, int n, float s) const { out[(long)m * ldo + n] = s + bias[n]; }
};

struct GemvSiluBf16 {
  const float* bias;
  bf16* out;
  int ldo;
  __device__ void operator()(int m, int n, float s) const {
    out[(long)m * ldo + n] = f2bf(silu(s + bias[n]));
  }
};

// K % 512 == 0: lane l holds k = 512 b + 8 l + 0..7 for each of the K / 512 blocks b.  MM rows
// of a per chunk; ceil(M / MM) chunks.
template <int K, int MM, class Epi>
__global__ __launch_bounds__(256) void gemv_kernel(const bf16* __restrict__ a, int lda,
                                                   const bf16* __restrict__ W, int ldw, int M,
                                                   int N, Epi epi) {
  constexpr int KB = K / 512;
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kGemvRows;
  if (n0 >= N) return;
  bf16x8 wv[kGemvRows][KB];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
    for (int b = 0; b < KB; ++b)
      wv[r][b] = *reinterpret_cast<const bf16x8*>(W + (long)min(n0 + r, N - 1) * ldw + 512 * b +
                                                  8 * lane);
  for (int m0 = 0; m0 < M; m0 += MM) {
    float av[MM][KB][8];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const bf16x8 v = m0 + m < M
                             ? *reinterpret_cast<const bf16x8*>(a + (long)(m0 + m) * lda + 512 * b + 8 * lane)
                             : bf16x8{};
#pragma unroll
        for (int e = 0; e < 8; ++e) av[m][b][e] = bf2f(v[e]);
      }
    float acc[kGemvRows][MM];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
          for (int e = 0; e < 8; ++e) s = fmaf(bf2f(wv[r][b][e]), av[m][b][e], s);
        acc[r][m] = wave_sum(s);
      }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m)
          if (m0 + m < M && n0 + r < N) epi(m0 + m, n0 + r, acc[r][m]);
    }
  }
}

template <int K, class Epi>
hipError_t launch_gemv_k(const bf16* a, int lda, const bf16* W, int ldw, int M, int N,
                         const Epi& epi, hipStream_t stream) {
  const unsigned blocks = (unsigned)((N + 4 * kGemvRows - 1) / (4 * kGemvRows));
  if (M == 1)
    hipLaunchKernelGGL((gemv_kernel<K, 1, Epi>), dim3(blocks), dim3(256), 0, stream, a, lda, W,
                       ldw, M, N, epi);
  else if (M == 2)
    hipLaunchKernelGGL((gemv_kernel<K, 2, Epi>), dim3(blocks), dim3(256), 0, stream, a, lda, W,
                       ldw, M, N, epi);
  else
    hipLaunchKernelGGL((gemv_kernel<K, 4, Epi>), dim3(blocks), dim3(256), 0, stream, a, lda, W,
                       ldw, M, N, epi);
  return hipGetLastError();
}

template <class Epi>
hipError_t launch_gemv(const bf16* a, int lda, const bf16* W, int ldw, int M, int N, int K,
                       const Epi& epi, hipStream_t stream) {
  if (K == 1024) return launch_gemv_k<1024>(a, lda, W, ldw, M, N, epi, stream);
  if (K == 512) return launch_gemv_k<512>(a, lda, W, ldw, M, N, epi, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool gemv_supported(int M, int K, int lda, int ldw) {
  return M >= 1 && (K == 1024 || K == 512) && lda % 8 == 0 && ldw % 8 == 0;
}

hipError_t gemv_bias_f32(const bf16* a, int lda, const bf16* W, int ldw, const float* bias, int M,
                         int N, int K, float* out, int ldo, hipStream_t stream) {
  if (!gemv_supported(M, K, lda, ldw)) return hipErrorInvalidValue;
  for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
    const hipError_t e = launch_gemv(a + (long)m0 * lda, lda, W, ldw, min(kGemvMaxM, M - m0), N, K,
                                     GemvF32{bias, out + (long)m0 * ldo, ldo}, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t gemv_bias_silu_bf16(const bf16* a, int lda, const bf16* W, int ldw, const float* bias,
                               int M, int N, int K, bf16* out, int ldo, hipStream_t stream) {
  if (!gemv_supported(M, K, lda, ldw)) return hipErrorInvalidValue;
  for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
    const hipError_t e = launch_gemv(a + (long)m0 * lda, lda, W, ldw, min(kGemvMaxM, M - m0), N, K,
                                     GemvSiluBf16{bias, out + (long)m0 * ldo, ldo}, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace fcv
