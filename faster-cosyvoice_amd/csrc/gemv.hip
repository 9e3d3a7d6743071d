// Skinny products out[m, n] = f(sum_k W[n, k] a[m, k] + bias[n]) for rows of a that share
// one W: the timestep MLP and the AdaLN projection, whose time is reading W (the concatenated
// AdaLN weights are 137216 x 1024 f16 = 281 MB per evaluation).  Bandwidth-bound, so no MFMA:
// one wave owns 4 rows of W; lane l reads k in [8l, 8l + 8) of every 512-wide k block, so each
// load instruction covers 1 KB of one W row contiguously.  A launch takes up to 16 rows of a,
// in chunks of up to 4 against the W rows held in registers; each chunk's 4 x 4 partial sums
// are reduced together across the wave (reduce16) and written by the lanes holding them.  More rows take more launches of
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

struct GemvSiluF16 {
  const float* bias;
  f16* out;
  int ldo;
  __device__ void operator()(int m, int n, float s) const {
    out[(long)m * ldo + n] = f2h(silu(s + bias[n]));
  }
};

// Wave sums of 16 values at once: halving exchanges (xor 32, 16, 8, 4: a lane keeps half of its
// values, adds the partner's copies of them and hands over the other half), then a butterfly
// over the last 4 lanes; lane 4 j returns the full sum of value j (15 + 2 exchanges instead of
// 16 x 6).
template <int H>
__device__ __forceinline__ void halve(float (&p)[16], bool upper, int mask) {
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float send = upper ? p[i] : p[i + H];
    const float keep = upper ? p[i + H] : p[i];
    p[i] = keep + __shfl_xor(send, mask);
  }
}
__device__ __forceinline__ float reduce16(float (&p)[16], int lane) {
  halve<8>(p, lane & 32, 32);
  halve<4>(p, lane & 16, 16);
  halve<2>(p, lane & 8, 8);
  halve<1>(p, lane & 4, 4);
  float t = p[0];
  t += __shfl_xor(t, 2);
  t += __shfl_xor(t, 1);
  return t;
}

// K % 512 == 0: lane l holds k = 512 b + 8 l + 0..7 for each of the K / 512 blocks b.  MM rows
// of a per chunk; ceil(M / MM) chunks.
template <int K, int MM, class Epi>
__global__ __launch_bounds__(256) void gemv_kernel(const f16* __restrict__ a, int lda,
                                                   const f16* __restrict__ W, int ldw, int M,
                                                   int N, Epi epi) {
  constexpr int KB = K / 512;
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kGemvRows;
  if (n0 >= N) return;
  f16x8 wv[kGemvRows][KB];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
    for (int b = 0; b < KB; ++b)
      wv[r][b] = *reinterpret_cast<const f16x8*>(W + (long)min(n0 + r, N - 1) * ldw + 512 * b +
                                                  8 * lane);
  for (int m0 = 0; m0 < M; m0 += MM) {
    float av[MM][KB][8];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const f16x8 v = m0 + m < M
                             ? *reinterpret_cast<const f16x8*>(a + (long)(m0 + m) * lda + 512 * b + 8 * lane)
                             : f16x8{};
#pragma unroll
        for (int e = 0; e < 8; ++e) av[m][b][e] = h2f(v[e]);
      }
    // partial sums, value v = r * MM + m, padded to 16 values
    float p[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) p[v] = 0.0f;
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
          for (int e = 0; e < 8; ++e) s = fmaf(h2f(wv[r][b][e]), av[m][b][e], s);
        p[r * MM + m] = s;
      }
    // lane 4 j ends with the full sum of value j
    const float t = reduce16(p, lane);
    const int v = lane >> 2, r = v / MM, m = v % MM;
    if ((lane & 3) == 0 && v < kGemvRows * MM && m0 + m < M && n0 + r < N) epi(m0 + m, n0 + r, t);
  }
}

template <int K, class Epi>
hipError_t launch_gemv_k(const f16* a, int lda, const f16* W, int ldw, int M, int N,
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
hipError_t launch_gemv(const f16* a, int lda, const f16* W, int ldw, int M, int N, int K,
                       const Epi& epi, hipStream_t stream) {
  if (K == 1024) return launch_gemv_k<1024>(a, lda, W, ldw, M, N, epi, stream);
  if (K == 512) return launch_gemv_k<512>(a, lda, W, ldw, M, N, epi, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool gemv_supported(int M, int K, int lda, int ldw) {
  return M >= 1 && (K == 1024 || K == 512) && lda % 8 == 0 && ldw % 8 == 0;
}

hipError_t gemv_bias_f32(const f16* a, int lda, const f16* W, int ldw, const float* bias, int M,
                         int N, int K, float* out, int ldo, hipStream_t stream) {
  if (!gemv_supported(M, K, lda, ldw)) return hipErrorInvalidValue;
  for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
    const hipError_t e = launch_gemv(a + (long)m0 * lda, lda, W, ldw, min(kGemvMaxM, M - m0), N, K,
                                     GemvF32{bias, out + (long)m0 * ldo, ldo}, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t gemv_bias_silu_f16(const f16* a, int lda, const f16* W, int ldw, const float* bias,
                               int M, int N, int K, f16* out, int ldo, hipStream_t stream) {
  if (!gemv_supported(M, K, lda, ldw)) return hipErrorInvalidValue;
  for (int m0 = 0; m0 < M; m0 += kGemvMaxM) {
    const hipError_t e = launch_gemv(a + (long)m0 * lda, lda, W, ldw, min(kGemvMaxM, M - m0), N, K,
                                     GemvSiluF16{bias, out + (long)m0 * ldo, ldo}, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace fcv
