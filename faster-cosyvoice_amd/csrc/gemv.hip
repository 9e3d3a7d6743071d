// Skinny products out[m, n] = f(sum_k W[n, k] a[m, k] + bias[n]) for rows of a that share
// one W: the timestep MLP and the AdaLN projection (and, at the end of this file, the
// LayerNorm fold's column terms), whose time is reading W (the concatenated
// AdaLN weights are 137216 x 1024 bf16 = 281 MB per evaluation).  Bandwidth-bound, so no MFMA:
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

struct GemvSiluBf16 {
  const float* bias;
  bf16* out;
  int ldo;
  __device__ void operator()(int m, int n, float s) const {
    out[(long)m * ldo + n] = f2bf(silu(s + bias[n]));
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
          for (int e = 0; e < 8; ++e) s = fmaf(bf2f(wv[r][b][e]), av[m][b][e], s);
        p[r * MM + m] = s;
      }
    // lane 4 j ends with the full sum of value j
    const float t = reduce16(p, lane);
    const int v = lane >> 2, r = v / MM, m = v % MM;
    if ((lane & 3) == 0 && v < kGemvRows * MM && m0 + m < M && n0 + r < N) epi(m0 + m, n0 + r, t);
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

// ---- LayerNorm fold column terms (adaln_fold) ------------------------------------------
// One wave per kFoldRows rows of W (a block's QKV rows, then its FF1 rows), converted to fp32
// in registers; lane l holds k = 512 b + 8 l + 0..7.  For each modulation row a wave forms
// 2 kFoldRows partial dot products (each W row against g and against shift) and reduces them
// together (reduce16): lane 4 i ends with the full sum of value i.  (Staging the g and shift
// rows in LDS once per workgroup measured slower: 166 against 135 us for 10 rows.)
constexpr int kFoldRows = 8;
constexpr int kFoldDim = 1024;
static_assert(2 * kFoldRows == 16, "reduce16 takes 16 values");

__global__ __launch_bounds__(256) void adaln_fold_kernel(
    const bf16* __restrict__ qkv_w, const float* __restrict__ qkv_b, const bf16* __restrict__ ff1_w,
    const float* __restrict__ ff1_b, int depth, int ff_dim, const float* __restrict__ mod,
    long mod_width, int n_t, float* __restrict__ fold) {
  constexpr int D = kFoldDim;
  const int lane = threadIdx.x & 63;
  const int waves_per_block = (3 * D + ff_dim) / kFoldRows;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gw >= depth * waves_per_block) return;
  const int l = gw / waves_per_block;
  const int r0 = (gw - l * waves_per_block) * kFoldRows;  // row of [QKV rows | FF1 rows]
  const bool att = r0 < 3 * D;
  const int rf = r0 - 3 * D;
  const bf16* W = att ? qkv_w + ((long)l * 3 * D + r0) * D : ff1_w + ((long)l * ff_dim + rf) * D;
  const float* bias = att ? qkv_b + (long)l * 3 * D + r0 : ff1_b + (long)l * ff_dim + rf;
  const long per_block = 6L * D + 2L * ff_dim;
  const long u_off = att ? r0 : 6L * D + rf;
  const long v_off = att ? 3L * D + r0 : 6L * D + ff_dim + rf;
  const int g_off = att ? D : 4 * D, s_off = att ? 0 : 3 * D;

  float w[kFoldRows][16];
#pragma unroll
  for (int r = 0; r < kFoldRows; ++r)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(W + (long)r * D + 512 * b + 8 * lane);
#pragma unroll
      for (int e = 0; e < 8; ++e) w[r][8 * b + e] = bf2f(v[e]);
    }
  for (int s = 0; s < n_t; ++s) {
    const float* mrow = mod + s * mod_width + (long)l * 6 * D;
    float g[16], sh[16];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 gv = *reinterpret_cast<const float4*>(mrow + g_off + 512 * b + 8 * lane + 4 * h);
        const float4 sv = *reinterpret_cast<const float4*>(mrow + s_off + 512 * b + 8 * lane + 4 * h);
        const int e = 8 * b + 4 * h;
        g[e] = gv.x, g[e + 1] = gv.y, g[e + 2] = gv.z, g[e + 3] = gv.w;
        sh[e] = sv.x, sh[e + 1] = sv.y, sh[e + 2] = sv.z, sh[e + 3] = sv.w;
      }
    float p[2 * kFoldRows];
#pragma unroll
    for (int r = 0; r < kFoldRows; ++r) {
      float a = 0.0f, c = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        a = fmaf(w[r][e], g[e], a);
        c = fmaf(w[r][e], sh[e], c);
      }
      p[2 * r] = a;
      p[2 * r + 1] = c;
    }
    const float t = reduce16(p, lane);
    if ((lane & 3) == 0) {
      const int vi = lane >> 2, r = vi >> 1;
      float* out = fold + ((long)s * depth + l) * per_block;
      if (vi & 1)
        out[v_off + r] = t + bias[r];
      else
        out[u_off + r] = t;
    }
  }
}

}  // namespace

hipError_t adaln_fold(const bf16* qkv_w, const float* qkv_b, const bf16* ff1_w,
                      const float* ff1_b, int depth, int dim, int ff_dim, const float* mod,
                      long mod_width, int n_t, float* fold, hipStream_t stream) {
  if (dim != kFoldDim || ff_dim % kFoldRows != 0 || depth < 1 || n_t < 1 ||
      mod_width < 6L * dim * depth || mod_width % 4 != 0)
    return hipErrorInvalidValue;
  const long waves = (long)depth * ((3 * dim + ff_dim) / kFoldRows);
  hipLaunchKernelGGL(adaln_fold_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream,
                     qkv_w, qkv_b, ff1_w, ff1_b, depth, ff_dim, mod, mod_width, n_t, fold);
  return hipGetLastError();
}

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
