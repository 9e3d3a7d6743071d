// HiFT vocoder kernels on gfx950 (see hift.hpp for the layout and the launch contracts).
//
// Every convolution of the vocoder -- the fp64 F0 predictor, conv_pre, the upsampling convs,
// the strided source convs, the resblock convs and conv_post -- is one implicit GEMM on the
// matrix cores (v_mfma_{f32,f64}_16x16x4): weights are the A operand (rows = output channels),
// the gathered input rows the B operand, so a lane's four accumulators are four channels of one
// time step (consecutive in fp32; four apart in fp64, whose 16x16 result is laid out by rows
// 4 e + lane / 16).  Operands go through LDS K-contiguous, 32 (or 16) input channels of one tap
// per chunk, with a register-prefetched double buffer.  A workgroup owns 64 time rows x 64
// output channels (32 x 32 in launches too small to give every CU a 64 x 64 tile).  Activations that sit between two convolutions are fused: LeakyReLU into the
// input prologue, bias, ELU, residual add, Snake and the resblock mean into the epilogue, and
// the epilogue can also write Snake(y) as a second output for the next conv.
#include <math.h>

#include <cstdlib>

#include "hift.hpp"

namespace fcv {
namespace {

constexpr int kTileR = 64;  // time rows per workgroup
constexpr int kTileC = 64;  // output channels per workgroup
constexpr long kSmallTileBelow = 256;  // 64x64 tiles per launch under which 32x32 tiles run

typedef double f64x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Vec4;
template <> struct Vec4<float> { using type = f32x4; };
template <> struct Vec4<double> { using type = f64x4; };

__device__ __forceinline__ f32x4 mfma_16x16x4(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f64x4 mfma_16x16x4(double a, double b, const f64x4& c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// largest d with cu[d] <= row
__device__ __forceinline__ int doc_of(const int32_t* cu, int n_docs, int row) {
  int lo = 0, hi = n_docs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Snake(x) = x + sin(a x)^2 / (a + 1e-9), with inv = 1 / (a + 1e-9) precomputed in fp32.
// sin by v_sin_f32 on the fractional part of the argument in turns (v_fract_f32 is exact).
__device__ __forceinline__ float snake(float x, float a, float inv) {
  const float turns = (x * a) * 0.15915494309189535f;
  const float s = __builtin_amdgcn_sinf(__builtin_amdgcn_fractf(turns));
  return x + inv * (s * s);
}

template <typename T>
__device__ __forceinline__ T elu(T x) { return x > T(0) ? x : T(expm1(x)); }

// epilogue of one output element (row, channel c) from its accumulator value
template <typename T>
__device__ __forceinline__ void conv_store1(const HiftConv& p, long row, int c, T acc) {
  T v = acc + static_cast<const T*>(p.bias)[c];
  if constexpr (sizeof(T) == 8) {
    if (p.elu) v = elu(v);
  }
  const long i = row * p.ldo + c;
  if (p.add) v = v + static_cast<const T*>(p.add)[row * p.ld_add + c];
  if (p.mode == HIFT_ACC_ADD) v = static_cast<const T*>(p.accin)[i] + v;
  if (p.mode == HIFT_ACC_ADD_DIV) v = (static_cast<const T*>(p.accin)[i] + v) / T(p.div);
  if constexpr (sizeof(T) == 4) {
    if (p.snake_out) v = snake(v, p.alpha[c], p.inv_alpha[c]);
    if (p.out2) static_cast<float*>(p.out2)[i] = snake(v, p.alpha2[c], p.inv_alpha2[c]);
  }
  static_cast<T*>(p.out)[i] = v;
}

__device__ __forceinline__ float4 ld4f(const float* q) { return *reinterpret_cast<const float4*>(q); }

// conv_store1 for the four consecutive fp32 channels c .. c + 3 of one row, with 16-byte loads
// and stores (same operations in the same order, so the results are bit-identical)
__device__ __forceinline__ void conv_store4(const HiftConv& p, long row, int c, const f32x4& acc) {
  const float4 b = ld4f(static_cast<const float*>(p.bias) + c);
  float v[4] = {acc[0] + b.x, acc[1] + b.y, acc[2] + b.z, acc[3] + b.w};
  const long i = row * p.ldo + c;
  if (p.add) {
    const float4 a = ld4f(static_cast<const float*>(p.add) + row * p.ld_add + c);
    v[0] = v[0] + a.x; v[1] = v[1] + a.y; v[2] = v[2] + a.z; v[3] = v[3] + a.w;
  }
  if (p.mode != HIFT_ACC_WRITE) {
    const float4 a = ld4f(static_cast<const float*>(p.accin) + i);
    v[0] = a.x + v[0]; v[1] = a.y + v[1]; v[2] = a.z + v[2]; v[3] = a.w + v[3];
    if (p.mode == HIFT_ACC_ADD_DIV)
      for (int e = 0; e < 4; ++e) v[e] = v[e] / p.div;
  }
  // the Snakes one channel at a time: four inlined sinf at once spill
  if (p.snake_out) {
#pragma unroll 1
    for (int e = 0; e < 4; ++e) v[e] = snake(v[e], p.alpha[c + e], p.inv_alpha[c + e]);
  }
  if (p.out2) {
    float w[4];
#pragma unroll 1
    for (int e = 0; e < 4; ++e) w[e] = snake(v[e], p.alpha2[c + e], p.inv_alpha2[c + e]);
    *reinterpret_cast<float4*>(static_cast<float*>(p.out2) + i) = float4{w[0], w[1], w[2], w[3]};
  }
  *reinterpret_cast<float4*>(static_cast<float*>(p.out) + i) = float4{v[0], v[1], v[2], v[3]};
}

// The 16x16x4 accumulators of lane (li, lg) hold, for the tile's channel base cb:
//   fp32: channels cb + 4 lg + e;  fp64: channels cb + 4 e + lg  (e = 0..3)
template <typename T>
__device__ void conv_store(const HiftConv& p, long row, int cb, int lg,
                           const typename Vec4<T>::type& acc) {
  if constexpr (sizeof(T) == 4) {
    if (p.vec4 && cb + 4 * lg + 3 < p.cout) {
      conv_store4(p, row, cb + 4 * lg, acc);
      return;
    }
  }
  for (int e = 0; e < 4; ++e) {
    const int c = sizeof(T) == 4 ? cb + 4 * lg + e : cb + 4 * e + lg;
    if (c < p.cout) conv_store1<T>(p, row, c, acc[e]);
  }
}

// BK input channels of one tap per chunk (cin_pad % BK == 0), each lane feeding
// k = 16 m + 4 lg + s at MFMA step (m, s).  A workgroup owns TS time rows x TS output channels
// (TS = 64, or 32 for launches too small to give every CU a 64x64 tile); its four waves each
// own a TS/2 x TS/2 quarter.  Loaders: at TS = 64 every thread moves BK / 16 groups of 4
// elements of one weight row and one input row; at TS = 32 waves 0-1 move the weight rows and
// waves 2-3 the input rows, the same groups each.  Every output element accumulates the chunks
// in the same order with the same lane/slot -> k rule at both sizes, so the tile size does not
// change a result.
template <typename T, int BK, int TS>
__global__ __launch_bounds__(256) void hift_conv_kernel(const HiftConv p,
                                                        const HiftDocs* __restrict__ docs) {
  using VT = typename Vec4<T>::type;
  constexpr int PITCH = BK + 4;  // LDS row pitch in elements (conflict-free 16-byte reads)
  constexpr int G = BK / 16;
  constexpr int NQ = TS / 32;    // 16x16 accumulator tiles per wave along each side
  static_assert(TS == 64 || TS == 32, "tile size");
  __shared__ __attribute__((aligned(16))) T sA[2][TS][PITCH];
  __shared__ __attribute__((aligned(16))) T sB[2][TS][PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wc = wave & 1, wt = wave >> 1;
  const int li = lane & 15, lg = lane >> 4;
  const int n_docs = docs->n;
  const int rows_out = docs->b[n_docs];  // live rows (the grid covers the capacity)
  const int r0 = blockIdx.x * TS;
  if (r0 >= rows_out) return;
  const int co0 = blockIdx.y * TS;
  const int cpt = p.cin_pad / BK;
  const int KC = p.k * cpt;
  const long kcin = (long)p.k * p.cin_pad;

  // loader roles: weight row / input row lr, 4-element quarter lq of each 16-channel group;
  // at TS = 32 a thread loads the weights (ld_w) or the inputs (ld_x), not both
  const int lr = TS == 64 ? tid >> 2 : (tid & 127) >> 2, lq = tid & 3;
  const bool ld_w = TS == 64 || tid < 128, ld_x = TS == 64 || tid >= 128;
  const int r = r0 + lr;
  const bool valid = ld_x && r < rows_out;
  int in_base = 0, in_len = 0, pos = 0;
  if (valid) {
    const int d = doc_of(docs->b, n_docs, r);
    pos = r - docs->b[d];
    in_base = docs->a[d];
    in_len = docs->a[d + 1] - in_base;
  }
  const T* X = static_cast<const T*>(p.x);
  const T* W = static_cast<const T*>(p.w) + (long)(co0 + lr) * kcin + 4 * lq;

  // Two register sets: the loads of chunk kc + 2 are issued while chunk kc is computed and
  // chunk kc + 1 (loaded one iteration earlier) is written to LDS, so every load has about two
  // chunk computations to arrive.  The sets are picked by compile-time index (loop unrolled by 2).
  VT ra[2][G], rb[2][G];
  auto fetch = [&](int kc, VT (&a)[G], VT (&b)[G]) {
    const int tap = kc / cpt;
    const int c0 = (kc - tap * cpt) * BK + 4 * lq;
    const int u = pos * p.stride + tap * p.dil - p.pad;
    const int q = p.up > 1 ? (u >= 0 ? u / p.up : -1) : u;
    const bool live = valid && q >= 0 && q < in_len;
    const T* xr = X + (long)(in_base + q) * p.ldx + c0;
#pragma unroll
    for (int m = 0; m < G; ++m) {
      if (ld_w) a[m] = *reinterpret_cast<const VT*>(W + (long)kc * BK + 16 * m);
      b[m] = VT{T(0), T(0), T(0), T(0)};
      if (live) b[m] = *reinterpret_cast<const VT*>(xr + 16 * m);
    }
  };
  // the input prologue runs here, when the data is needed, so fetch never waits for its loads
  auto stash = [&](int buf, const VT (&a)[G], const VT (&b)[G]) {
#pragma unroll
    for (int m = 0; m < G; ++m) {
      VT bm = b[m];
      if constexpr (sizeof(T) == 4) {
        if (p.pro == HIFT_PRO_LEAKY) {
#pragma unroll
          for (int e = 0; e < 4; ++e) bm[e] = bm[e] > 0.0f ? bm[e] : bm[e] * p.slope;
        }
      }
      if (ld_w) *reinterpret_cast<VT*>(&sA[buf][lr][16 * m + 4 * lq]) = a[m];
      if (ld_x) *reinterpret_cast<VT*>(&sB[buf][lr][16 * m + 4 * lq]) = bm;
    }
  };

  VT acc[NQ][NQ];
#pragma unroll
  for (int a = 0; a < NQ; ++a)
#pragma unroll
    for (int b = 0; b < NQ; ++b) acc[a][b] = VT{T(0), T(0), T(0), T(0)};

  auto compute = [&](int cur) {
#pragma unroll
    for (int m = 0; m < G; ++m) {
      VT av[NQ], bv[NQ];
#pragma unroll
      for (int a = 0; a < NQ; ++a)
        av[a] = *reinterpret_cast<const VT*>(&sA[cur][wc * (TS / 2) + a * 16 + li][16 * m + 4 * lg]);
#pragma unroll
      for (int b = 0; b < NQ; ++b)
        bv[b] = *reinterpret_cast<const VT*>(&sB[cur][wt * (TS / 2) + b * 16 + li][16 * m + 4 * lg]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int a = 0; a < NQ; ++a)
#pragma unroll
          for (int b = 0; b < NQ; ++b) acc[a][b] = mfma_16x16x4(av[a][s], bv[b][s], acc[a][b]);
    }
  };

  fetch(0, ra[0], rb[0]);
  fetch(min(1, KC - 1), ra[1], rb[1]);
  stash(0, ra[0], rb[0]);
  __syncthreads();
  // Fetches and stashes run unconditionally (chunk indices clamped to the last chunk; a surplus
  // chunk lands in the LDS buffer no later computation reads), so no path leaves a load
  // pending and the compiler does not wait for the loads before the computation they overlap.
  // The fences keep each fetch ahead of its computation.
  for (int kc = 0; kc < KC; kc += 2) {
    // chunk kc is in LDS buffer 0; register set 1 holds chunk kc + 1
    fetch(min(kc + 2, KC - 1), ra[0], rb[0]);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    stash(1, ra[1], rb[1]);
    __syncthreads();
    if (kc + 1 >= KC) break;
    // chunk kc + 1 is in buffer 1; register set 0 holds chunk kc + 2
    fetch(min(kc + 3, KC - 1), ra[1], rb[1]);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    stash(0, ra[0], rb[0]);
    __syncthreads();
  }

  // D[i = channel][j = row]: lane holds row li and four channels of each 16x16 tile
#pragma unroll
  for (int b = 0; b < NQ; ++b) {
    const int rr = r0 + wt * (TS / 2) + b * 16 + li;
    if (rr >= rows_out) continue;
    const int d = doc_of(docs->b, n_docs, rr);
    const int pp = rr - docs->b[d];
    const long row_w = p.reflect ? (long)docs->b[d] + d + 1 + pp : rr;
#pragma unroll
    for (int a = 0; a < NQ; ++a) {
      const int cb = co0 + wc * (TS / 2) + a * 16;
      conv_store<T>(p, row_w, cb, lg, acc[a][b]);
      // reflection padding (1, 0): row 0 of the document repeats the result's row 1
      if (p.reflect && pp == 1) conv_store<T>(p, (long)docs->b[d] + d, cb, lg, acc[a][b]);
    }
  }
}

__global__ __launch_bounds__(256) void snake_kernel(const float* __restrict__ x, int ldx,
                                                    float* __restrict__ out, int ldo, int C,
                                                    const float* __restrict__ alpha,
                                                    const float* __restrict__ inv_alpha,
                                                    const HiftDocs* __restrict__ docs) {
  const int rows = docs->b[docs->n];
  const int q = C / 4;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * q) return;
  const long r = i / q;
  const int c = (int)(i - r * q) * 4;
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + r * ldx + c);
  f32x4 y;
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = snake(v[e], alpha[c + e], inv_alpha[c + e]);
  *reinterpret_cast<f32x4*>(out + r * ldo + c) = y;
}

__global__ __launch_bounds__(256) void to_f64_kernel(const float* __restrict__ x,
                                                     double* __restrict__ y, int C,
                                                     const HiftDocs* __restrict__ docs) {
  const long n = (long)docs->a[docs->n] * C;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (double)x[i];
}

__global__ __launch_bounds__(64) void f0_head_kernel(const double* __restrict__ h, int C,
                                                     const double* __restrict__ w,
                                                     const double* __restrict__ b,
                                                     float* __restrict__ f0,
                                                     const HiftDocs* __restrict__ docs) {
  const long r = blockIdx.x;
  if (r >= docs->b[docs->n]) return;
  double s = 0.0;
  for (int c = threadIdx.x; c < C; c += 64) s = fma(h[r * C + c], w[c], s);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (threadIdx.x == 0) f0[r] = (float)fabs(s + b[0]);
}

// One thread per (document, harmonic): the per-frame phase increment of harmonic h is
// rad = frac(f0 (h+1) / sr); the frame-rate value is the linear interpolation the reference
// takes from the sample-rate sequence (whose first sample also carries rand_ini[h]); the
// phase is the running sum in frame order, times 2 pi, times the upsampling scale.  The running
// sum is held in fp64 and rounded to fp32 at every frame, which is what the reference's
// torch.cumsum over the fp32 rad values (cosyvoice/hifigan/generator.py:255) computes on the
// CPU, whose kernel accumulates fp32 in double: an fp32 running sum drifts by ~1e-6 relative
// per few hundred frames, and the phase multiplies that by 2 pi x 480.
__global__ __launch_bounds__(64) void source_phase_kernel(const HiftSource p,
                                                          const HiftDocs* __restrict__ docs) {
#pragma clang fp contract(off)
  const int d = blockIdx.x;
  const int h = threadIdx.x;
  if (h >= p.H || d >= docs->n) return;
  const int f_base = docs->a[d];
  const int T = docs->a[d + 1] - f_base;
  const long L = (long)T * p.scale;
  const float mult = (float)(h + 1);
  const float sr = (float)p.sampling_rate;
  const float scale = (float)p.scale;
  auto rad_at = [&](long i) {
    const float x = (p.f0[f_base + i / p.scale] * mult) / sr;
    float v = x - floorf(x);
    if (i == 0) v = v + p.rand_ini[h];
    return v;
  };
  double c = 0.0;
  for (int t = 0; t < T; ++t) {
    float src = scale * ((float)t + 0.5f) - 0.5f;
    if (src < 0.0f) src = 0.0f;
    const long i0 = (long)src;
    const float l1 = fminf(fmaxf(src - (float)i0, 0.0f), 1.0f);
    const float l0 = 1.0f - l1;
    const long i1 = i0 + (i0 < L - 1 ? 1 : 0);
    const float a = l0 * rad_at(i0);
    const float b = l1 * rad_at(i1);
    c = c + (double)(a + b);
    float ph = ((float)c * 2.0f) * 3.14159265358979323846f;
    ph = ph * scale;
    p.sines[(long)(f_base + t) * p.H + h] = sinf(ph) * p.sine_amp;
  }
}

__global__ __launch_bounds__(256) void source_sample_kernel(const HiftSource p,
                                                            const HiftDocs* __restrict__ docs) {
#pragma clang fp contract(off)
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= docs->b[docs->n]) return;
  const int d = doc_of(docs->b, docs->n, n);
  const int pos = n - docs->b[d];
  const int fr = docs->a[d] + pos / p.scale;
  const float f0 = p.f0[fr];
  const float uv = f0 > p.voiced_threshold ? 1.0f : 0.0f;
  const float amp = uv * p.noise_std + ((1.0f - uv) * p.sine_amp) / 3.0f;
  const float* noise = p.table + (long)pos * p.H;
  float acc = 0.0f;
  for (int h = 0; h < p.H; ++h) {
    const float wave = p.sines[(long)fr * p.H + h] * uv + amp * noise[h];
    acc = acc + p.lin_w[h] * wave;
  }
  p.s[n] = tanhf(acc + p.lin_b[0]);
}

// cos / sin of 2 pi m / 16 for m = 0..15
__device__ __forceinline__ float cos16(int m) { return cospif((float)(m & 15) / 8.0f); }
__device__ __forceinline__ float sin16(int m) { return sinpif((float)(m & 15) / 8.0f); }

__global__ __launch_bounds__(256) void stft_kernel(const float* __restrict__ s,
                                                   const float* __restrict__ win,
                                                   float* __restrict__ out, int ld,
                                                   const HiftDocs* __restrict__ docs) {
  const int f = blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= docs->b[docs->n]) return;
  const int d = doc_of(docs->b, docs->n, f);
  const int fl = f - docs->b[d];
  const float* x = s + docs->a[d];
  const int L = docs->a[d + 1] - docs->a[d];
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    int i = 4 * fl + j - 8;
    if (i < 0) i = -i;
    if (i >= L) i = 2 * (L - 1) - i;
    v[j] = x[i] * win[j];
  }
  float* o = out + (long)f * ld;
#pragma unroll
  for (int k = 0; k <= 8; ++k) {
    float re = 0.0f, im = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      re = fmaf(v[j], cos16(j * k), re);
      im = fmaf(-v[j], sin16(j * k), im);
    }
    o[k] = re;
    o[9 + k] = im;
  }
  for (int c = 18; c < ld; ++c) o[c] = 0.0f;
}

// windowed inverse real DFT of one frame: mag = min(exp(y[k]), 100), ph = sin(y[9 + k])
__global__ __launch_bounds__(256) void istft_frame_kernel(const float* __restrict__ y, int ldy,
                                                          const float* __restrict__ win,
                                                          float* __restrict__ fr,
                                                          const HiftDocs* __restrict__ docs) {
  const int f = blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= docs->a[docs->n]) return;
  const float* row = y + (long)f * ldy;
  float re[9], im[9];
#pragma unroll
  for (int k = 0; k <= 8; ++k) {
    const float mag = fminf(expf(row[k]), 100.0f);
    const float ph = sinf(row[9 + k]);
    re[k] = mag * cosf(ph);
    im[k] = mag * sinf(ph);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float acc = re[0] + ((j & 1) ? -re[8] : re[8]);
    float h = 0.0f;
#pragma unroll
    for (int k = 1; k <= 7; ++k) h = h + (re[k] * cos16(j * k) - im[k] * sin16(j * k));
    acc = (acc + 2.0f * h) * (1.0f / 16.0f);
    fr[(long)f * 16 + j] = acc * win[j];
  }
}

// overlap-add: output sample pos of document d sits at padded position pos + 8 of the frame
// sequence; divided by the overlap-added squared window, clamped
__global__ __launch_bounds__(256) void istft_ola_kernel(const float* __restrict__ fr,
                                                        const float* __restrict__ win,
                                                        float* __restrict__ out, float limit,
                                                        const HiftDocs* __restrict__ docs) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= docs->b[docs->n]) return;
  const int d = doc_of(docs->b, docs->n, n);
  const int P = n - docs->b[d] + 8;
  const int f_base = docs->a[d];
  const int F = docs->a[d + 1] - f_base;
  float y = 0.0f, env = 0.0f;
  const int f_hi = min(P / 4, F - 1);
  for (int f = max(0, (P - 12) / 4); f <= f_hi; ++f) {
    const int j = P - 4 * f;
    if (j < 0 || j >= 16) continue;
    y = y + fr[(long)(f_base + f) * 16 + j];
    env = env + win[j] * win[j];
  }
  const float v = y / env;
  out[n] = fminf(fmaxf(v, -limit), limit);
}

__global__ __launch_bounds__(256) void copy_live_kernel(const float* __restrict__ src,
                                                        float* __restrict__ dst,
                                                        const HiftDocs* __restrict__ docs) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < docs->b[docs->n]) dst[i] = src[i];
}

unsigned blocks_for(long n, int threads) { return (unsigned)((n + threads - 1) / threads); }

bool aligned16(const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; }

template <typename T>
hipError_t launch_conv(const HiftConv& p_in, const HiftDocs* docs, hipStream_t stream) {
  if (p_in.rows_out <= 0) return hipSuccess;
  if (p_in.cin_pad % 16 != 0) return hipErrorInvalidValue;
  HiftConv p = p_in;
  // 16-byte epilogue accesses when every row pitch and base the epilogue touches allows them
  p.vec4 = sizeof(T) == 4 && p.ldo % 4 == 0 && aligned16(p.out) && aligned16(p.bias) &&
           (!p.add || (p.ld_add % 4 == 0 && aligned16(p.add))) &&
           (p.mode == HIFT_ACC_WRITE || aligned16(p.accin)) &&
           (!p.snake_out || (aligned16(p.alpha) && aligned16(p.inv_alpha))) &&
           (!p.out2 || (aligned16(p.out2) && aligned16(p.alpha2) && aligned16(p.inv_alpha2)));
  // 64x64 tiles, or 32x32 where 64x64 tiles would not give every CU one (the grid covers the
  // capacity, so a captured call and its replays use the same size; results do not depend on it).
  // FCV_HIFT_TILE=32 or 64 forces one size: a test hook, since both must give the same bits.
  const long tiles64 = (long)((p.rows_out + kTileR - 1) / kTileR) * ((p.cout + kTileC - 1) / kTileC);
  const char* forced = std::getenv("FCV_HIFT_TILE");
  const int force = forced ? std::atoi(forced) : 0;
  if (force == 32 || (force != 64 && tiles64 < kSmallTileBelow)) {
    const dim3 grid((p.rows_out + 31) / 32, (p.cout + 31) / 32);
    if (p.cin_pad % 32 == 0)
      hipLaunchKernelGGL((hift_conv_kernel<T, 32, 32>), grid, dim3(256), 0, stream, p, docs);
    else
      hipLaunchKernelGGL((hift_conv_kernel<T, 16, 32>), grid, dim3(256), 0, stream, p, docs);
    return hipGetLastError();
  }
  const dim3 grid((p.rows_out + kTileR - 1) / kTileR, (p.cout + kTileC - 1) / kTileC);
  if (p.cin_pad % 32 == 0)
    hipLaunchKernelGGL((hift_conv_kernel<T, 32, 64>), grid, dim3(256), 0, stream, p, docs);
  else
    hipLaunchKernelGGL((hift_conv_kernel<T, 16, 64>), grid, dim3(256), 0, stream, p, docs);
  return hipGetLastError();
}

}  // namespace

hipError_t hift_conv_f32(const HiftConv& p, const HiftDocs* docs, hipStream_t stream) {
  return launch_conv<float>(p, docs, stream);
}
hipError_t hift_conv_f64(const HiftConv& p, const HiftDocs* docs, hipStream_t stream) {
  return launch_conv<double>(p, docs, stream);
}

hipError_t hift_snake(const float* x, int ldx, float* out, int ldo, int rows, int C,
                      const float* alpha, const float* inv_alpha, const HiftDocs* docs,
                      hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const long n = (long)rows * (C / 4);
  hipLaunchKernelGGL(snake_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, x, ldx, out,
                     ldo, C, alpha, inv_alpha, docs);
  return hipGetLastError();
}

hipError_t hift_to_f64(const float* x, double* y, int rows, int C, const HiftDocs* docs,
                       hipStream_t stream) {
  const long n = (long)rows * C;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(to_f64_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, x, y, C,
                     docs);
  return hipGetLastError();
}

hipError_t hift_f0_head(const double* h, int C, const double* cls_w, const double* cls_b,
                        int rows, float* f0, const HiftDocs* docs, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(f0_head_kernel, dim3(rows), dim3(64), 0, stream, h, C, cls_w, cls_b, f0,
                     docs);
  return hipGetLastError();
}

hipError_t hift_source(const HiftSource& p, const HiftDocs* docs, hipStream_t stream) {
  if (p.docs_cap <= 0) return hipSuccess;
  hipLaunchKernelGGL(source_phase_kernel, dim3(p.docs_cap), dim3(64), 0, stream, p, docs);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.samples_cap <= 0) return hipSuccess;
  hipLaunchKernelGGL(source_sample_kernel, dim3(blocks_for(p.samples_cap, 256)), dim3(256), 0,
                     stream, p, docs);
  return hipGetLastError();
}

hipError_t hift_copy_live(const float* src, float* dst, int rows, const HiftDocs* docs,
                          hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(copy_live_kernel, dim3(blocks_for(rows, 256)), dim3(256), 0, stream, src,
                     dst, docs);
  return hipGetLastError();
}

hipError_t hift_stft(const float* s, const float* window, float* out, int ld, int frames,
                     const HiftDocs* docs, hipStream_t stream) {
  if (frames <= 0) return hipSuccess;
  hipLaunchKernelGGL(stft_kernel, dim3(blocks_for(frames, 256)), dim3(256), 0, stream, s, window,
                     out, ld, docs);
  return hipGetLastError();
}

hipError_t hift_istft(const float* y, int ldy, const float* window, float* fr, float* out,
                      float limit, int frames, int samples, const HiftDocs* docs,
                      hipStream_t stream) {
  if (frames > 0) {
    hipLaunchKernelGGL(istft_frame_kernel, dim3(blocks_for(frames, 256)), dim3(256), 0, stream, y,
                       ldy, window, fr, docs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (samples <= 0) return hipSuccess;
  hipLaunchKernelGGL(istft_ola_kernel, dim3(blocks_for(samples, 256)), dim3(256), 0, stream, fr,
                     window, out, limit, docs);
  return hipGetLastError();
}

}  // namespace fcv
