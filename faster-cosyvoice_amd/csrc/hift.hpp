// Kernels of the HiFT vocoder (hift.hip) and their launch parameters; the orchestration and the
// C ABI live in hift_capi.hip.  All activations are time-major: row = time step of one
// document, channels contiguous; documents are packed one after another.  Every launch reads
// the per-document row prefix sums and the live document count from a table in device memory
// (HiftDocs, at most kHiftMaxDocs documents), and its grid covers a capacity: workgroups past the
// live rows exit.  So a captured vocoder call replays for any layout that fits its capacity.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace fcv {

constexpr int kHiftMaxDocs = 256;

// n live documents and two exclusive prefix sums over them: a = input rows, b = output rows
// (live input rows a[n], live output rows b[n])
struct HiftDocs {
  int32_t n;
  int32_t a[kHiftMaxDocs + 1];
  int32_t b[kHiftMaxDocs + 1];
};

enum { HIFT_PRO_NONE = 0, HIFT_PRO_LEAKY = 1 };
enum { HIFT_ACC_WRITE = 0, HIFT_ACC_ADD = 1, HIFT_ACC_ADD_DIV = 2 };

// One 1-D convolution as an implicit GEMM: out[r][co] over output rows r of every document.
// Input position of tap j for output position p of a document:
//   u = p * stride + j * dil - pad;  q = up > 1 ? (u >= 0 ? u / up : -1) : u
// and the input row is read when 0 <= q < the document's input length (zero otherwise).
// Weights are packed [cout rounded up to 64][k][cin_pad] (cin_pad % 16 == 0, zero padding).
struct HiftConv {
  const void* x; int ldx;                 // input rows [*][ldx], ldx >= cin_pad
  const void* w; const void* bias;
  int cout, cin_pad, k, stride, dil, pad, up;
  int rows_out;                            // capacity the grid covers (live: docs->b[docs->n])
  int reflect;                             // write row p + 1 (row 0 = row 2 of the result)
  int pro; float slope;                    // prologue on the inputs (fp32 only)
  int elu;                                 // epilogue ELU (fp64 only)
  const void* add; int ld_add;             // y += add[row] (layout of out)
  int mode; const void* accin; float div;  // y = accin + y  or  (accin + y) / div
  const float* alpha; const float* inv_alpha;    // snake_out: out = snake(y)
  int snake_out;
  void* out; int ldo;
  void* out2; const float* alpha2; const float* inv_alpha2;  // out2 = snake(y) (optional)
  int vec4;                                // set by the launch: 16-byte epilogue accesses
};

hipError_t hift_conv_f32(const HiftConv& p, const HiftDocs* docs, hipStream_t stream);
hipError_t hift_conv_f64(const HiftConv& p, const HiftDocs* docs, hipStream_t stream);

// out[r][c] = snake(x[r][c]) for the live rows docs->b[docs->n] (grid: `rows`) x C channels
// (C % 4 == 0), row strides ldx / ldo
hipError_t hift_snake(const float* x, int ldx, float* out, int ldo, int rows, int C,
                      const float* alpha, const float* inv_alpha, const HiftDocs* docs,
                      hipStream_t stream);

// fp32 -> fp64 of the live rows docs->a[docs->n] (grid: `rows`) x C values
hipError_t hift_to_f64(const float* x, double* y, int rows, int C, const HiftDocs* docs,
                       hipStream_t stream);

// f0[r] = (float)|cls_w . h[r] + cls_b| (fp64 dot over C channels), one wave per live row
// docs->b[docs->n] (grid: `rows`)
hipError_t hift_f0_head(const double* h, int C, const double* cls_w, const double* cls_b,
                        int rows, float* f0, const HiftDocs* docs, hipStream_t stream);

struct HiftSource {
  const float* f0;          // frame F0, rows by docs.a
  const float* rand_ini;    // [H]
  const float* table;       // noise table [max_samples][H]
  int max_samples;
  const float* lin_w; const float* lin_b;  // [H], [1]
  int H, scale, sampling_rate;
  float sine_amp, noise_std, voiced_threshold;
  int docs_cap;             // documents the phase grid covers
  int samples_cap;          // samples the merge grid covers
  float* sines;             // [frames][H] work: sin(phase) * sine_amp per frame
  float* s;                 // [samples] source, rows by docs.b
};
// per-frame phases (sequential sum per document and harmonic) then per-sample merge
hipError_t hift_source(const HiftSource& p, const HiftDocs* docs, hipStream_t stream);

// dst[i] = src[i] for the live rows docs->b[docs->n] (grid: `rows`)
hipError_t hift_copy_live(const float* src, float* dst, int rows, const HiftDocs* docs,
                          hipStream_t stream);

// STFT frames (n_fft 16, hop 4, centred, reflect padding) of each document's source:
// out[f][0..8] = Re, out[f][9..17] = Im, out[f][18..ld) = 0; docs.a = samples, docs.b = frames
// (grid: `frames`)
hipError_t hift_stft(const float* s, const float* window, float* out, int ld, int frames,
                     const HiftDocs* docs, hipStream_t stream);

// iSTFT: per frame f of y [frames][ldy] (log-magnitudes 0..8, phase inputs 9..17), the
// windowed inverse real DFT into fr [frames][16]; then centred overlap-add divided by the
// window envelope, clamped to +-limit, keeping the first docs.b lengths of each document.
// docs.a = frames, docs.b = output samples (grids: `frames`, `samples`).
hipError_t hift_istft(const float* y, int ldy, const float* window, float* fr, float* out,
                      float limit, int frames, int samples, const HiftDocs* docs,
                      hipStream_t stream);

}  // namespace fcv
