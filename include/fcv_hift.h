/*
 * fcv_hift.h -- C ABI of the HiFT vocoder in libfcvdit.so: Mel frames -> 24 kHz waveform.
 *
 * It replaces CausalHiFTGenerator.inference (faster_cosyvoice/token2wav/cosyvoice/hifigan/
 * generator.py:578-735, with CausalConvRNNF0Predictor, hifigan/f0_predictor.py:62-103), the
 * step after the Flow in token2wav.py:128-131 (offline) and :188-200 (streaming).  Several
 * requests are vocoded in one call as packed documents; each document is processed exactly as
 * the reference processes one request (its own causal padding, STFT edges and F0 source), so a
 * document's waveform does not depend on what it is packed with.
 *
 * Conventions are those of fcv_dit.h: device pointers unless the name ends in `_host`, fp32
 * row-major tensors, FCV_OK or an error code (message in fcv_last_error()), no allocation of
 * caller memory.  Mel input is time-major: [sum of frames][in_channels].
 */
#ifndef FCV_HIFT_H
#define FCV_HIFT_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "fcv_dit.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FCV_HIFT_MAX 4
#define FCV_HIFT_MAX_DOCS 256

/* Vocoder shape (builders.py:38-50 gives the CosyVoice3 values in the comments).  Supported:
 * 1 <= n_stages, n_kernels, n_dilations <= 4; in_channels and every stage's channels
 * (base_channels >> (i + 1)) multiples of 16; n_fft = 16, hop_len = 4; f0_channels % 64 == 0. */
typedef struct FcvHiftDims {
  int32_t in_channels;                      /* 80 */
  int32_t base_channels;                    /* 512 */
  int32_t nb_harmonics;                     /* 8 (9 sines with the fundamental) */
  int32_t sampling_rate;                    /* 24000 */
  float nsf_alpha, nsf_sigma, nsf_voiced_threshold;  /* 0.1, 0.003, 10 */
  int32_t n_stages;                         /* 3 */
  int32_t upsample_rates[FCV_HIFT_MAX];     /* 8 5 3 */
  int32_t upsample_kernels[FCV_HIFT_MAX];   /* 16 11 7 */
  int32_t n_kernels;                        /* 3 resblocks per stage */
  int32_t resblock_kernels[FCV_HIFT_MAX];   /* 3 7 11 */
  int32_t n_dilations;                      /* 3 per resblock */
  int32_t resblock_dilations[FCV_HIFT_MAX][FCV_HIFT_MAX];  /* [kernel][j]: 1 3 5 */
  int32_t source_kernels[FCV_HIFT_MAX];     /* per stage: 7 7 11 */
  int32_t source_dilations[FCV_HIFT_MAX][FCV_HIFT_MAX];    /* [stage][j]: 1 3 5 */
  int32_t n_fft, hop_len;                   /* 16, 4 */
  int32_t conv_pre_look_right;              /* 4 */
  int32_t f0_channels;                      /* 512 */
  float lrelu_slope, audio_limit;           /* 0.1, 0.99 */
  int32_t noise_samples;                    /* rows of the source noise table (300 * 24000) */
} FcvHiftDims;

/* Number of device pointers fcv_hift_create expects, in this order (weight norm folded,
 * w = g * v / ||v||; every conv weight packed [ceil64(cout)][k][ceil16(cin)] with zeros in the
 * padding; a = Snake alpha, ia = 1 / (alpha + 1e-9) in fp32):
 *   source merge: l_linear.weight [H], l_linear.bias [1]
 *   conv_pre w, b
 *   for each stage: ups.i w, b
 *   for each stage: source_downs.i w, b           (input channels n_fft + 2, padded to 32)
 *   for each stage: source_resblocks.i: for each dilation j: convs1.j w, b, convs2.j w, b,
 *                   activations1.j a, ia, activations2.j a, ia
 *   for each stage, each kernel: resblocks.(stage * n_kernels + kernel): same 8 per dilation
 *   conv_post w, b                                (18 outputs)
 *   f0_predictor.condnet.{0,2,4,6,8} w, b          (fp64)
 *   f0_predictor.classifier w [f0_channels], b [1] (fp64)
 *   Hann window [n_fft] (periodic), rand_ini [H], noise table [noise_samples][H]
 * All fp32 unless marked fp64; H = nb_harmonics + 1.  Returns 0 for unsupported dims. */
int32_t fcv_hift_weight_count(const FcvHiftDims* dims);

typedef struct FcvHift FcvHift;

/* Validate the dims and keep the pointer table (caller-owned memory, must outlive the handle). */
int fcv_hift_create(const FcvHiftDims* dims, const void* const* weights, int32_t n_weights,
                    FcvHift** out);
int fcv_hift_destroy(FcvHift* hift);

/* Waveform samples produced for a document of `frames` Mel frames:
 * finalize != 0: frames * upsample_scale (480 for CosyVoice3); otherwise the last
 * 3 + conv_pre_look_right + 1 frames are right context and (frames - 8) * 480 samples come out
 * (generator.py:700-731).  -1 if the document is too short. */
int64_t fcv_hift_output_samples(const FcvHift* hift, int32_t frames, int32_t finalize);

/* Device workspace for one fcv_hift_inference call over these documents. */
size_t fcv_hift_workspace_bytes(const FcvHift* hift, const int32_t* frames_host,
                                const int32_t* finalize_host, int32_t n_docs);

/* Vocode `n_docs` packed documents (CausalHiFTGenerator.inference, generator.py:719-735):
 * mel [sum frames][in_channels]; speech_out gets each document's
 * fcv_hift_output_samples(frames, finalize) samples one after another, clamped to
 * +-audio_limit; source_out (optional, NULL to skip) gets each document's harmonic source
 * (frames_f0 * upsample_scale samples, frames_f0 = frames or frames - 3).
 * finalize_host NULL: every document is final.  Asynchronous on `stream`. */
int fcv_hift_inference(FcvHift* hift, const float* mel, const int32_t* frames_host,
                       const int32_t* finalize_host, int32_t n_docs, float* speech_out,
                       float* source_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* Device workspace of a call capacity: at most frames_cap Mel frames in docs_cap documents. */
size_t fcv_hift_workspace_bytes_capacity(const FcvHift* hift, int32_t frames_cap,
                                         int32_t docs_cap);

/* fcv_hift_inference inside a capacity (sum of frames <= frames_cap, n_docs <= docs_cap), with
 * the graph pool: replaces the reference's per-bucket CUDA graphs of the streaming vocoder
 * (hift_graph.py:65-169; HiftStreamGraph pads each request to its bucket and replays).  The
 * workspace carve-up and every grid depend on the capacity only; the call's layout is written
 * into the workspace and read by the kernels, so with use_graph != 0 the launch sequence
 * captured for (capacity, workspace, mel, speech_out, source_out) replays for any later layout
 * of that capacity, bit-identical to an eager call.  A key is captured on its second call; the
 * handle keeps the 4 most recently used graphs.  The layout is copied from host memory on
 * `stream` before the launches (the copy is complete when the call returns). */
int fcv_hift_inference_capacity(FcvHift* hift, const float* mel, const int32_t* frames_host,
                                const int32_t* finalize_host, int32_t n_docs, int32_t frames_cap,
                                int32_t docs_cap, float* speech_out, float* source_out,
                                void* workspace, size_t workspace_bytes, int32_t use_graph,
                                hipStream_t stream);

/* Vocoder graphs the handle holds (at most 4) and the calls it has captured so far.  No
 * counterpart in the reference (whose graph runner logs each capture, hift_graph.py:136-137). */
int fcv_hift_graph_stats(const FcvHift* hift, int32_t* pooled, int32_t* captures);

#ifdef __cplusplus
}
#endif

#endif /* FCV_HIFT_H */
