/*
 * fcv_flow.h -- C ABI of the Flow front-end in libfcvdit.so: the step that turns speech tokens,
 * prompt Mel frames and speaker x-vectors into the packed estimator inputs mu / cond / spks.
 *
 * It replaces the front half of the reference's flow_inference_batched and
 * flow_inference_batched_streaming (faster_cosyvoice/token2wav/flashinfer_flow.py:144-162 and
 * :187-262): token embedding with clamped ids, PreLookaheadLayer
 * (cosyvoice/transformer/upsample_encoder.py:55-92), repeat_interleave to Mel frames, the
 * speaker normalize + affine projection and the prompt copy into the condition.  Outputs are
 * written as packed rows (document after document, no padding), the layout fcv_dit_solve reads.
 *
 * Conventions are those of fcv_dit.h: device pointers unless the name ends in `_host`, fp32
 * row-major tensors, FCV_OK or an error code (message in fcv_last_error()), no allocation of
 * caller memory.  Calls are asynchronous on `stream` (the per-document tables travel in the
 * kernel arguments, so no host-to-device copy or synchronisation happens inside a call) and
 * may be captured into a hipGraph.  Calls that share a workspace must be issued on one stream.
 * A call covers at most FCV_FLOW_MAX_DOCS documents; larger batches are split by the caller
 * (results do not depend on how documents are grouped into calls).
 */
#ifndef FCV_FLOW_H
#define FCV_FLOW_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "fcv_dit.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FCV_FLOW_MAX_DOCS 256

/* Front-end shape (builders.py:29-35: input_size = output_size = 80, vocab_size 6561,
 * spk_embed_dim 192, PreLookaheadLayer(in_channels=80, channels=1024, pre_lookahead_len=3),
 * token_mel_ratio 2).  Supported: feat_dim == 80, channels % 128 == 0, 0 <= lookahead <= 7,
 * 1 <= token_mel_ratio <= 8, 1 <= spk_dim <= 256. */
typedef struct FcvFlowDims {
  int32_t vocab;            /* rows of the token embedding table */
  int32_t feat_dim;         /* 80: embedding width = Mel channels */
  int32_t channels;         /* 1024: PreLookaheadLayer hidden channels */
  int32_t lookahead;        /* 3: pre_lookahead_len; conv1 has lookahead + 1 taps */
  int32_t token_mel_ratio;  /* 2: Mel frames per token */
  int32_t spk_dim;          /* 192: x-vector width */
} FcvFlowDims;

/* fp32 weights (device pointers, caller-owned, 16-byte aligned).  The two convolution weights
 * are re-laid out tap-major so that one output's weights are contiguous:
 *   la1_w[c][tap * feat_dim + i] = pre_lookahead_layer.conv1.weight[c][i][tap]
 *   la2_w[o][tap * channels + c] = pre_lookahead_layer.conv2.weight[o][c][tap]   (3 taps) */
typedef struct FcvFlowWeights {
  const float* embed;  /* [vocab][feat_dim]              input_embedding.weight */
  const float* la1_w;  /* [channels][(lookahead+1)*feat_dim] */
  const float* la1_b;  /* [channels]                     pre_lookahead_layer.conv1.bias */
  const float* la2_w;  /* [feat_dim][3*channels] */
  const float* la2_b;  /* [feat_dim]                     pre_lookahead_layer.conv2.bias */
  const float* spk_w;  /* [feat_dim][spk_dim]            spk_embed_affine_layer.weight */
  const float* spk_b;  /* [feat_dim]                     spk_embed_affine_layer.bias */
} FcvFlowWeights;

/* Device workspace of fcv_flow_token_features for a call producing `out_tokens` token rows
 * (hidden conv1 activations and conv2 partial sums).  Monotone in out_tokens. */
size_t fcv_flow_workspace_bytes(const FcvFlowDims* dims, int32_t out_tokens);

/* Token features -> packed mu rows.  Document d owns tokens[cu_tokens_host[d] ..
 * cu_tokens_host[d+1]) (int32 ids; negative ids read row 0 as clamp(min=0) does; ids >= vocab
 * are the caller's error and read row vocab-1).  finalize_host[d] != 0 (or finalize_host ==
 * NULL: every document) treats the document as complete: right zero padding of `lookahead`
 * frames (flashinfer_flow.py:149-150, 197-198).  finalize_host[d] == 0 routes the last
 * `lookahead` tokens to conv1 as right context only (flashinfer_flow.py:199-203): the document
 * then yields len - lookahead token rows and needs len > lookahead.  Per output token t of a
 * document with token embeddings e(.):
 *   h(t)  = leaky_relu(conv1 over e(t) .. e(t+lookahead), zero past the document's tokens)
 *   y(t)  = conv2 over h(t-2) .. h(t) (zero before the document start) + e(t)
 * and y(t) is written to Mel rows ratio*t .. ratio*t + ratio-1 of mu_out
 * ([ratio * out_tokens][feat_dim], document d starting at ratio * its first output token). */
int fcv_flow_token_features(const FcvFlowDims* dims, const FcvFlowWeights* weights,
                            const int32_t* tokens, const int32_t* cu_tokens_host,
                            const int32_t* finalize_host, int32_t n_docs, float* mu_out,
                            void* workspace, size_t workspace_bytes, hipStream_t stream);

/* fcv_flow_token_features without a workspace argument: no counterpart in the reference.  It is
 * for callers that cannot allocate device memory (code under hipGraph capture, serving loops or
 * harnesses that forbid hipMalloc).  Same inputs, outputs and results as
 * fcv_flow_token_features; the workspace is the library's own 32 MiB device array, one copy per
 * GPU, held until the process ends, so a call takes at most FCV_FLOW_NOALLOC_SCRATCH_BYTES of
 * workspace (fcv_flow_workspace_bytes): 5041 output tokens at the builders.py dims.  Larger
 * calls fail with FCV_ERR_INVALID.  The call allocates nothing.  Calls that overlap on one GPU
 * (on different streams or threads) race on the array: issue them on one stream. */
#define FCV_FLOW_NOALLOC_SCRATCH_BYTES (32u << 20)
int fcv_flow_token_features_noalloc(const FcvFlowDims* dims, const FcvFlowWeights* weights,
                                    const int32_t* tokens, const int32_t* cu_tokens_host,
                                    const int32_t* finalize_host, int32_t n_docs, float* mu_out,
                                    hipStream_t stream);

/* Speaker path (flashinfer_flow.py:145-146, :230-231): spks_out[n] = spk_w . (xvec[n] /
 * max(||xvec[n]||_2, 1e-12)) + spk_b.  xvec: [n][spk_dim]; spks_out: [n][feat_dim]. */
int fcv_flow_speaker(const FcvFlowDims* dims, const FcvFlowWeights* weights, const float* xvec,
                     int32_t n, float* spks_out, hipStream_t stream);

/* Prompt copy into the condition (_copy_prompt_features, flashinfer_flow.py:93-115), packed:
 * cond_out row cu_mel_host[d] + p = prompt row cu_prompt_host[d] + p for
 * p < min(prompt length, Mel length) of document d, zero for the rest of the document.
 * prompt: [cu_prompt_host[n_docs]][feat_dim]; cond_out: [cu_mel_host[n_docs]][feat_dim]. */
int fcv_flow_prompt_cond(const FcvFlowDims* dims, const float* prompt,
                         const int32_t* cu_prompt_host, const int32_t* cu_mel_host,
                         int32_t n_docs, float* cond_out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FCV_FLOW_H */
