/*
 * fcv_dit.h -- C ABI of libfcvdit.so, the MI355X (gfx950) CosyVoice3 Token2Wav DiT estimator.
 *
 * The library replaces the estimator plugin that the reference installs as
 * `flow.decoder.estimator` (faster_cosyvoice/token2wav/flashinfer_dit.py:951-988) and the
 * packed CFG Euler loop that calls it (faster_cosyvoice/token2wav/flashinfer_flow.py:16-74).
 * Its calling pattern mirrors the reference's raw-pointer estimator form, the TensorRT
 * branch of ConditionalCFM.forward_estimator (cosyvoice/flow/flow_matching.py:129-153):
 * device pointers plus an explicit stream, output written into caller memory.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless its name ends in `_host`.
 *   - All boundary tensors are fp32 and row-major; "packed rows" means documents laid out one
 *     after another without padding, document d owning rows [cu_seqlens[d], cu_seqlens[d+1]).
 *   - Functions return FCV_OK (0) or an error code; fcv_last_error() gives the message of the
 *     last failure on the calling thread.  Nothing in the library allocates caller memory.
 *   - A handle is not re-entrant: one handle per stream / thread, as in the reference
 *     (flashinfer_attention.py:36-42 keeps one plan per wrapper).
 */
#ifndef FCV_DIT_H
#define FCV_DIT_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FCV_OK = 0,
  FCV_ERR_INVALID = 1,   /* bad argument, shape or layout (Python: ValueError) */
  FCV_ERR_RUNTIME = 2,   /* HIP error (Python: RuntimeError) */
  FCV_ERR_STATE = 3      /* call order violated, e.g. forward before plan (RuntimeError) */
};

enum { FCV_MASK_FULL = 0, FCV_MASK_CHUNK_CAUSAL = 1 };

/* Model shape.  Supported: dim = heads * 64 = 1024, dim_head 64, ff_dim % 128 == 0,
 * mel_dim 80, conv_groups * 64 == dim, conv_kernel <= 31, rope_dim <= dim_head, even.
 * Mirrors FlashInferDiT.__init__ (flashinfer_dit.py:128-186) / builders.py:17-21. */
typedef struct FcvDitDims {
  int32_t dim, depth, heads, dim_head, ff_dim, mel_dim;
  int32_t conv_kernel, conv_groups;
  int32_t rope_dim; /* flat q/k columns that rotate: 64 = head 0 (flashinfer_dit.py:61) */
  int32_t max_pos;  /* rows of the RoPE tables; documents may not be longer */
} FcvDitDims;

/* Derived inference weights (device pointers, caller-owned, must outlive the handle).
 * Weight matrices are IEEE fp16 (the dtype apply_flashinfer gives the reference's DiT,
 * flashinfer_dit.py:963), biases and RoPE tables fp32.  Derivation follows FlashInferDiT.finalize_weights
 * (flashinfer_dit.py:228-313): fused QKV, "+1" folded into the AdaLN scale biases, one
 * concatenated AdaLN projection, conv weights re-laid out per group and tap. */
typedef struct FcvDitWeights {
  const void* temb_w1;  const float* temb_b1;  /* fp16 [dim][256], fp32 [dim] */
  const void* temb_w2;  const float* temb_b2;  /* fp16 [dim][dim] */
  const void* ada_w;    const float* ada_b;    /* fp16 [depth*6*dim + 2*dim][dim] */
  const void* in_w;     const float* in_b;     /* fp16 [dim][4*mel] (x, cond, mu, spks) */
  const void* conv1_w;  const float* conv1_b;  /* fp16 [groups][kernel][64][64] (g, tap, co, ci) */
  const void* conv2_w;  const float* conv2_b;
  const void* qkv_w;    const float* qkv_b;    /* fp16 [depth][3*dim][dim] */
  const void* out_w;    const float* out_b;    /* fp16 [depth][dim][dim] */
  const void* ff1_w;    const float* ff1_b;    /* fp16 [depth][ff][dim] */
  const void* ff2_w;    const float* ff2_b;    /* fp16 [depth][dim][ff] */
  const void* proj_w;   const float* proj_b;   /* fp16 [128][dim], fp32 [128]; rows >= mel zero */
  const float* rope_cos; const float* rope_sin; /* fp32 [max_pos][rope_dim/2] */
} FcvDitWeights;

typedef struct FcvDit FcvDit;

/* Message of the last failed call on this thread ("" if none). */
const char* fcv_last_error(void);

/* Create / destroy an estimator handle (FlashInferDiT construction + finalize_weights,
 * flashinfer_dit.py:128-186,228-313).  No device memory is allocated. */
int fcv_dit_create(const FcvDitDims* dims, const FcvDitWeights* weights, FcvDit** out);
int fcv_dit_destroy(FcvDit* dit);

/* Device workspace needed for a packed batch of `rows` rows and `n_docs` documents, or for a
 * capacity of that many (fcv_dit_plan_capacity) (replaces the reference's 64 MB FlashInfer
 * workspace, flashinfer_attention.py:13,55, and the activations torch allocates per forward).
 * Monotone in both arguments. */
size_t fcv_dit_workspace_bytes(const FcvDit* dit, int32_t rows, int32_t n_docs);

/* Plan a packed layout (replaces RaggedAttentionRunner._prepare / wrapper.plan,
 * flashinfer_attention.py:88-123, and _get_packed_layout, flashinfer_dit.py:364-405).
 * cu_seqlens_host: [n_docs+1] exclusive prefix sums, cu[0] = 0, non-decreasing, every
 * document 1 <= length <= max_pos, and (rows + 7 per document) x max(2 ff_dim, 4 dim) bytes
 * below 2 GB (the kernels address activations by 32-bit byte offsets; about 5 x 10^5 rows at
 * the Token2Wav dims).  mask_mode: FCV_MASK_FULL or FCV_MASK_CHUNK_CAUSAL
 * (key k visible to query q iff k/chunk <= q/chunk, flashinfer_attention.py:16-33).
 * The workspace is bound to the handle until the next plan.  Synchronous on `stream`.
 * Same as fcv_dit_plan_capacity with a capacity of exactly this layout's rows and documents. */
int fcv_dit_plan(FcvDit* dit, const int32_t* cu_seqlens_host, int32_t n_docs, int32_t mask_mode,
                 int32_t chunk, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Plan a layout inside a capacity of rows_cap caller rows in docs_cap documents (the layout
 * must fit: rows <= rows_cap, n_docs <= docs_cap).  The replacement of the reference's bucketed
 * graph runners (flashinfer_dit.py:742-804: one captured graph per padded length, a runtime
 * padding boundary) for the packed layout: the workspace layout and every kernel grid depend on
 * the capacity only, and the kernels read the layout's live row, tile and document tables from
 * the workspace, so a solve graph captured under one layout replays for any other layout
 * planned into the same capacity (and workspace), with results bit-identical to an exact plan.
 * Workspace: fcv_dit_workspace_bytes(dit, rows_cap, docs_cap). */
int fcv_dit_plan_capacity(FcvDit* dit, const int32_t* cu_seqlens_host, int32_t n_docs,
                          int32_t mask_mode, int32_t chunk, int32_t rows_cap, int32_t docs_cap,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

/* One estimator forward over the planned packed batch (FlashInferDiT._forward_packed,
 * flashinfer_dit.py:447-543).  x, mu, cond: [rows][mel]; spks: [n_docs][mel];
 * t: [n_t] with n_t == 1 (shared by every document) or n_t == n_docs; v_out: [rows][mel]. */
int fcv_dit_forward(FcvDit* dit, const float* x, const float* mu, const float* cond,
                    const float* spks, const float* t, int32_t n_t, float* v_out,
                    hipStream_t stream);

/* CFG combine + Euler update of one step (flashinfer_flow.py:66-70) on a planned batch whose
 * documents are [cond_0..cond_{B-1}, uncond_0..uncond_{B-1}]: for the first half of the rows
 * x += dt * ((1+cfg) v_cond - cfg v_uncond), then the second half is set equal to the first. */
int fcv_euler_cfg_step(FcvDit* dit, float* x, const float* v, float dt, float cfg,
                       hipStream_t stream);

/* Full CFG Euler solve (solve_euler_batched, flashinfer_flow.py:16-74) over the planned
 * batch: n_steps x (forward with t_host[step] shared by all documents, then the CFG Euler
 * update with dt_host[step]).  x: [rows][mel], both halves equal on entry, updated in place.
 * mu/cond/spks as in fcv_dit_forward (zeros in the unconditional half).  use_graph != 0
 * replays a hipGraph of the whole loop when the plan's capacity and mask, the workspace and the
 * pointers and the schedule (dt_host, cfg, n_steps) match a captured graph's; the handle keeps
 * the 4 most recently used graphs (the reference pools 4 plans, flashinfer_dit.py:143,192-226).
 * A solve with a new key runs eagerly, and the next solve with that same key captures it (a
 * capture costs more than one eager run, so a key used once is never captured).  Layouts
 * planned into one capacity share a key.  Results are identical either way.  n_steps <= 64. */
int fcv_dit_solve(FcvDit* dit, float* x, const float* mu, const float* cond, const float* spks,
                  const float* t_host, const float* dt_host, int32_t n_steps, float cfg,
                  int32_t use_graph, hipStream_t stream);

/* A solve schedule shared by handles: the modulation rows of an n_steps Euler schedule (every
 * block's AdaLN shift/scale/gate and the final (scale, shift), _project_modulations
 * flashinfer_dit.py:430-445) for t_host[0..n_steps),
 * computed once by fcv_dit_schedule into a caller buffer of fcv_dit_schedule_bytes(dit,
 * n_steps) bytes (256-byte aligned; 0 for an invalid n_steps).  fcv_dit_solve_scheduled is
 * fcv_dit_solve reading its modulation rows from that buffer instead of computing them: the
 * request groups of one solve, each on its own handle and stream over the same weights, pass
 * one buffer and pay for one pass over the AdaLN weights instead of one per group (the
 * reference's single packed batch computes them once, flashinfer_flow.py:16-74).  The buffer
 * must come from a handle over the same weights, hold at least n_steps steps, and stay intact
 * until every solve reading it has finished; its pointer is part of the captured graph's key.
 * Results are bit-identical to fcv_dit_solve with the same t_host. */
size_t fcv_dit_schedule_bytes(const FcvDit* dit, int32_t n_steps);
int fcv_dit_schedule(FcvDit* dit, const float* t_host, int32_t n_steps, void* schedule,
                     size_t schedule_bytes, hipStream_t stream);
int fcv_dit_solve_scheduled(FcvDit* dit, float* x, const float* mu, const float* cond,
                            const float* spks, const float* dt_host, int32_t n_steps, float cfg,
                            const void* schedule, size_t schedule_bytes, int32_t use_graph,
                            hipStream_t stream);

/* Padded channel-first [batch][channels][padded_len] <-> packed rows [rows][channels] for the
 * planned layout (document b = batch row b), used by the drop-in padded estimator call
 * (flashinfer_dit.py:469-471 gather, :536-543 scatter into zeros). */
int fcv_pack_padded(FcvDit* dit, const float* src, int32_t batch, int32_t channels,
                    int32_t padded_len, float* dst, hipStream_t stream);
int fcv_unpack_padded(FcvDit* dit, const float* src, int32_t batch, int32_t channels,
                      int32_t padded_len, float* dst, hipStream_t stream);

/* Solve graphs the handle holds (at most 4) and how many solves it has captured so far: a
 * layout planned into a captured capacity replays without a new capture.  No counterpart in the
 * reference beyond its plan_calls counter (flashinfer_attention.py:61-62). */
int fcv_dit_graph_stats(const FcvDit* dit, int32_t* pooled, int32_t* captures);

/* Planned layout facts (for callers sizing buffers): rows, documents, attention tiles. */
int fcv_dit_plan_info(const FcvDit* dit, int32_t* rows, int32_t* n_docs, int32_t* n_tiles);

/* Kernel timing probe.  No counterpart in the reference (whose only profiling hook is the
 * plan_calls counter, flashinfer_attention.py:61-62); it lets a benchmark time one kernel live
 * inside a solve.  Arms a probe on `stage`: during every later forward/solve call the library
 * records a HIP event pair (timing-only events, no system-scope fence) around that stage's
 * launch in block 1 (whose launches every later block repeats; block 0 for a one-block
 * model), or around
 * its one launch for stages outside the blocks, for the first n_pairs launches counted from the
 * start of the call.  With repeat > 1 the probed launch is issued
 * `repeat` times back to back between the two events, so per-launch event overhead is
 * amortised; only stages whose launch is idempotent accept repeat > 1 (QKV, attention, FF1,
 * LN-modulate, conv, AdaLN, input and output projections).  n_pairs == 0 disarms.  Arming or
 * disarming drops the captured graph.  fcv_dit_probe_read waits for the last pair and writes up
 * to `cap` per-launch durations in ms (pair time / repeat); *n_out = number of pairs recorded by
 * the last call. */
enum {
  FCV_STAGE_QKV = 0, FCV_STAGE_ATTENTION = 1, FCV_STAGE_OUT_PROJ = 2, FCV_STAGE_FF1 = 3,
  FCV_STAGE_FF2 = 4, FCV_STAGE_LN_MOD = 5, FCV_STAGE_CONV = 6, FCV_STAGE_ADALN = 7,
  FCV_STAGE_IN_PROJ = 8, FCV_STAGE_PROJ_OUT = 9, FCV_STAGE_EULER = 10, FCV_STAGE_FORWARD = 11,
  FCV_STAGE_COUNT = 12
};
int fcv_dit_probe_arm(FcvDit* dit, int32_t stage, int32_t n_pairs, int32_t repeat);
int fcv_dit_probe_read(FcvDit* dit, float* ms_out, int32_t cap, int32_t* n_out);

#ifdef __cplusplus
}
#endif

#endif /* FCV_DIT_H */
