// Host-side launchers of the gfx950 DiT estimator kernels (one .hip file per kernel family).
// All launchers are asynchronous on `stream` and return hipGetLastError() of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace fcv {

// ---- live counts -------------------------------------------------------------------------
// A planned layout's counts as the kernels read them from device memory (int32[4] in the
// workspace): the grids are sized for the plan's capacity and the workgroups past the live
// count exit at once, so a graph captured for a capacity replays for any layout that fits it.
// Launchers given live == nullptr use their static count arguments.
enum { kLiveRows = 0, kLiveTiles = 1, kLiveHalfRows = 2 };  // internal rows, attention tiles, rc

// ---- GEMM: C[M,N] = A[M,K] . W[N,K]^T (+ bias) with a fused epilogue -------------------
// Requirements checked by the caller: N % 128 == 0, K % 64 == 0, lda/ldw % 8 == 0.
// M is the capacity the grid is sized for; m_live (when not null) holds the live row count
// (<= M).

// out_f32[r, c] = acc + bias[c];  out_f16[r, c] = f16(same)   (input projection)
hipError_t gemm_bias_f32_f16(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                              int M, int N, int K, float* out_f32, f16* out_f16, int ldo,
                              hipStream_t stream, const int32_t* m_live = nullptr);

// out[r, c] = acc + bias[c] for c < n_valid (fp32; AdaLN projection)
hipError_t gemm_bias_f32(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                         int M, int N, int K, float* out, int ldo, int n_valid, hipStream_t stream);

// out[row_map[r], c] = acc + bias[c] for c < n_valid and row_map[r] >= 0 (proj_out)
hipError_t gemm_bias_f32_rowmap(const f16* A, int lda, const f16* W, int ldw,
                                const float* bias, int M, int N, int K, float* out, int ldo,
                                int n_valid, const int32_t* row_map, hipStream_t stream,
                                const int32_t* m_live = nullptr);

// out[r, c] = f16(silu(acc + bias[c]))   (timestep MLP)
hipError_t gemm_bias_silu_f16(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                               int M, int N, int K, f16* out, int ldo, hipStream_t stream);

// out[r, c] = f16(gelu_tanh(acc + bias[c]))   (FF1)
hipError_t gemm_bias_gelu_f16(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                              int M, int N, int K, f16* out, int ldo, hipStream_t stream,
                              const int32_t* m_live = nullptr);

// h[r, c] += gate[c] * (acc + bias[c]), gate row = mod + docid[r] * mod_stride + gate_off
// (out-projection and FF2 gated residuals).
hipError_t gemm_gated_residual(const f16* A, int lda, const f16* W, int ldw, const float* bias,
                               int M, int N, int K, float* h, int ldh, const float* mod,
                               long mod_stride, const int32_t* docid, hipStream_t stream,
                               const int32_t* m_live = nullptr);

// Fused QKV projection: bias, interleaved RoPE on columns [0, rope_dim) of q and k
// (angles from cos/sin tables [max_pos][rope_dim/2], row position min(pos[r], max_pos-1)),
// scatter to q, k : [heads][rp][dim_head] and vt : [heads][dim_head][rp] (V transposed).
hipError_t gemm_qkv_rope(const f16* A, int lda, const f16* W, int ldw, const float* bias, int M,
                         int dim, int heads, const int32_t* pos, const float* rope_cos,
                         const float* rope_sin, int rope_dim, int max_pos, f16* q, f16* k,
                         f16* vt, int rp, hipStream_t stream, const int32_t* m_live = nullptr);

// ---- skinny products (few rows sharing W, K in {512, 1024}): bandwidth-bound, no MFMA -------
// Launches of up to 16 rows each; a row's result is the same whatever M is.
bool gemv_supported(int M, int K, int lda, int ldw);
// out[m, n] = acc + bias[n]
hipError_t gemv_bias_f32(const f16* a, int lda, const f16* W, int ldw, const float* bias, int M,
                         int N, int K, float* out, int ldo, hipStream_t stream);
// out[m, n] = f16(silu(acc + bias[n]))
hipError_t gemv_bias_silu_f16(const f16* a, int lda, const f16* W, int ldw, const float* bias,
                               int M, int N, int K, f16* out, int ldo, hipStream_t stream);

// ---- attention ----------------------------------------------------------------------------
// Varlen attention, head_dim 64.  tiles (16-byte aligned) holds one 4-int entry per tile of
// kAttnTileQ queries: {document start row (a multiple of 8), document length, first query
// row, unused}.  q, k: [heads][rp][64], vt: [heads][64][rp].  chunk == 0: full attention
// inside each document; chunk > 0: key visible iff (key_pos / chunk) <= (query_pos / chunk).
// n_tiles is the grid's capacity; tiles_live (when not null) holds the live tile count.
hipError_t attention_varlen(const f16* q, const f16* k, const f16* vt, f16* o,
                            const int32_t* tiles, int n_tiles, int rp, int heads, int chunk,
                            hipStream_t stream, const int32_t* tiles_live = nullptr);
constexpr int kAttnTileInts = 4;  // ints per tile entry
constexpr int kAttnTileQ = 128;

// ---- causal grouped conv position embedding (64 channels per group) -------------------------
// y[r, g*64+co] = mish(bias + sum_{j,ci} W[g][j][co][ci] x[r-(taps-1)+j, g*64+ci]), rows before
// the row's document start read as zero.  out_f16 != null: store y;  h != null: h += y.
hipError_t conv_causal_mish(const f16* x, int C, const f16* w, const float* bias, int taps,
                            const int32_t* pos, int rows, f16* out_f16, float* h,
                            hipStream_t stream, const int32_t* rows_live = nullptr);

// ---- bandwidth-bound kernels -----------------------------------------------------------------
// out[r, :] = f16(LN(h[r, :]) * scale + shift), scale/shift rows = mod + docid[r]*mod_stride + off
hipError_t layer_norm_modulate(const float* h, int C, int rows, const float* mod, long mod_stride,
                               int shift_off, int scale_off, const int32_t* docid, f16* out,
                               hipStream_t stream, const int32_t* rows_live = nullptr);

// docid[r], pos[r] from device cu_seqlens[n_docs+1].
hipError_t build_row_index(const int32_t* cu_seqlens, int n_docs, int rows, int32_t* docid,
                           int32_t* pos, hipStream_t stream);

// Internal (8-row aligned) layout: document d owns internal rows [cu_int[d], cu_int[d+1]) of
// which the first lens[d] are real.  docid/pos of every internal row; ext_row = caller row of
// a real row, -1 for a pad row.
hipError_t build_aligned_row_index(const int32_t* cu_int, const int32_t* lens,
                                   const int32_t* cu_ext, int n_docs, int rows_int, int32_t* docid,
                                   int32_t* pos, int32_t* ext_row, hipStream_t stream);

// a[r, 0:4*mel] = f16([x[e], cond[e], mu[e], spks[docid[r]]]) with e = ext_row[r]; zeros when e < 0
hipError_t pack_inputs(const float* x, const float* cond, const float* mu, const float* spks,
                       const int32_t* docid, const int32_t* ext_row, int rows, int mel, f16* a,
                       hipStream_t stream, const int32_t* rows_live = nullptr);

// out[m, 0:dim] = f16([sin(1000 t_m f), cos(1000 t_m f)]), f_i = exp(-i ln(1e4)/(dim/2-1))
hipError_t timestep_sinusoid(const float* t, int n_t, int dim, f16* out, hipStream_t stream);

// x[r] += dt * ((1+cfg) v[r] - cfg v[r+rc]); x[r+rc] = x[r]   for r < rc
// (rc = rc_live[0] when rc_live is not null; the grid covers the capacity rc)
hipError_t euler_cfg_update(float* x, const float* v, int rc, int mel, float dt, float cfg,
                            hipStream_t stream, const int32_t* rc_live = nullptr);

// [B, C, T] channel-first padded <-> packed rows [R, C]
hipError_t pack_padded(const float* src, int batch, int channels, int padded_len,
                       const int32_t* cu_seqlens, const int32_t* docid, const int32_t* pos,
                       int rows, float* dst, hipStream_t stream);
hipError_t unpack_padded(const float* src, int batch, int channels, int padded_len,
                         const int32_t* cu_seqlens, float* dst, hipStream_t stream);

}  // namespace fcv
