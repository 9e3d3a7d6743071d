// C ABI of libfcvdit.so: handle, layout planning, the packed DiT forward, the CFG Euler
// step and the hipGraph-captured solve.  See include/fcv_dit.h for the contract.
#include <algorithm>
#include <climits>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/fcv_dit.h"
#include "kernels.hpp"
#include "status.hpp"

using fcv::f16;

namespace {

thread_local std::string g_error;

}  // namespace

int fcv::fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

using fcv::fail;

namespace {

constexpr size_t kAlign = 256;
constexpr int kMaxSteps = 64;
// solver steps whose AdaLN modulations one pass over the projection weights computes: the
// skinny-product kernel's row limit, whose rows are each computed exactly as a single row is
// (a 10-step solve reads the 281 MB of AdaLN weights once)
constexpr int kModGroup = 16;
constexpr int kRowTile = 128;
constexpr size_t kGraphPool = 4;   // captured solves kept per handle (least recently used goes)
constexpr size_t kSeenKeys = 8;    // solve keys remembered for the capture-on-second-sight rule

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Layout {
  // byte offsets inside the workspace
  size_t h, nbuf, obuf, q, k, vt, u, ain, vbuf;
  size_t docid, pos, ext_row, docid_ext, pos_ext, cu_int, lens, cu_ext, tiles, live;
  size_t mod, tsin, t1, t2, tbuf;
  size_t total;
};

// Internal rows: every document starts at a multiple of 8 rows (at most 7 pad rows each), so
// attention key tiles and 16-byte V^T loads are aligned to the document start.
long internal_rows_bound(long rows, long n_docs) { return rows + 7 * n_docs; }
long tiles_bound(long rows, long n_docs) {
  return internal_rows_bound(rows, n_docs) / fcv::kAttnTileQ + n_docs + 1;
}

// Workspace of a capacity: at most `rows` caller rows in at most `n_docs` documents.
Layout make_layout(const FcvDitDims& d, long rows, long n_docs) {
  const long ri = internal_rows_bound(rows, n_docs);
  const long rp = align_up(std::max<long>(ri, 1), kRowTile);
  const long n_tiles = tiles_bound(rows, n_docs);
  const long mod_width = (long)d.depth * 6 * d.dim + 2L * d.dim;
  const long nd = std::max<long>(n_docs, 1);
  Layout L{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, kAlign);
    return at;
  };
  L.h = take(rp * d.dim * 4);
  L.nbuf = take(rp * d.dim * 2);
  L.obuf = take(rp * d.dim * 2);
  L.q = take(rp * d.dim * 2);
  L.k = take(rp * d.dim * 2);
  L.vt = take(rp * d.dim * 2);
  L.u = take(rp * (long)d.ff_dim * 2);
  L.ain = take(rp * 4L * d.mel_dim * 2);
  L.vbuf = take(std::max<long>(rows, 1) * (long)d.mel_dim * 4);
  L.docid = take(rp * 4);
  L.pos = take(rp * 4);
  L.ext_row = take(rp * 4);
  L.docid_ext = take(std::max<long>(rows, 1) * 4);
  L.pos_ext = take(std::max<long>(rows, 1) * 4);
  L.cu_int = take((nd + 1) * 4);
  L.lens = take(nd * 4);
  L.cu_ext = take((nd + 1) * 4);
  L.tiles = take(n_tiles * fcv::kAttnTileInts * 4);
  L.live = take(4 * 4);
  const long nt = std::max<long>(nd, kModGroup);  // time rows: per document, or a step group
  L.mod = take(nt * mod_width * 4);
  L.tsin = take(nt * 256 * 2);
  L.t1 = take(nt * (long)d.dim * 2);
  L.t2 = take(nt * (long)d.dim * 2);
  L.tbuf = take(kMaxSteps * 4);
  L.total = off;
  return L;
}

}  // namespace

struct FcvDit {
  FcvDitDims dims{};
  FcvDitWeights w{};
  long mod_width = 0;

  // plan: `rows` caller rows (cu_host); `rows_int` internal 8-aligned rows.  The capacity
  // (rows_cap caller rows in docs_cap documents) sizes the workspace layout and every grid:
  // rint_cap internal rows, tiles_cap attention tiles, rc_cap caller rows per CFG half, rp the
  // row pitch of q, k and V^T.  The live counts sit in the workspace (Layout::live).
  bool planned = false;
  unsigned long generation = 0;
  int rows = 0, rows_int = 0, rp = 0, n_docs = 0, n_tiles = 0, mask_mode = 0, chunk = 0;
  int rows_cap = 0, docs_cap = 0, rint_cap = 0, tiles_cap = 0, rc_cap = 0;
  std::vector<int32_t> cu_host;
  char* ws = nullptr;
  size_t ws_bytes = 0;
  Layout L{};

  // timing probe (fcv_dit_probe_arm)
  int probe_stage = -1;
  int probe_pairs = 0;
  int probe_count = 0;
  int probe_repeat = 1;
  std::vector<hipEvent_t> probe_events;

  // graph pool: captured solves by key (capacity, mask, workspace, solver buffers, schedule),
  // most recently used first; seen: keys of recent solves (a key is captured on its second)
  struct Graph {
    std::vector<uintptr_t> key;
    hipGraphExec_t exec;
  };
  std::vector<Graph> graphs;
  std::vector<std::vector<uintptr_t>> seen;
  long captures = 0;  // solves captured into a graph over the handle's life

  template <class T>
  T* at(size_t off) const { return reinterpret_cast<T*>(ws + off); }
  const int32_t* live() const { return at<int32_t>(L.live); }

  void drop_graph() {
    for (Graph& g : graphs) (void)hipGraphExecDestroy(g.exec);
    graphs.clear();
    seen.clear();
  }

  void drop_probe() {
    for (hipEvent_t e : probe_events) (void)hipEventDestroy(e);
    probe_events.clear();
    probe_stage = -1;
    probe_pairs = 0;
    probe_count = 0;
    probe_repeat = 1;
  }

  // The probed launch of a stage: in block 1 (block 0 for a one-block model); layer -1 =
  // outside the blocks.
  bool probed(int stage, int layer) const {
    if (stage != probe_stage || probe_count >= probe_pairs) return false;
    const int target = dims.depth == 1 ? 0 : 1;
    return layer < 0 || layer == target;
  }
  hipError_t probe_begin(int stage, int layer, hipStream_t s) {
    if (!probed(stage, layer)) return hipSuccess;
    return hipEventRecord(probe_events[2 * probe_count], s);
  }
  // launches of `stage` in block `layer` to issue: `probe_repeat` while that launch is probed
  int launches(int stage, int layer) const { return probed(stage, layer) ? probe_repeat : 1; }
  hipError_t probe_end(int stage, int layer, hipStream_t s) {
    if (!probed(stage, layer)) return hipSuccess;
    return hipEventRecord(probe_events[2 * probe_count++ + 1], s);
  }
};

namespace {

// timestep embedding -> SiLU(temb) -> every block's AdaLN modulation in one projection, for
// n_t time values (device t): row i of `mod` (mod_width floats) belongs to t[i]
// (TimestepEmbedding modules.py:606-616; _project_modulations flashinfer_dit.py:430-445).
// tsin / t1 / t2: scratch for n_t rows of 256 / dim / dim fp16.
int modulation_rows(FcvDit* m, const float* t, int n_t, f16* tsin, f16* t1, f16* t2,
                    float* mod, hipStream_t s) {
  const FcvDitWeights& w = m->w;
  const int D = m->dims.dim;
  auto B = [](const void* p) { return reinterpret_cast<const f16*>(p); };
  FCV_HIP(fcv::timestep_sinusoid(t, n_t, 256, tsin, s));
  FCV_HIP(fcv::gemm_bias_silu_f16(tsin, 256, B(w.temb_w1), 256, w.temb_b1, n_t, D, 256, t1, D, s));
  FCV_HIP(fcv::gemm_bias_silu_f16(t1, D, B(w.temb_w2), D, w.temb_b2, n_t, D, D, t2, D, s));
  FCV_HIP(m->probe_begin(FCV_STAGE_ADALN, -1, s));
  for (int rep = m->launches(FCV_STAGE_ADALN, -1); rep > 0; --rep)
    FCV_HIP(fcv::gemm_bias_f32(t2, D, B(w.ada_w), D, w.ada_b, n_t, (int)m->mod_width, D, mod,
                               (int)m->mod_width, (int)m->mod_width, s));
  FCV_HIP(m->probe_end(FCV_STAGE_ADALN, -1, s));
  return FCV_OK;
}

// modulation_rows into the workspace's mod region
int compute_modulations(FcvDit* m, const float* t, int n_t, hipStream_t s) {
  return modulation_rows(m, t, n_t, m->at<f16>(m->L.tsin), m->at<f16>(m->L.t1),
                         m->at<f16>(m->L.t2), m->at<float>(m->L.mod), s);
}

// A solve schedule (fcv_dit_schedule): device t values, scratch for one group of kModGroup
// time rows, then every step's modulation row.
struct Schedule {
  size_t t, tsin, t1, t2, mod, total;
};
Schedule schedule_layout(const FcvDitDims& d, long n_steps) {
  Schedule S{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, kAlign);
    return at;
  };
  const long mod_width = (long)d.depth * 6 * d.dim + 2L * d.dim;
  S.t = take(kMaxSteps * 4);
  S.tsin = take(kModGroup * 256 * 2);
  S.t1 = take((long)kModGroup * d.dim * 2);
  S.t2 = take((long)kModGroup * d.dim * 2);
  S.mod = take(n_steps * mod_width * 4);
  S.total = off;
  return S;
}

int run_blocks(FcvDit* m, const float* x, const float* mu, const float* cond, const float* spks,
               const float* mod, long mod_stride, float* v_out, hipStream_t s);

// one estimator evaluation: modulations for t (1 shared value or one per document), then the
// network; `mod_row`, when not null, is an already computed shared-t modulation row
int run_forward(FcvDit* m, const float* x, const float* mu, const float* cond, const float* spks,
                const float* t, int n_t, const float* mod_row, float* v_out, hipStream_t s) {
  FCV_HIP(m->probe_begin(FCV_STAGE_FORWARD, -1, s));
  const float* mod = mod_row;
  long mod_stride = 0;
  if (!mod) {
    int rc = compute_modulations(m, t, n_t, s);
    if (rc != FCV_OK) return rc;
    mod = m->at<float>(m->L.mod);
    mod_stride = (n_t == 1) ? 0 : m->mod_width;
  }
  int rc = run_blocks(m, x, mu, cond, spks, mod, mod_stride, v_out, s);
  if (rc != FCV_OK) return rc;
  FCV_HIP(m->probe_end(FCV_STAGE_FORWARD, -1, s));
  return FCV_OK;
}

// The network on packed rows.  Every LayerNorm + modulation before a GEMM is a pass of its own
// (ln_mod_kernel, fp32 statistics) that writes the GEMM's normalized fp16 input: the same
// tensor the reference materializes (flashinfer_kernels.py:84-145).
int run_blocks(FcvDit* m, const float* x, const float* mu, const float* cond, const float* spks,
               const float* mod, long mod_stride, float* v_out, hipStream_t s) {
  const FcvDitDims& d = m->dims;
  const FcvDitWeights& w = m->w;
  // grids cover the plan's capacity; the kernels read the live counts
  const int R = m->rint_cap, D = d.dim, F = d.ff_dim, mel = d.mel_dim;
  const int32_t* live_rows = m->live() + fcv::kLiveRows;
  const int32_t* live_tiles = m->live() + fcv::kLiveTiles;
  auto B = [](const void* p) { return reinterpret_cast<const f16*>(p); };

  float* h = m->at<float>(m->L.h);
  f16* nbuf = m->at<f16>(m->L.nbuf);
  f16* obuf = m->at<f16>(m->L.obuf);
  f16* q = m->at<f16>(m->L.q);
  f16* k = m->at<f16>(m->L.k);
  f16* vt = m->at<f16>(m->L.vt);
  f16* u = m->at<f16>(m->L.u);
  f16* ain = m->at<f16>(m->L.ain);
  int32_t* docid = m->at<int32_t>(m->L.docid);
  int32_t* pos = m->at<int32_t>(m->L.pos);
  int32_t* ext_row = m->at<int32_t>(m->L.ext_row);
  int32_t* tiles = m->at<int32_t>(m->L.tiles);

  // input projection + causal conv position embedding (InputEmbedding dit.py:84-98)
  FCV_HIP(fcv::pack_inputs(x, cond, mu, spks, docid, ext_row, R, mel, ain, s, live_rows));
  FCV_HIP(m->probe_begin(FCV_STAGE_IN_PROJ, -1, s));
  for (int rep = m->launches(FCV_STAGE_IN_PROJ, -1); rep > 0; --rep)
    FCV_HIP(fcv::gemm_bias_f32_f16(ain, 4 * mel, B(w.in_w), 4 * mel, w.in_b, R, D, 4 * mel, h,
                                    nbuf, D, s, live_rows));
  FCV_HIP(m->probe_end(FCV_STAGE_IN_PROJ, -1, s));
  FCV_HIP(m->probe_begin(FCV_STAGE_CONV, -1, s));
  for (int rep = m->launches(FCV_STAGE_CONV, -1); rep > 0; --rep)
    FCV_HIP(fcv::conv_causal_mish(nbuf, D, B(w.conv1_w), w.conv1_b, d.conv_kernel, pos, R, obuf,
                                  nullptr, s, live_rows));
  FCV_HIP(m->probe_end(FCV_STAGE_CONV, -1, s));
  FCV_HIP(fcv::conv_causal_mish(obuf, D, B(w.conv2_w), w.conv2_b, d.conv_kernel, pos, R,
                                nullptr, h, s, live_rows));

  // transformer blocks (DiTBlock.forward modules.py:516-530)
  for (int l = 0; l < d.depth; ++l) {
    const long base = (long)l * 6 * D;
    FCV_HIP(m->probe_begin(FCV_STAGE_LN_MOD, l, s));
    for (int rep = m->launches(FCV_STAGE_LN_MOD, l); rep > 0; --rep)
      FCV_HIP(fcv::layer_norm_modulate(h, D, R, mod, mod_stride, (int)(base + 0), (int)(base + D),
                                       docid, nbuf, s, live_rows));
    FCV_HIP(m->probe_end(FCV_STAGE_LN_MOD, l, s));
    FCV_HIP(m->probe_begin(FCV_STAGE_QKV, l, s));
    for (int rep = m->launches(FCV_STAGE_QKV, l); rep > 0; --rep)
      FCV_HIP(fcv::gemm_qkv_rope(nbuf, D, B(w.qkv_w) + (long)l * 3 * D * D, D,
                                 w.qkv_b + (long)l * 3 * D, R, D, d.heads, pos, w.rope_cos,
                                 w.rope_sin, d.rope_dim, d.max_pos, q, k, vt, m->rp, s,
                                 live_rows));
    FCV_HIP(m->probe_end(FCV_STAGE_QKV, l, s));
    FCV_HIP(m->probe_begin(FCV_STAGE_ATTENTION, l, s));
    for (int rep = m->launches(FCV_STAGE_ATTENTION, l); rep > 0; --rep)
      FCV_HIP(fcv::attention_varlen(q, k, vt, obuf, tiles, m->tiles_cap, m->rp, d.heads,
                                    m->mask_mode == FCV_MASK_CHUNK_CAUSAL ? m->chunk : 0, s,
                                    live_tiles));
    FCV_HIP(m->probe_end(FCV_STAGE_ATTENTION, l, s));
    FCV_HIP(m->probe_begin(FCV_STAGE_OUT_PROJ, l, s));
    FCV_HIP(fcv::gemm_gated_residual(obuf, D, B(w.out_w) + (long)l * D * D, D,
                                     w.out_b + (long)l * D, R, D, D, h, D, mod + base + 2 * D,
                                     mod_stride, docid, s, live_rows));
    FCV_HIP(m->probe_end(FCV_STAGE_OUT_PROJ, l, s));
    FCV_HIP(fcv::layer_norm_modulate(h, D, R, mod, mod_stride, (int)(base + 3 * D),
                                     (int)(base + 4 * D), docid, nbuf, s, live_rows));
    FCV_HIP(m->probe_begin(FCV_STAGE_FF1, l, s));
    for (int rep = m->launches(FCV_STAGE_FF1, l); rep > 0; --rep)
      FCV_HIP(fcv::gemm_bias_gelu_f16(nbuf, D, B(w.ff1_w) + (long)l * F * D, D,
                                      w.ff1_b + (long)l * F, R, F, D, u, F, s, live_rows));
    FCV_HIP(m->probe_end(FCV_STAGE_FF1, l, s));
    FCV_HIP(m->probe_begin(FCV_STAGE_FF2, l, s));
    FCV_HIP(fcv::gemm_gated_residual(u, F, B(w.ff2_w) + (long)l * D * F, F,
                                     w.ff2_b + (long)l * D, R, D, F, h, D, mod + base + 5 * D,
                                     mod_stride, docid, s, live_rows));
    FCV_HIP(m->probe_end(FCV_STAGE_FF2, l, s));
  }

  // final AdaLN (scale, shift) + proj_out (dit.py:174-175, modules.py:260-265)
  const long fin = (long)d.depth * 6 * D;
  FCV_HIP(fcv::layer_norm_modulate(h, D, R, mod, mod_stride, (int)(fin + D), (int)fin, docid,
                                   nbuf, s, live_rows));
  FCV_HIP(m->probe_begin(FCV_STAGE_PROJ_OUT, -1, s));
  for (int rep = m->launches(FCV_STAGE_PROJ_OUT, -1); rep > 0; --rep)
    FCV_HIP(fcv::gemm_bias_f32_rowmap(nbuf, D, B(w.proj_w), D, w.proj_b, R, 128, D, v_out, mel,
                                      mel, ext_row, s, live_rows));
  FCV_HIP(m->probe_end(FCV_STAGE_PROJ_OUT, -1, s));
  return FCV_OK;
}

}  // namespace

extern "C" {

const char* fcv_last_error(void) { return g_error.c_str(); }

int fcv_dit_create(const FcvDitDims* dims, const FcvDitWeights* weights, FcvDit** out) {
  FCV_CHECK(dims && weights && out, FCV_ERR_INVALID, "null argument");
  const FcvDitDims& d = *dims;
  FCV_CHECK(d.dim == 1024, FCV_ERR_INVALID, "dim must be 1024");
  FCV_CHECK(d.dim_head == 64 && d.heads * d.dim_head == d.dim, FCV_ERR_INVALID,
            "heads * dim_head must equal dim with dim_head 64");
  FCV_CHECK(d.depth >= 1, FCV_ERR_INVALID, "depth must be >= 1");
  FCV_CHECK(d.ff_dim > 0 && d.ff_dim % 128 == 0, FCV_ERR_INVALID, "ff_dim must be a multiple of 128");
  FCV_CHECK(d.mel_dim > 0 && d.mel_dim % 16 == 0 && d.mel_dim <= 128, FCV_ERR_INVALID,
            "mel_dim must be a multiple of 16 and <= 128");
  FCV_CHECK(d.conv_groups * 64 == d.dim, FCV_ERR_INVALID, "conv groups must hold 64 channels");
  FCV_CHECK(d.conv_kernel >= 1 && d.conv_kernel <= 31, FCV_ERR_INVALID, "conv_kernel must be in [1, 31]");
  FCV_CHECK(d.rope_dim >= 0 && d.rope_dim <= d.dim_head && d.rope_dim % 16 == 0, FCV_ERR_INVALID,
            "rope_dim must be a multiple of 16 and <= dim_head");
  FCV_CHECK(d.max_pos >= 1, FCV_ERR_INVALID, "max_pos must be >= 1");
  const FcvDitWeights& w = *weights;
  const void* req[] = {w.temb_w1, w.temb_b1, w.temb_w2, w.temb_b2, w.ada_w, w.ada_b, w.in_w,
                       w.in_b, w.conv1_w, w.conv1_b, w.conv2_w, w.conv2_b, w.qkv_w, w.qkv_b,
                       w.out_w, w.out_b, w.ff1_w, w.ff1_b, w.ff2_w, w.ff2_b, w.proj_w, w.proj_b,
                       w.rope_cos, w.rope_sin};
  for (const void* p : req) FCV_CHECK(p != nullptr, FCV_ERR_INVALID, "null weight pointer");
  FcvDit* m = new FcvDit();
  m->dims = d;
  m->w = w;
  m->mod_width = (long)d.depth * 6 * d.dim + 2L * d.dim;
  *out = m;
  return FCV_OK;
}

int fcv_dit_destroy(FcvDit* dit) {
  if (!dit) return FCV_OK;
  dit->drop_graph();
  dit->drop_probe();
  delete dit;
  return FCV_OK;
}

size_t fcv_dit_workspace_bytes(const FcvDit* dit, int32_t rows, int32_t n_docs) {
  if (!dit || rows < 0 || n_docs < 0) return 0;
  return make_layout(dit->dims, rows, n_docs).total;
}

int fcv_dit_plan_capacity(FcvDit* m, const int32_t* cu_host, int32_t n_docs, int32_t mask_mode,
                          int32_t chunk, int32_t rows_cap, int32_t docs_cap, void* workspace,
                          size_t workspace_bytes, hipStream_t s) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(cu_host && n_docs >= 1, FCV_ERR_INVALID, "need at least one document");
  FCV_CHECK(mask_mode == FCV_MASK_FULL || mask_mode == FCV_MASK_CHUNK_CAUSAL, FCV_ERR_INVALID,
            "mask_mode must be 0 (full) or 1 (chunk-causal)");
  FCV_CHECK(mask_mode == FCV_MASK_FULL || chunk >= 1, FCV_ERR_INVALID, "chunk must be >= 1");
  FCV_CHECK(cu_host[0] == 0, FCV_ERR_INVALID, "cu_seqlens[0] must be 0");
  for (int d = 0; d < n_docs; ++d) {
    const long len = (long)cu_host[d + 1] - cu_host[d];
    FCV_CHECK(len >= 1, FCV_ERR_INVALID,
              "document " + std::to_string(d) + " has length " + std::to_string(len) + " (< 1)");
    FCV_CHECK(len <= m->dims.max_pos, FCV_ERR_INVALID,
              "document " + std::to_string(d) + " is longer than max_pos " +
                  std::to_string(m->dims.max_pos));
  }
  const int rows = cu_host[n_docs];
  FCV_CHECK(rows <= rows_cap && n_docs <= docs_cap, FCV_ERR_INVALID,
            "layout of " + std::to_string(rows) + " rows in " + std::to_string(n_docs) +
                " documents exceeds the capacity (" + std::to_string(rows_cap) + " rows, " +
                std::to_string(docs_cap) + " documents)");
  // the kernels address activations by 32-bit byte offsets within buffer ranges held as an
  // int: the widest row (the FF hidden row in f16 or the fp32 residual row) times the internal
  // rows of the capacity must stay below 2 GB
  const long row_bytes = std::max<long>(2L * m->dims.ff_dim, 4L * m->dims.dim);
  FCV_CHECK(align_up(internal_rows_bound(rows_cap, docs_cap), kRowTile) * row_bytes < (1L << 31),
            FCV_ERR_INVALID,
            "too many rows: (rows + 7 per document) x " + std::to_string(row_bytes) +
                " bytes must stay below 2 GB");

  // internal layout: document starts rounded up to multiples of 8 rows
  std::vector<int32_t> cu_int(n_docs + 1, 0), lens(n_docs);
  for (int d = 0; d < n_docs; ++d) {
    lens[d] = cu_host[d + 1] - cu_host[d];
    cu_int[d + 1] = cu_int[d] + (int32_t)align_up(lens[d], 8);
  }
  const int rows_int = cu_int[n_docs];

  // attention tiles: {doc start, doc length, first query row, 0} in internal rows, most
  // expensive first (LPT order)
  struct T { int doc, q0; long cost; };
  std::vector<T> tl;
  for (int d = 0; d < n_docs; ++d) {
    const int start = cu_int[d], end = cu_int[d] + lens[d];
    for (int q0 = start; q0 < end; q0 += fcv::kAttnTileQ) {
      int q_last = std::min(q0 + fcv::kAttnTileQ - 1, end - 1);
      long kv = end - start;
      if (mask_mode == FCV_MASK_CHUNK_CAUSAL)
        kv = std::min<long>(kv, ((q_last - start) / chunk + 1) * (long)chunk);
      tl.push_back({d, q0, kv});
    }
  }
  std::stable_sort(tl.begin(), tl.end(), [](const T& a, const T& b) { return a.cost > b.cost; });
  std::vector<int32_t> tiles_host;
  tiles_host.reserve(tl.size() * fcv::kAttnTileInts);
  for (const T& t : tl) {
    tiles_host.push_back(cu_int[t.doc]);
    tiles_host.push_back(lens[t.doc]);
    tiles_host.push_back(t.q0);
    tiles_host.push_back(0);
  }

  const Layout L = make_layout(m->dims, rows_cap, docs_cap);
  FCV_CHECK(workspace != nullptr, FCV_ERR_INVALID, "null workspace");
  FCV_CHECK(workspace_bytes >= L.total, FCV_ERR_INVALID,
            "workspace too small: need " + std::to_string(L.total) + " bytes, got " +
                std::to_string(workspace_bytes));
  FCV_CHECK(reinterpret_cast<uintptr_t>(workspace) % kAlign == 0, FCV_ERR_INVALID,
            "workspace must be 256-byte aligned");

  m->planned = false;
  m->ws = static_cast<char*>(workspace);
  m->ws_bytes = workspace_bytes;
  m->L = L;
  m->rows = rows;
  m->rows_int = rows_int;
  m->n_docs = n_docs;
  m->n_tiles = (int)tl.size();
  m->mask_mode = mask_mode;
  m->chunk = mask_mode == FCV_MASK_CHUNK_CAUSAL ? chunk : 0;
  m->cu_host.assign(cu_host, cu_host + n_docs + 1);
  m->rows_cap = rows_cap;
  m->docs_cap = docs_cap;
  m->rint_cap = (int)internal_rows_bound(rows_cap, docs_cap);
  m->tiles_cap = (int)tiles_bound(rows_cap, docs_cap);
  m->rc_cap = rows_cap / 2;
  m->rp = (int)align_up(std::max(m->rint_cap, 1), kRowTile);
  const std::vector<int32_t> live = {rows_int, m->n_tiles, rows / 2, 0};

  auto h2d = [&](size_t off, const std::vector<int32_t>& v) {
    return hipMemcpyAsync(m->ws + off, v.data(), v.size() * sizeof(int32_t),
                          hipMemcpyHostToDevice, s);
  };
  FCV_HIP(h2d(L.cu_ext, m->cu_host));
  FCV_HIP(h2d(L.cu_int, cu_int));
  FCV_HIP(h2d(L.lens, lens));
  FCV_HIP(h2d(L.tiles, tiles_host));
  FCV_HIP(h2d(L.live, live));
  FCV_HIP(fcv::build_row_index(m->at<int32_t>(L.cu_ext), n_docs, rows,
                               m->at<int32_t>(L.docid_ext), m->at<int32_t>(L.pos_ext), s));
  FCV_HIP(fcv::build_aligned_row_index(m->at<int32_t>(L.cu_int), m->at<int32_t>(L.lens),
                                       m->at<int32_t>(L.cu_ext), n_docs, rows_int,
                                       m->at<int32_t>(L.docid), m->at<int32_t>(L.pos),
                                       m->at<int32_t>(L.ext_row), s));
  FCV_HIP(hipStreamSynchronize(s));
  m->planned = true;
  m->generation++;
  return FCV_OK;
}

int fcv_dit_plan(FcvDit* m, const int32_t* cu_host, int32_t n_docs, int32_t mask_mode,
                 int32_t chunk, void* workspace, size_t workspace_bytes, hipStream_t s) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(cu_host && n_docs >= 1, FCV_ERR_INVALID, "need at least one document");
  return fcv_dit_plan_capacity(m, cu_host, n_docs, mask_mode, chunk, cu_host[n_docs], n_docs,
                               workspace, workspace_bytes, s);
}

int fcv_dit_graph_stats(const FcvDit* m, int32_t* pooled, int32_t* captures) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  if (pooled) *pooled = (int32_t)m->graphs.size();
  if (captures) *captures = (int32_t)std::min<long>(m->captures, INT32_MAX);
  return FCV_OK;
}

int fcv_dit_plan_info(const FcvDit* m, int32_t* rows, int32_t* n_docs, int32_t* n_tiles) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "no layout planned");
  if (rows) *rows = m->rows;
  if (n_docs) *n_docs = m->n_docs;
  if (n_tiles) *n_tiles = m->n_tiles;
  return FCV_OK;
}

int fcv_dit_forward(FcvDit* m, const float* x, const float* mu, const float* cond,
                    const float* spks, const float* t, int32_t n_t, float* v_out,
                    hipStream_t s) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "fcv_dit_forward called before fcv_dit_plan");
  FCV_CHECK(x && mu && cond && spks && t && v_out, FCV_ERR_INVALID,
            "spks and cond are required (null input pointer)");
  FCV_CHECK(n_t == 1 || n_t == m->n_docs, FCV_ERR_INVALID, "n_t must be 1 or n_docs");
  m->probe_count = 0;
  return run_forward(m, x, mu, cond, spks, t, n_t, nullptr, v_out, s);
}

static int check_cfg_layout(const FcvDit* m) {
  FCV_CHECK(m->n_docs % 2 == 0, FCV_ERR_INVALID, "CFG batch needs an even number of documents");
  const int half = m->n_docs / 2;
  for (int d = 0; d < half; ++d) {
    FCV_CHECK(m->cu_host[d + 1] - m->cu_host[d] == m->cu_host[half + d + 1] - m->cu_host[half + d],
              FCV_ERR_INVALID, "CFG halves must have equal document lengths");
  }
  return FCV_OK;
}

int fcv_euler_cfg_step(FcvDit* m, float* x, const float* v, float dt, float cfg, hipStream_t s) {
  FCV_CHECK(m && x && v, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "no layout planned");
  int rc = check_cfg_layout(m);
  if (rc != FCV_OK) return rc;
  FCV_HIP(fcv::euler_cfg_update(x, v, m->rows / 2, m->dims.mel_dim, dt, cfg, s));
  return FCV_OK;
}

}  // extern "C"

namespace {

// The CFG Euler loop of fcv_dit_solve (sched == nullptr: the modulation rows are computed in
// the loop, kModGroup steps per pass over the AdaLN weights) and of fcv_dit_solve_scheduled
// (sched: a schedule buffer holding every step's rows).
int solve_loop(FcvDit* m, float* x, const float* mu, const float* cond, const float* spks,
               const float* t_host, const float* dt_host, int32_t n_steps, float cfg,
               const char* sched, int32_t use_graph, hipStream_t s) {
  int rc = check_cfg_layout(m);
  if (rc != FCV_OK) return rc;

  float* tbuf = m->at<float>(m->L.tbuf);
  float* vbuf = m->at<float>(m->L.vbuf);
  const int mel = m->dims.mel_dim;
  const Schedule S = schedule_layout(m->dims, n_steps);
  if (!sched)
    FCV_HIP(hipMemcpyAsync(tbuf, t_host, n_steps * sizeof(float), hipMemcpyHostToDevice, s));

  auto body = [&]() -> int {
    m->probe_count = 0;
    const float* mod = sched ? reinterpret_cast<const float*>(sched + S.mod) : m->at<float>(m->L.mod);
    for (int step = 0; step < n_steps; ++step) {
      // every kModGroup steps, one pass over the AdaLN weights gives the next steps' rows
      if (!sched && step % kModGroup == 0) {
        int r = compute_modulations(m, tbuf + step, std::min(kModGroup, n_steps - step), s);
        if (r != FCV_OK) return r;
      }
      const int row = sched ? step : step % kModGroup;
      int r = run_forward(m, x, mu, cond, spks, nullptr, 1, mod + row * m->mod_width, vbuf, s);
      if (r != FCV_OK) return r;
      FCV_HIP(m->probe_begin(FCV_STAGE_EULER, -1, s));
      FCV_HIP(fcv::euler_cfg_update(x, vbuf, m->rc_cap, mel, dt_host[step], cfg, s,
                                    m->live() + fcv::kLiveHalfRows));
      FCV_HIP(m->probe_end(FCV_STAGE_EULER, -1, s));
    }
    return FCV_OK;
  };
  // What a captured loop bakes in: the capacity (workspace offsets and grids), the mask, the
  // workspace and solver buffers, the schedule buffer, and the schedule (t is read from tbuf or
  // the schedule buffer).  The layout itself is read from the workspace at run time, so any
  // layout planned into the same capacity replays.
  std::vector<uintptr_t> key = {(uintptr_t)m->rows_cap, (uintptr_t)m->docs_cap,
                                (uintptr_t)m->mask_mode, (uintptr_t)m->chunk, (uintptr_t)m->ws,
                                (uintptr_t)x, (uintptr_t)mu, (uintptr_t)cond, (uintptr_t)spks,
                                (uintptr_t)sched, (uintptr_t)n_steps};
  uint32_t bits;
  std::memcpy(&bits, &cfg, 4);
  key.push_back(bits);
  for (int i = 0; i < n_steps; ++i) {
    std::memcpy(&bits, &dt_host[i], 4);
    key.push_back(bits);
  }
  if (!use_graph) return body();
  auto hit = std::find_if(m->graphs.begin(), m->graphs.end(),
                          [&](const FcvDit::Graph& g) { return g.key == key; });
  if (hit == m->graphs.end()) {
    // Capturing and instantiating the loop costs more than running it once eagerly, so a key is
    // captured on its second solve: a capacity used once never pays for a capture.
    auto seen = std::find(m->seen.begin(), m->seen.end(), key);
    if (seen == m->seen.end()) {
      m->seen.insert(m->seen.begin(), key);
      if (m->seen.size() > kSeenKeys) m->seen.pop_back();
      return body();
    }
    m->seen.erase(seen);
    FCV_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int r = body();
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (r != FCV_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return r;
    }
    if (e != hipSuccess)
      return fail(FCV_ERR_RUNTIME, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess)
      return fail(FCV_ERR_RUNTIME, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    if (m->graphs.size() >= kGraphPool) {
      (void)hipGraphExecDestroy(m->graphs.back().exec);
      m->graphs.pop_back();
    }
    m->graphs.insert(m->graphs.begin(), FcvDit::Graph{key, exec});
    m->captures++;
  } else if (hit != m->graphs.begin()) {
    std::rotate(m->graphs.begin(), hit, hit + 1);  // most recently used first
  }
  FCV_HIP(hipGraphLaunch(m->graphs.front().exec, s));
  return FCV_OK;
}

}  // namespace

extern "C" {

int fcv_dit_solve(FcvDit* m, float* x, const float* mu, const float* cond, const float* spks,
                  const float* t_host, const float* dt_host, int32_t n_steps, float cfg,
                  int32_t use_graph, hipStream_t s) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "fcv_dit_solve called before fcv_dit_plan");
  FCV_CHECK(x && mu && cond && spks && t_host && dt_host, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(n_steps >= 1 && n_steps <= kMaxSteps, FCV_ERR_INVALID, "n_steps must be in [1, 64]");
  return solve_loop(m, x, mu, cond, spks, t_host, dt_host, n_steps, cfg, nullptr, use_graph, s);
}

size_t fcv_dit_schedule_bytes(const FcvDit* m, int32_t n_steps) {
  if (!m || n_steps < 1 || n_steps > kMaxSteps) return 0;
  return schedule_layout(m->dims, n_steps).total;
}

int fcv_dit_schedule(FcvDit* m, const float* t_host, int32_t n_steps, void* sched,
                     size_t sched_bytes, hipStream_t s) {
  FCV_CHECK(m && t_host && sched, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(n_steps >= 1 && n_steps <= kMaxSteps, FCV_ERR_INVALID, "n_steps must be in [1, 64]");
  FCV_CHECK(((uintptr_t)sched) % kAlign == 0, FCV_ERR_INVALID,
            "schedule buffer must be 256-byte aligned");
  const Schedule S = schedule_layout(m->dims, n_steps);
  FCV_CHECK(sched_bytes >= S.total, FCV_ERR_INVALID, "schedule buffer too small");
  char* b = static_cast<char*>(sched);
  float* t = reinterpret_cast<float*>(b + S.t);
  FCV_HIP(hipMemcpyAsync(t, t_host, n_steps * sizeof(float), hipMemcpyHostToDevice, s));
  for (int step = 0; step < n_steps; step += kModGroup) {
    int r = modulation_rows(m, t + step, std::min(kModGroup, n_steps - step),
                            reinterpret_cast<f16*>(b + S.tsin), reinterpret_cast<f16*>(b + S.t1),
                            reinterpret_cast<f16*>(b + S.t2),
                            reinterpret_cast<float*>(b + S.mod) + step * m->mod_width, s);
    if (r != FCV_OK) return r;
  }
  return FCV_OK;
}

int fcv_dit_solve_scheduled(FcvDit* m, float* x, const float* mu, const float* cond,
                            const float* spks, const float* dt_host, int32_t n_steps, float cfg,
                            const void* sched, size_t sched_bytes, int32_t use_graph,
                            hipStream_t s) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "fcv_dit_solve_scheduled called before fcv_dit_plan");
  FCV_CHECK(x && mu && cond && spks && dt_host && sched, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(n_steps >= 1 && n_steps <= kMaxSteps, FCV_ERR_INVALID, "n_steps must be in [1, 64]");
  FCV_CHECK(sched_bytes >= schedule_layout(m->dims, n_steps).total, FCV_ERR_INVALID,
            "schedule buffer too small for n_steps");
  return solve_loop(m, x, mu, cond, spks, nullptr, dt_host, n_steps, cfg,
                    static_cast<const char*>(sched), use_graph, s);
}

int fcv_pack_padded(FcvDit* m, const float* src, int32_t batch, int32_t channels,
                    int32_t padded_len, float* dst, hipStream_t s) {
  FCV_CHECK(m && src && dst, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "no layout planned");
  FCV_CHECK(batch == m->n_docs, FCV_ERR_INVALID, "batch must equal the planned document count");
  for (int d = 0; d < m->n_docs; ++d)
    FCV_CHECK(m->cu_host[d + 1] - m->cu_host[d] <= padded_len, FCV_ERR_INVALID,
              "document longer than padded_len");
  FCV_HIP(fcv::pack_padded(src, batch, channels, padded_len, m->at<int32_t>(m->L.cu_ext),
                           m->at<int32_t>(m->L.docid_ext), m->at<int32_t>(m->L.pos_ext), m->rows,
                           dst, s));
  return FCV_OK;
}

int fcv_unpack_padded(FcvDit* m, const float* src, int32_t batch, int32_t channels,
                      int32_t padded_len, float* dst, hipStream_t s) {
  FCV_CHECK(m && src && dst, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(m->planned, FCV_ERR_STATE, "no layout planned");
  FCV_CHECK(batch == m->n_docs, FCV_ERR_INVALID, "batch must equal the planned document count");
  for (int d = 0; d < m->n_docs; ++d)
    FCV_CHECK(m->cu_host[d + 1] - m->cu_host[d] <= padded_len, FCV_ERR_INVALID,
              "document longer than padded_len");
  FCV_HIP(fcv::unpack_padded(src, batch, channels, padded_len, m->at<int32_t>(m->L.cu_ext), dst,
                             s));
  return FCV_OK;
}

int fcv_dit_probe_arm(FcvDit* m, int32_t stage, int32_t n_pairs, int32_t repeat) {
  FCV_CHECK(m, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(stage >= 0 && stage < FCV_STAGE_COUNT, FCV_ERR_INVALID, "unknown stage");
  FCV_CHECK(n_pairs >= 0 && n_pairs <= 4096, FCV_ERR_INVALID, "n_pairs must be in [0, 4096]");
  FCV_CHECK(repeat >= 1 && repeat <= 64, FCV_ERR_INVALID, "repeat must be in [1, 64]");
  // stages whose launch accumulates into its output (gated residuals, conv2, Euler) or that
  // span several launches cannot be repeated
  const bool idempotent = stage != FCV_STAGE_OUT_PROJ && stage != FCV_STAGE_FF2 &&
                          stage != FCV_STAGE_EULER && stage != FCV_STAGE_FORWARD;
  FCV_CHECK(repeat == 1 || idempotent, FCV_ERR_INVALID,
            "repeat > 1 needs a stage whose launch is idempotent");
  m->drop_graph();
  m->drop_probe();
  if (n_pairs == 0) return FCV_OK;
  m->probe_events.resize(2 * n_pairs, nullptr);
  for (auto& e : m->probe_events) {
    // timing-only events: no system-scope fence (and its cache write-back) at each record,
    // so a pair measures the kernel between them, as a kernel trace does
    hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
    if (err != hipSuccess) {
      m->drop_probe();
      return fail(FCV_ERR_RUNTIME, std::string("hipEventCreate: ") + hipGetErrorString(err));
    }
  }
  m->probe_stage = stage;
  m->probe_pairs = n_pairs;
  m->probe_repeat = repeat;
  return FCV_OK;
}

int fcv_dit_probe_read(FcvDit* m, float* ms_out, int32_t cap, int32_t* n_out) {
  FCV_CHECK(m && ms_out && n_out, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(m->probe_stage >= 0, FCV_ERR_STATE, "no probe armed");
  const int n = std::min(m->probe_count, (int)cap);
  if (n > 0) FCV_HIP(hipEventSynchronize(m->probe_events[2 * (m->probe_count - 1) + 1]));
  for (int i = 0; i < n; ++i) {
    FCV_HIP(hipEventElapsedTime(&ms_out[i], m->probe_events[2 * i], m->probe_events[2 * i + 1]));
    ms_out[i] /= (float)m->probe_repeat;
  }
  *n_out = m->probe_count;
  return FCV_OK;
}

}  // extern "C"
