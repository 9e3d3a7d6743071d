// Flow front-end on gfx950: token embedding + PreLookaheadLayer + repeat to Mel rows, the
// speaker projection and the prompt copy into the condition (see include/fcv_flow.h).
//
// The front-end runs once per request, in fp32 (the reference runs it in the flow's dtype).
// Both convolutions are GEMMs with a gathered operand and run on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32):
//   conv1: H^T[c][t]  = W1[c][k] . E[k][t],  k = tap * F + i,  E[tap*F+i][t] = e(t + tap)[i]
//   conv2: Y^T[o][t]  = W2[o][k] . G[k][t],  k = tap * C + c,  G[tap*C+c][t] = h(t - 2 + tap)[c]
// with the weights as the A operand (rows = output channels) and the gathered token rows as
// the B operand, so a lane's four accumulators are four consecutive channels of one token and
// leave as one 16-byte store.  Both operands are staged through LDS K-contiguous, 16 K values
// per chunk; lane (i, g) of the 16x16x4 MFMA feeds k = 4g + s at step s, so one 16-byte LDS
// read covers four steps.  conv2 (80 outputs, K = 3072) splits K eight ways into partial sums
// that a finishing kernel adds in a fixed order together with the bias, the residual and the
// repeat to Mel rows.  No tile or split depends on the batch, so a document's result does not
// depend on what it is packed with.  The per-document prefix sums travel by value in the kernel
// arguments (DocTables, at most kMaxDocs documents), so a call needs no host-to-device copy and
// no synchronisation.
#include <mutex>
#include <string>

#include "../../include/fcv_flow.h"
#include "kernels.hpp"
#include "status.hpp"

namespace fcv {
namespace {

constexpr int kFeat = 80;     // supported feat_dim
constexpr int kBK = 16;       // K values per LDS chunk
constexpr int kPitch = 20;    // LDS row pitch in floats (16 + 4: conflict-free 16-byte reads)
constexpr int kSplit = 8;     // conv2 K split (fixed)
constexpr int kTileT = 64;    // token rows per workgroup (both convolutions)
constexpr int kTileC = 128;   // conv1 output channels per workgroup
constexpr size_t kAlign = 256;
constexpr int kMaxDocs = FCV_FLOW_MAX_DOCS;

// two exclusive prefix sums over the documents of a call, passed by value
struct DocTables {
  int32_t a[kMaxDocs + 1];
  int32_t b[kMaxDocs + 1];
};
static_assert(sizeof(DocTables) <= 2304, "document tables must fit the kernel arguments");

__device__ __forceinline__ f32x4 mfma16(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// largest d with cu[d] <= row (cu non-decreasing, cu[0] = 0 <= row)
__device__ __forceinline__ int find_doc(const int32_t* cu, int n_docs, int row) {
  int lo = 0, hi = n_docs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ float leaky_relu(float x) { return x > 0.0f ? x : 0.01f * x; }

// ---- conv1: h[t][c] = leaky_relu(b1[c] + sum_k W1[c][k] E[k][t]) ---------------------------
// Workgroup tile 128 channels x 64 tokens; wave (wc, wt) owns 64 channels x 32 tokens.
// tab.a = token prefix sums, tab.b = output-token prefix sums
__global__ __launch_bounds__(256) void lookahead_conv1_kernel(
    const int32_t* __restrict__ tokens, const DocTables tab, int n_docs, int n_out,
    const float* __restrict__ embed, int vocab, const float* __restrict__ W1,
    const float* __restrict__ b1, int C, int taps, float* __restrict__ h) {
  __shared__ __attribute__((aligned(16))) float sA[2][kTileC][kPitch];
  __shared__ __attribute__((aligned(16))) float sB[2][kTileT][kPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wc = wave & 1, wt = wave >> 1;
  const int li = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * kTileT;
  const int c0 = blockIdx.y * kTileC;
  const int K = taps * kFeat;
  constexpr int CPT = kFeat / kBK;  // chunks per tap
  const int KC = taps * CPT;

  // loader roles: weight rows lr and lr + 64, token row lr, 16-byte quarter lq
  const int lr = tid >> 2, lq = tid & 3;
  const int t_ld = t0 + lr;
  int tb = 0, n_left = 0;  // token index of tap 0 and tokens left in the document from there
  if (t_ld < n_out) {
    const int d = find_doc(tab.b, n_docs, t_ld);
    tb = tab.a[d] + (t_ld - tab.b[d]);
    n_left = tab.a[d + 1] - tb;
  }
  const float* wrow0 = W1 + (long)(c0 + lr) * K + 4 * lq;
  const float* wrow1 = wrow0 + 64L * K;

  f32x4 ra0, ra1, rb;
  auto fetch = [&](int kc) {
    const int tap = kc / CPT;
    const int i0 = (kc - tap * CPT) * kBK;
    ra0 = *reinterpret_cast<const f32x4*>(wrow0 + kc * kBK);
    ra1 = *reinterpret_cast<const f32x4*>(wrow1 + kc * kBK);
    rb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (tap < n_left) {
      const int id = min(max(tokens[tb + tap], 0), vocab - 1);
      rb = *reinterpret_cast<const f32x4*>(embed + (long)id * kFeat + i0 + 4 * lq);
    }
  };
  auto stash = [&](int buf) {
    *reinterpret_cast<f32x4*>(&sA[buf][lr][4 * lq]) = ra0;
    *reinterpret_cast<f32x4*>(&sA[buf][lr + 64][4 * lq]) = ra1;
    *reinterpret_cast<f32x4*>(&sB[buf][lr][4 * lq]) = rb;
  };

  f32x4 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  fetch(0);
  stash(0);
  __syncthreads();
  // the next chunk is fetched and stashed unconditionally (clamped to the last chunk; the
  // surplus lands in the buffer no later iteration reads), so the compiler does not wait for
  // the fetch before this chunk's MFMAs; the fence keeps the fetch at the top
  for (int kc = 0; kc < KC; ++kc) {
    const int cur = kc & 1;
    fetch(min(kc + 1, KC - 1));
    __builtin_amdgcn_sched_barrier(0);
    f32x4 av[4], bv[2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
      av[a] = *reinterpret_cast<const f32x4*>(&sA[cur][wc * 64 + a * 16 + li][4 * lg]);
#pragma unroll
    for (int b = 0; b < 2; ++b)
      bv[b] = *reinterpret_cast<const f32x4*>(&sB[cur][wt * 32 + b * 16 + li][4 * lg]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = mfma16(av[a][s], bv[b][s], acc[a][b]);
    stash(cur ^ 1);
    __syncthreads();
  }

  // D[i = channel][j = token]: lane holds token li, channels 4 lg + 0..3 of each tile
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int t = t0 + wt * 32 + b * 16 + li;
    if (t >= n_out) continue;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int c = c0 + wc * 64 + a * 16 + 4 * lg;
      const f32x4 bias = *reinterpret_cast<const f32x4*>(b1 + c);
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = leaky_relu(acc[a][b][e] + bias[e]);
      *reinterpret_cast<f32x4*>(h + (long)t * C + c) = v;
    }
  }
}

// ---- conv2 partial sums: part[s][t][o] = sum over split s of W2[o][k] G[k][t] --------------
// Workgroup tile 80 outputs x 64 tokens, K range split blockIdx.y of kSplit; wave w owns
// tokens 16 w .. 16 w + 15 and all five 16-output tiles.
// tab.b = output-token prefix sums
__global__ __launch_bounds__(256) void lookahead_conv2_kernel(
    const float* __restrict__ h, const DocTables tab, int n_docs, int n_out,
    const float* __restrict__ W2, int C, float* __restrict__ part) {
  constexpr int TAPS = 3;
  constexpr int OT = kFeat / 16;  // 5 output tiles
  __shared__ __attribute__((aligned(16))) float sA[2][kFeat][kPitch];
  __shared__ __attribute__((aligned(16))) float sB[2][kTileT][kPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * kTileT;
  const int split = blockIdx.y;
  const int K = TAPS * C;
  const int CPT = C / kBK;
  const int KC = TAPS * CPT;
  const int kc_begin = split * (KC / kSplit);
  const int kc_end = kc_begin + KC / kSplit;

  const int lr = tid >> 2, lq = tid & 3;
  const int t_ld = t0 + lr;
  int pos = -1;  // position of the loader's token in its document (-1: past the batch)
  if (t_ld < n_out) pos = t_ld - tab.b[find_doc(tab.b, n_docs, t_ld)];
  const bool second = lr < kFeat - 64;  // rows 64..79 of the weight tile
  const float* wrow0 = W2 + (long)lr * K + 4 * lq;
  const float* wrow1 = W2 + (long)(64 + (second ? lr : 0)) * K + 4 * lq;

  f32x4 ra0, ra1, rb;
  auto fetch = [&](int kc) {
    const int tap = kc / CPT;
    const int cc = (kc - tap * CPT) * kBK;
    ra0 = *reinterpret_cast<const f32x4*>(wrow0 + kc * kBK);
    if (second) ra1 = *reinterpret_cast<const f32x4*>(wrow1 + kc * kBK);
    rb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // h row t - 2 + tap, which lies in the same document iff pos - 2 + tap >= 0
    if (pos >= 0 && pos + tap >= TAPS - 1)
      rb = *reinterpret_cast<const f32x4*>(h + (long)(t_ld - (TAPS - 1) + tap) * C + cc + 4 * lq);
  };
  auto stash = [&](int buf) {
    *reinterpret_cast<f32x4*>(&sA[buf][lr][4 * lq]) = ra0;
    if (second) *reinterpret_cast<f32x4*>(&sA[buf][64 + lr][4 * lq]) = ra1;
    *reinterpret_cast<f32x4*>(&sB[buf][lr][4 * lq]) = rb;
  };

  f32x4 acc[OT];
#pragma unroll
  for (int a = 0; a < OT; ++a) acc[a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  fetch(kc_begin);
  stash(0);
  __syncthreads();
  for (int kc = kc_begin; kc < kc_end; ++kc) {
    const int cur = (kc - kc_begin) & 1;
    fetch(min(kc + 1, kc_end - 1));  // unconditional, as in the first layer's loop
    __builtin_amdgcn_sched_barrier(0);
    f32x4 av[OT];
#pragma unroll
    for (int a = 0; a < OT; ++a)
      av[a] = *reinterpret_cast<const f32x4*>(&sA[cur][a * 16 + li][4 * lg]);
    const f32x4 bv = *reinterpret_cast<const f32x4*>(&sB[cur][wave * 16 + li][4 * lg]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int a = 0; a < OT; ++a) acc[a] = mfma16(av[a][s], bv[s], acc[a]);
    stash(cur ^ 1);
    __syncthreads();
  }

  const int t = t0 + wave * 16 + li;
  if (t >= n_out) return;
  float* dst = part + ((long)split * n_out + t) * kFeat + 4 * lg;
#pragma unroll
  for (int a = 0; a < OT; ++a) *reinterpret_cast<f32x4*>(dst + a * 16) = acc[a];
}

// ---- finish: y = b2 + sum_s part[s] + e(t), written to Mel rows ratio*t .. +ratio-1 --------
__global__ __launch_bounds__(256) void lookahead_finish_kernel(
    const float* __restrict__ part, const int32_t* __restrict__ tokens, const DocTables tab,
    int n_docs, int n_out, const float* __restrict__ embed, int vocab,
    const float* __restrict__ b2, int ratio, float* __restrict__ mu) {
  constexpr int Q = kFeat / 4;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)n_out * Q) return;
  const int t = (int)(idx / Q);
  const int o = (int)(idx - (long)t * Q) * 4;
  const int d = find_doc(tab.b, n_docs, t);
  const int id = min(max(tokens[tab.a[d] + (t - tab.b[d])], 0), vocab - 1);
  f32x4 s = *reinterpret_cast<const f32x4*>(part + (long)t * kFeat + o);
#pragma unroll
  for (int k = 1; k < kSplit; ++k) {
    const f32x4 p = *reinterpret_cast<const f32x4*>(part + ((long)k * n_out + t) * kFeat + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] += p[e];
  }
  const f32x4 bias = *reinterpret_cast<const f32x4*>(b2 + o);
  const f32x4 res = *reinterpret_cast<const f32x4*>(embed + (long)id * kFeat + o);
  f32x4 y;
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = (s[e] + bias[e]) + res[e];
  for (int j = 0; j < ratio; ++j)
    *reinterpret_cast<f32x4*>(mu + ((long)t * ratio + j) * kFeat + o) = y;
}

// ---- speaker: out[n] = W (x / max(||x||, 1e-12)) + b; one wave per x-vector ----------------
__global__ __launch_bounds__(64) void speaker_kernel(const float* __restrict__ x, int D,
                                                     const float* __restrict__ W,
                                                     const float* __restrict__ b, int F,
                                                     float* __restrict__ out) {
  __shared__ float sx[256];
  const int n = blockIdx.x;
  const int lane = threadIdx.x;
  float ss = 0.0f;
  for (int i = lane; i < D; i += 64) {
    const float v = x[(long)n * D + i];
    sx[i] = v;
    ss = fmaf(v, v, ss);
  }
  const float denom = fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
  __syncthreads();
  for (int i = lane; i < D; i += 64) sx[i] = sx[i] / denom;
  __syncthreads();
  for (int o = lane; o < F; o += 64) {
    const float* w = W + (long)o * D;
    float acc = 0.0f;
    for (int i = 0; i < D; ++i) acc = fmaf(w[i], sx[i], acc);
    out[(long)n * F + o] = acc + b[o];
  }
}

// ---- prompt copy: cond[row] = prompt[...] for the first min(plen, mel_len) rows, else 0 ------
// tab.a = prompt-row prefix sums, tab.b = Mel-row prefix sums
__global__ __launch_bounds__(256) void prompt_cond_kernel(const float* __restrict__ prompt,
                                                          const DocTables tab, int n_docs,
                                                          int rows, float* __restrict__ cond) {
  constexpr int Q = kFeat / 4;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * Q) return;
  const int r = (int)(idx / Q);
  const int o = (int)(idx - (long)r * Q) * 4;
  const int d = find_doc(tab.b, n_docs, r);
  const int p = r - tab.b[d];
  f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (p < tab.a[d + 1] - tab.a[d])
    v = *reinterpret_cast<const f32x4*>(prompt + (long)(tab.a[d] + p) * kFeat + o);
  *reinterpret_cast<f32x4*>(cond + (long)r * kFeat + o) = v;
}

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct FlowLayout {
  size_t hidden, part, total;
};

FlowLayout flow_layout(const FcvFlowDims& d, int out_tokens) {
  FlowLayout L;
  L.hidden = 0;
  L.part = align_up(sizeof(float) * (size_t)out_tokens * d.channels);
  L.total = L.part + align_up(sizeof(float) * (size_t)kSplit * out_tokens * d.feat_dim);
  return L;
}

int check_dims(const FcvFlowDims* dims) {
  FCV_CHECK(dims, FCV_ERR_INVALID, "null dims");
  const FcvFlowDims& d = *dims;
  FCV_CHECK(d.feat_dim == kFeat, FCV_ERR_INVALID, "feat_dim must be 80");
  FCV_CHECK(d.channels > 0 && d.channels % kTileC == 0, FCV_ERR_INVALID,
            "channels must be a positive multiple of 128");
  FCV_CHECK(d.lookahead >= 0 && d.lookahead <= 7, FCV_ERR_INVALID, "lookahead must be in [0, 7]");
  FCV_CHECK(d.token_mel_ratio >= 1 && d.token_mel_ratio <= 8, FCV_ERR_INVALID,
            "token_mel_ratio must be in [1, 8]");
  FCV_CHECK(d.spk_dim >= 1 && d.spk_dim <= 256, FCV_ERR_INVALID, "spk_dim must be in [1, 256]");
  FCV_CHECK(d.vocab >= 1, FCV_ERR_INVALID, "vocab must be >= 1");
  return FCV_OK;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Checks one token-features call and builds its per-document tables (tab.a: token prefix sums,
// tab.b: output-token prefix sums) and its output token count.
int prepare_token_features(const FcvFlowDims* dims, const FcvFlowWeights* weights,
                           const int32_t* tokens, const int32_t* cu_tokens_host,
                           const int32_t* finalize_host, int32_t n_docs, float* mu_out,
                           DocTables* tab, int* n_out) {
  if (int rc = check_dims(dims)) return rc;
  const FcvFlowDims& d = *dims;
  FCV_CHECK(weights && weights->embed && weights->la1_w && weights->la1_b && weights->la2_w &&
                weights->la2_b,
            FCV_ERR_INVALID, "null weight pointer");
  const FcvFlowWeights& w = *weights;
  FCV_CHECK(aligned16(w.embed) && aligned16(w.la1_w) && aligned16(w.la1_b) &&
                aligned16(w.la2_w) && aligned16(w.la2_b),
            FCV_ERR_INVALID, "weights must be 16-byte aligned");
  FCV_CHECK(tokens && cu_tokens_host && mu_out, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(aligned16(mu_out), FCV_ERR_INVALID, "mu_out must be 16-byte aligned");
  FCV_CHECK(n_docs >= 1 && n_docs <= kMaxDocs, FCV_ERR_INVALID,
            "n_docs must be in [1, " + std::to_string(kMaxDocs) + "]");
  FCV_CHECK(cu_tokens_host[0] == 0, FCV_ERR_INVALID, "cu_tokens[0] must be 0");
  tab->a[0] = tab->b[0] = 0;
  for (int i = 0; i < n_docs; ++i) {
    const long len = (long)cu_tokens_host[i + 1] - cu_tokens_host[i];
    FCV_CHECK(len >= 1, FCV_ERR_INVALID, "document " + std::to_string(i) + " has no tokens");
    const bool fin = finalize_host == nullptr || finalize_host[i] != 0;
    FCV_CHECK(fin || len > d.lookahead, FCV_ERR_INVALID,
              "document " + std::to_string(i) + " is not finalized and has no more tokens than "
              "the lookahead");
    const long out = tab->b[i] + len - (fin ? 0 : d.lookahead);
    FCV_CHECK(cu_tokens_host[i + 1] <= (1 << 24) && out <= (1 << 24), FCV_ERR_INVALID,
              "too many tokens");
    tab->a[i + 1] = cu_tokens_host[i + 1];
    tab->b[i + 1] = (int32_t)out;
  }
  *n_out = tab->b[n_docs];
  return FCV_OK;
}

// The three kernels of a checked call, with the workspace at `ws` (flow_layout of n_out).
int launch_token_features(const FcvFlowDims& d, const FcvFlowWeights& w, const int32_t* tokens,
                          const DocTables& tab, int n_docs, int n_out, float* mu_out, char* ws,
                          hipStream_t stream) {
  const FlowLayout L = flow_layout(d, n_out);
  float* hid = reinterpret_cast<float*>(ws + L.hidden);
  float* part = reinterpret_cast<float*>(ws + L.part);
  const int t_tiles = (n_out + kTileT - 1) / kTileT;
  hipLaunchKernelGGL(lookahead_conv1_kernel, dim3(t_tiles, d.channels / kTileC), dim3(256), 0,
                     stream, tokens, tab, n_docs, n_out, w.embed, d.vocab, w.la1_w, w.la1_b,
                     d.channels, d.lookahead + 1, hid);
  FCV_HIP(hipGetLastError());
  hipLaunchKernelGGL(lookahead_conv2_kernel, dim3(t_tiles, kSplit), dim3(256), 0, stream, hid,
                     tab, n_docs, n_out, w.la2_w, d.channels, part);
  FCV_HIP(hipGetLastError());
  const long items = (long)n_out * (kFeat / 4);
  hipLaunchKernelGGL(lookahead_finish_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     stream, part, tokens, tab, n_docs, n_out, w.embed, d.vocab, w.la2_b,
                     d.token_mel_ratio, mu_out);
  FCV_HIP(hipGetLastError());
  return FCV_OK;
}

}  // namespace

// ---- scratch of fcv_flow_token_features_noalloc ----------------------------------------------
// The workspace of the no-allocation entry point: a file-scope device array, one copy per GPU,
// held from module load until the process ends.  Every no-allocation call on a GPU uses that
// GPU's copy (calls that overlap on one GPU race on it).  Host code never passes the array's
// name to a kernel (on the host it is a stand-in, not a device address): scratch_for looks up
// each device's address once, with that device current, and the launches take that address.
// Nothing in it needs clearing: conv1 writes every hidden row a call reads and conv2 every
// partial sum the finishing kernel reads.
constexpr size_t kScratchBytes = FCV_FLOW_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch_ptr[kMaxScratchDevices] = {};

// output tokens a call can take within the scratch at these dims
int noalloc_max_tokens(const FcvFlowDims& d) {
  int lo = 0, hi = 1 << 24;
  while (lo < hi) {
    const int mid = lo + (hi - lo + 1) / 2;
    if (flow_layout(d, mid).total <= kScratchBytes) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Device address of `scratch` on the device `stream` belongs to (looked up once per device).
int scratch_for(hipStream_t stream, char** out) {
  int dev = 0;
  if (stream) {
    FCV_HIP(hipStreamGetDevice(stream, &dev));
  } else {
    FCV_HIP(hipGetDevice(&dev));
  }
  FCV_CHECK(dev >= 0 && dev < kMaxScratchDevices, FCV_ERR_RUNTIME,
            "device index " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    int current = 0;
    FCV_HIP(hipGetDevice(&current));
    if (current != dev) FCV_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current != dev) (void)hipSetDevice(current);
    if (e != hipSuccess)
      return fail(FCV_ERR_RUNTIME, std::string("hipGetSymbolAddress(scratch): ") +
                                       hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return FCV_OK;
}

}  // namespace
}  // namespace fcv

using fcv::fail;

extern "C" {

size_t fcv_flow_workspace_bytes(const FcvFlowDims* dims, int32_t out_tokens) {
  if (!dims || out_tokens < 0) return 0;
  return fcv::flow_layout(*dims, out_tokens).total;
}

int fcv_flow_token_features(const FcvFlowDims* dims, const FcvFlowWeights* weights,
                            const int32_t* tokens, const int32_t* cu_tokens_host,
                            const int32_t* finalize_host, int32_t n_docs, float* mu_out,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
  fcv::DocTables tab{};
  int n_out = 0;
  if (int rc = fcv::prepare_token_features(dims, weights, tokens, cu_tokens_host, finalize_host,
                                           n_docs, mu_out, &tab, &n_out))
    return rc;
  FCV_CHECK(workspace, FCV_ERR_INVALID, "null workspace");
  const fcv::FlowLayout L = fcv::flow_layout(*dims, n_out);
  FCV_CHECK(workspace_bytes >= L.total, FCV_ERR_INVALID,
            "workspace too small: need " + std::to_string(L.total) + " bytes");
  FCV_CHECK(reinterpret_cast<uintptr_t>(workspace) % fcv::kAlign == 0, FCV_ERR_INVALID,
            "workspace must be 256-byte aligned");
  return fcv::launch_token_features(*dims, *weights, tokens, tab, n_docs, n_out, mu_out,
                                    static_cast<char*>(workspace), stream);
}

int fcv_flow_token_features_noalloc(const FcvFlowDims* dims, const FcvFlowWeights* weights,
                                    const int32_t* tokens, const int32_t* cu_tokens_host,
                                    const int32_t* finalize_host, int32_t n_docs, float* mu_out,
                                    hipStream_t stream) {
  fcv::DocTables tab{};
  int n_out = 0;
  if (int rc = fcv::prepare_token_features(dims, weights, tokens, cu_tokens_host, finalize_host,
                                           n_docs, mu_out, &tab, &n_out))
    return rc;
  const fcv::FlowLayout L = fcv::flow_layout(*dims, n_out);
  FCV_CHECK(L.total <= fcv::kScratchBytes, FCV_ERR_INVALID,
            std::to_string(n_out) + " output tokens need " + std::to_string(L.total) +
                " bytes of scratch; the no-allocation entry point holds " +
                std::to_string(fcv::kScratchBytes) + " (at most " +
                std::to_string(fcv::noalloc_max_tokens(*dims)) +
                " output tokens per call at these dims): split the batch or pass a workspace "
                "to fcv_flow_token_features");
  char* ws = nullptr;
  if (int rc = fcv::scratch_for(stream, &ws)) return rc;
  return fcv::launch_token_features(*dims, *weights, tokens, tab, n_docs, n_out, mu_out, ws,
                                    stream);
}

int fcv_flow_speaker(const FcvFlowDims* dims, const FcvFlowWeights* weights, const float* xvec,
                     int32_t n, float* spks_out, hipStream_t stream) {
  if (int rc = fcv::check_dims(dims)) return rc;
  FCV_CHECK(weights && weights->spk_w && weights->spk_b, FCV_ERR_INVALID, "null weight pointer");
  FCV_CHECK(xvec && spks_out, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(n >= 1, FCV_ERR_INVALID, "need at least one x-vector");
  hipLaunchKernelGGL(fcv::speaker_kernel, dim3(n), dim3(64), 0, stream, xvec, dims->spk_dim,
                     weights->spk_w, weights->spk_b, dims->feat_dim, spks_out);
  FCV_HIP(hipGetLastError());
  return FCV_OK;
}

int fcv_flow_prompt_cond(const FcvFlowDims* dims, const float* prompt,
                         const int32_t* cu_prompt_host, const int32_t* cu_mel_host,
                         int32_t n_docs, float* cond_out, hipStream_t stream) {
  if (int rc = fcv::check_dims(dims)) return rc;
  FCV_CHECK(cu_prompt_host && cu_mel_host && cond_out, FCV_ERR_INVALID, "null argument");
  FCV_CHECK(n_docs >= 1 && n_docs <= fcv::kMaxDocs, FCV_ERR_INVALID,
            "n_docs must be in [1, " + std::to_string(fcv::kMaxDocs) + "]");
  FCV_CHECK(cu_prompt_host[0] == 0 && cu_mel_host[0] == 0, FCV_ERR_INVALID,
            "prefix sums must start at 0");
  FCV_CHECK(fcv::aligned16(cond_out) && (prompt == nullptr || fcv::aligned16(prompt)),
            FCV_ERR_INVALID, "prompt and cond_out must be 16-byte aligned");
  fcv::DocTables tab{};  // a: prompt-row prefix sums, b: Mel-row prefix sums
  for (int i = 0; i < n_docs; ++i) {
    FCV_CHECK(cu_prompt_host[i + 1] >= cu_prompt_host[i], FCV_ERR_INVALID,
              "prompt prefix sums must be non-decreasing");
    FCV_CHECK(cu_mel_host[i + 1] > cu_mel_host[i], FCV_ERR_INVALID,
              "every document needs at least one Mel row");
    FCV_CHECK(cu_mel_host[i + 1] <= (1 << 26) && cu_prompt_host[i + 1] <= (1 << 26),
              FCV_ERR_INVALID, "too many rows");
    tab.a[i + 1] = cu_prompt_host[i + 1];
    tab.b[i + 1] = cu_mel_host[i + 1];
  }
  FCV_CHECK(tab.a[n_docs] == 0 || prompt != nullptr, FCV_ERR_INVALID, "null prompt");
  const int rows = tab.b[n_docs];
  const long items = (long)rows * (fcv::kFeat / 4);
  hipLaunchKernelGGL(fcv::prompt_cond_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     stream, prompt, tab, n_docs, rows, cond_out);
  FCV_HIP(hipGetLastError());
  return FCV_OK;
}

}  // extern "C"
