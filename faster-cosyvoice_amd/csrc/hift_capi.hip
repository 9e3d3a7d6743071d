// C ABI of the HiFT vocoder (include/fcv_hift.h): validation, per-call document tables, the
// workspace carve-up and the launch sequence of CausalHiFTGenerator.inference over packed
// documents, and the pool of captured calls.
//
// A call has a capacity (total Mel frames, documents): the workspace carve-up and every grid
// depend on it only.  The call's own layout -- the per-document prefix sums of each launch --
// is written into a table block of the workspace before the launches, and the kernels read it
// there.  So the launch sequence captured for a capacity replays for any later layout of that
// capacity (the reference captures one graph per padded length, hift_graph.py:65-169, and pads
// each request to it).
#include <algorithm>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "../../include/fcv_hift.h"
#include "hift.hpp"
#include "status.hpp"

using fcv::fail;
using fcv::HiftConv;
using fcv::HiftDocs;

struct FcvHift {
  FcvHiftDims d;
  std::vector<const void*> w;
  int i_lin, i_pre, i_ups, i_down, i_srb, i_rb, i_post, i_f0, i_cls, i_win, i_ini, i_tab;
  // captured calls by key (capacity, workspace, buffers), most recently used first; seen: keys
  // of recent graph-eligible calls (a key is captured on its second call)
  struct Graph {
    std::vector<uintptr_t> key;
    hipGraphExec_t exec;
  };
  std::vector<Graph> graphs;
  std::vector<std::vector<uintptr_t>> seen;
  long captures = 0;
};

namespace {

constexpr size_t kAlign = 256;
constexpr int kSpecLd = 32;   // STFT / conv_post rows: 18 channels padded to 32
constexpr int kFrameLd = 16;  // iSTFT frames

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int causal_padding(int k, int dil) { return (k * dil - dil) / 2 * 2 + (k + 1) % 2; }

int stage_channels(const FcvHiftDims& d, int i) { return d.base_channels >> (i + 1); }

int upsample_scale(const FcvHiftDims& d) {
  int s = d.hop_len;
  for (int i = 0; i < d.n_stages; ++i) s *= d.upsample_rates[i];
  return s;
}

// (kernel, stride) of source_downs[i] (generator.py:640-655)
std::pair<int, int> source_down(const FcvHiftDims& d, int i) {
  int u = 1;
  for (int j = i + 1; j < d.n_stages; ++j) u *= d.upsample_rates[j];
  return u == 1 ? std::make_pair(1, 1) : std::make_pair(2 * u, u);
}

int weight_count(const FcvHiftDims& d) {
  const int S = d.n_stages, K = d.n_kernels, D = d.n_dilations;
  return 2 + 2 + 2 * S + 2 * S + 8 * D * S + 8 * D * S * K + 2 + 10 + 2 + 3;
}

int check_dims(const FcvHiftDims* dims) {
  FCV_CHECK(dims, FCV_ERR_INVALID, "null dims");
  const FcvHiftDims& d = *dims;
  FCV_CHECK(d.n_stages >= 1 && d.n_stages <= FCV_HIFT_MAX && d.n_kernels >= 1 &&
                d.n_kernels <= FCV_HIFT_MAX && d.n_dilations >= 1 &&
                d.n_dilations <= FCV_HIFT_MAX,
            FCV_ERR_INVALID, "n_stages, n_kernels and n_dilations must be in [1, 4]");
  FCV_CHECK(d.in_channels > 0 && d.in_channels % 16 == 0, FCV_ERR_INVALID,
            "in_channels must be a positive multiple of 16");
  for (int i = 0; i < d.n_stages; ++i) {
    FCV_CHECK(stage_channels(d, i) >= 16 && stage_channels(d, i) % 16 == 0 &&
                  (d.base_channels >> (i + 1) << (i + 1)) == d.base_channels,
              FCV_ERR_INVALID, "every stage's channels must be a multiple of 16");
    FCV_CHECK(d.upsample_rates[i] >= 1 && d.upsample_kernels[i] >= 1 &&
                  d.source_kernels[i] >= 1,
              FCV_ERR_INVALID, "bad upsampling or source kernel");
    for (int j = 0; j < d.n_dilations; ++j)
      FCV_CHECK(d.source_dilations[i][j] >= 1, FCV_ERR_INVALID, "bad source dilation");
  }
  for (int k = 0; k < d.n_kernels; ++k) {
    FCV_CHECK(d.resblock_kernels[k] >= 1, FCV_ERR_INVALID, "bad resblock kernel");
    for (int j = 0; j < d.n_dilations; ++j)
      FCV_CHECK(d.resblock_dilations[k][j] >= 1, FCV_ERR_INVALID, "bad resblock dilation");
  }
  FCV_CHECK(d.n_fft == 16 && d.hop_len == 4, FCV_ERR_INVALID, "n_fft must be 16 and hop_len 4");
  FCV_CHECK(d.nb_harmonics >= 0 && d.nb_harmonics < 64, FCV_ERR_INVALID,
            "nb_harmonics must be in [0, 63]");
  FCV_CHECK(d.f0_channels > 0 && d.f0_channels % 64 == 0, FCV_ERR_INVALID,
            "f0_channels must be a positive multiple of 64");
  FCV_CHECK(d.conv_pre_look_right >= 0 && d.sampling_rate > 0 && d.noise_samples > 0,
            FCV_ERR_INVALID, "bad conv_pre_look_right, sampling_rate or noise_samples");
  return FCV_OK;
}

// per-call lengths of one document
struct DocLens {
  int mel, f0, x, spec, samples, src;  // frames in, F0 frames, conv_pre frames, STFT frames, out
};

bool doc_lens(const FcvHiftDims& d, int frames, bool fin, DocLens* out) {
  const int scale = upsample_scale(d);
  DocLens L;
  L.mel = frames;
  L.f0 = fin ? frames : frames - 3;
  L.x = fin ? L.f0 : L.f0 - d.conv_pre_look_right;
  if (frames < 1 || L.x < 1) return false;
  const int stage_rate = scale / d.hop_len;
  L.spec = stage_rate * L.x + 1;
  L.samples = d.hop_len * (L.spec - 1) - (fin ? 0 : scale);
  L.src = scale * L.f0;
  if (L.samples < 0) return false;
  *out = L;
  return true;
}

constexpr size_t kGraphPool = 4;  // captured calls kept per handle (least recently used goes)
constexpr size_t kSeenKeys = 8;   // keys remembered for the capture-on-second-call rule

// The workspace carve-up and the grids of a capacity: at most `frames` Mel frames in at most
// `docs` documents.  Every per-call total is bounded by these (a document's F0, conv_pre and
// STFT frame counts, samples and stage rows grow with its Mel frames; each document adds at
// most one STFT frame and one reflection row).
struct Capacity {
  int frames, docs;
  int spec, samples, src;              // STFT frames, output samples, source samples
  std::vector<int> stage, stage_w;     // upsampling-conv rows and written rows per stage
  size_t mel64, h64a, h64b, f0buf, sines, srcbuf, specbuf, xa, xn, xs, r, t1, s1, si, y, fr,
      tables, total;
};

// Tables of one call, in launch order (see run): their count for n_stages stages.
int table_count(const FcvHiftDims& d) { return 7 + 3 * d.n_stages; }

Capacity make_capacity(const FcvHiftDims& d, int frames, int docs) {
  Capacity C;
  C.frames = frames;
  C.docs = docs;
  const int scale = upsample_scale(d);
  const int stage_rate = scale / d.hop_len;
  C.spec = stage_rate * frames + docs;
  C.samples = d.hop_len * C.spec;
  C.src = scale * frames;
  size_t smax = (size_t)frames * d.base_channels;
  int rate = 1;
  for (int s = 0; s < d.n_stages; ++s) {
    rate *= d.upsample_rates[s];
    C.stage.push_back(rate * frames);
    C.stage_w.push_back(rate * frames + (s == d.n_stages - 1 ? docs : 0));
    smax = std::max(smax, (size_t)C.stage_w.back() * stage_channels(d, s));
  }
  const int H = d.nb_harmonics + 1;
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += align_up(bytes); return o; };
  C.mel64 = take(sizeof(double) * frames * d.in_channels);
  C.h64a = take(sizeof(double) * frames * d.f0_channels);
  C.h64b = take(sizeof(double) * frames * d.f0_channels);
  C.f0buf = take(sizeof(float) * frames);
  C.sines = take(sizeof(float) * frames * H);
  C.srcbuf = take(sizeof(float) * C.src);
  C.specbuf = take(sizeof(float) * C.spec * kSpecLd);
  for (size_t* b : {&C.xa, &C.xn, &C.xs, &C.r, &C.t1, &C.s1, &C.si})
    *b = take(sizeof(float) * smax);
  C.y = take(sizeof(float) * C.spec * kSpecLd);
  C.fr = take(sizeof(float) * C.spec * kFrameLd);
  C.tables = take(sizeof(HiftDocs) * table_count(d));
  C.total = off;
  return C;
}

// The layout of one call: per-document lengths and their prefix sums.
struct Plan {
  int n_docs;
  std::vector<DocLens> lens;
  std::vector<int> mel, f0, x, spec, samples, src;
  std::vector<std::vector<int>> stage;  // compute rows of stage i (no reflection pad)
};

std::vector<int> prefix(const std::vector<DocLens>& v, int DocLens::*m) {
  std::vector<int> out(v.size() + 1, 0);
  for (size_t i = 0; i < v.size(); ++i) out[i + 1] = out[i] + v[i].*m;
  return out;
}

int make_plan(const FcvHift* h, const int32_t* frames, const int32_t* finalize, int n_docs,
              Plan* P) {
  const FcvHiftDims& d = h->d;
  FCV_CHECK(frames && n_docs >= 1 && n_docs <= FCV_HIFT_MAX_DOCS, FCV_ERR_INVALID,
            "n_docs must be in [1, 256]");
  P->n_docs = n_docs;
  P->lens.resize(n_docs);
  long total_src = 0;
  for (int i = 0; i < n_docs; ++i) {
    const bool fin = finalize == nullptr || finalize[i] != 0;
    FCV_CHECK(frames[i] >= 1 && frames[i] <= (1 << 20), FCV_ERR_INVALID,
              "document " + std::to_string(i) + " has a bad frame count");
    FCV_CHECK(doc_lens(d, frames[i], fin, &P->lens[i]), FCV_ERR_INVALID,
              "document " + std::to_string(i) + " is too short for a non-final chunk");
    FCV_CHECK(P->lens[i].src <= d.noise_samples, FCV_ERR_INVALID,
              "document " + std::to_string(i) + " is longer than the source noise table");
    total_src += P->lens[i].src;
  }
  FCV_CHECK(total_src < (1L << 30), FCV_ERR_INVALID, "too many samples in one call");
  P->mel = prefix(P->lens, &DocLens::mel);
  P->f0 = prefix(P->lens, &DocLens::f0);
  P->x = prefix(P->lens, &DocLens::x);
  P->spec = prefix(P->lens, &DocLens::spec);
  P->samples = prefix(P->lens, &DocLens::samples);
  P->src = prefix(P->lens, &DocLens::src);
  P->stage.assign(d.n_stages, std::vector<int>(n_docs + 1, 0));
  int rate = 1;
  for (int s = 0; s < d.n_stages; ++s) {
    rate *= d.upsample_rates[s];
    for (int i = 0; i < n_docs; ++i) P->stage[s][i + 1] = P->stage[s][i] + P->lens[i].x * rate;
  }
  return FCV_OK;
}

HiftDocs docs_of(const std::vector<int>& a, const std::vector<int>& b) {
  HiftDocs t{};
  t.n = (int32_t)a.size() - 1;
  for (size_t i = 0; i < a.size(); ++i) t.a[i] = a[i];
  for (size_t i = 0; i < b.size(); ++i) t.b[i] = b[i];
  return t;
}

// written rows of stage s: the last stage carries one reflection-pad row per document
std::vector<int> rows_written(const FcvHiftDims& d, const Plan& P, int s) {
  std::vector<int> rows_w = P.stage[s];
  if (s == d.n_stages - 1)
    for (int i = 0; i <= P.n_docs; ++i) rows_w[i] += i;
  return rows_w;
}

// Every table of a call, in the order run() uses them:
//   0 (mel, f0)  1 (f0, f0)  2 (f0, src)  3 (src, spec)  4 (mel, x)
//   per stage s: 5+3s (spec, rows_w)  6+3s (rows_w, rows_w)  7+3s (previous rows, stage rows)
//   5+3S (last rows_w, spec)  6+3S (spec, samples)
std::vector<HiftDocs> make_tables(const FcvHiftDims& d, const Plan& P) {
  std::vector<HiftDocs> t;
  t.push_back(docs_of(P.mel, P.f0));
  t.push_back(docs_of(P.f0, P.f0));
  t.push_back(docs_of(P.f0, P.src));
  t.push_back(docs_of(P.src, P.spec));
  t.push_back(docs_of(P.mel, P.x));
  std::vector<int> prev = P.x;
  for (int s = 0; s < d.n_stages; ++s) {
    const std::vector<int> rows_w = rows_written(d, P, s);
    t.push_back(docs_of(P.spec, rows_w));
    t.push_back(docs_of(rows_w, rows_w));
    t.push_back(docs_of(prev, P.stage[s]));
    prev = rows_w;
  }
  t.push_back(docs_of(prev, P.spec));
  t.push_back(docs_of(P.spec, P.samples));
  return t;
}

HiftConv conv_base(const void* x, int ldx, const void* w, const void* b, int cout, int cin_pad,
                   int k, void* out, int ldo, int rows_out) {
  HiftConv p{};
  p.x = x; p.ldx = ldx; p.w = w; p.bias = b; p.cout = cout; p.cin_pad = cin_pad; p.k = k;
  p.stride = 1; p.dil = 1; p.pad = 0; p.up = 1; p.rows_out = rows_out;
  p.out = out; p.ldo = ldo; p.div = 1.0f;
  return p;
}

// one ResBlock (generator.py:110-116) on x (rows by `docs`, C channels): for each dilation
// j: r = r + conv2(snake2(conv1(snake1(r)))); the last conv2 writes its result per `mode`
// (write / accin + y / (accin + y) / div) into `out`.  `wb` points at the block's 8 * D
// weight pointers.  x is read as the first residual; r holds the running value.  `rows` is the
// capacity the grids cover.
int run_resblock(const FcvHiftDims& d, const void* const* wb, int k, const int* dils,
                 const float* x, float* r, float* t1, float* s1, float* out, int mode,
                 const float* accin, float div, int C, int rows, const HiftDocs* docs,
                 hipStream_t st) {
  const int D = d.n_dilations;
  FCV_HIP(fcv::hift_snake(x, C, s1, C, rows, C, static_cast<const float*>(wb[4]),
                          static_cast<const float*>(wb[5]), docs, st));
  for (int j = 0; j < D; ++j) {
    const void* const* q = wb + 8 * j;
    HiftConv c1 = conv_base(s1, C, q[0], q[1], C, C, k, t1, C, rows);
    c1.dil = dils[j];
    c1.pad = causal_padding(k, dils[j]);
    c1.snake_out = 1;
    c1.alpha = static_cast<const float*>(q[6]);
    c1.inv_alpha = static_cast<const float*>(q[7]);
    FCV_HIP(fcv::hift_conv_f32(c1, docs, st));
    const bool last = j == D - 1;
    HiftConv c2 = conv_base(t1, C, q[2], q[3], C, C, k, last ? out : r, C, rows);
    c2.pad = causal_padding(k, 1);
    c2.add = j == 0 ? static_cast<const void*>(x) : static_cast<const void*>(r);
    c2.ld_add = C;
    if (last) {
      c2.mode = mode;
      c2.accin = accin;
      c2.div = div;
    } else {
      c2.out2 = s1;
      c2.alpha2 = static_cast<const float*>(wb[8 * (j + 1) + 4]);
      c2.inv_alpha2 = static_cast<const float*>(wb[8 * (j + 1) + 5]);
    }
    FCV_HIP(fcv::hift_conv_f32(c2, docs, st));
  }
  return FCV_OK;
}

// The launch sequence of one call over capacity C; the layout is in the table block.
int run(FcvHift* h, const float* mel, const Capacity& C, float* speech, float* source_out,
        char* ws, hipStream_t st) {
  const FcvHiftDims& d = h->d;
  const void* const* w = h->w.data();
  auto F32 = [&](size_t o) { return reinterpret_cast<float*>(ws + o); };
  auto F64 = [&](size_t o) { return reinterpret_cast<double*>(ws + o); };
  const HiftDocs* T = reinterpret_cast<const HiftDocs*>(ws + C.tables);
  const int H = d.nb_harmonics + 1;
  const int scale = upsample_scale(d);
  const int S = d.n_stages;

  // ---- F0 predictor (fp64) -------------------------------------------------------------
  FCV_HIP(fcv::hift_to_f64(mel, F64(C.mel64), C.frames, d.in_channels, T + 0, st));
  const int fc = d.f0_channels;
  HiftConv c0 = conv_base(F64(C.mel64), d.in_channels, w[h->i_f0], w[h->i_f0 + 1], fc,
                          d.in_channels, 4, F64(C.h64a), fc, C.frames);
  c0.elu = 1;  // right-side lookahead: no left padding, zero (or context) on the right
  FCV_HIP(fcv::hift_conv_f64(c0, T + 0, st));
  double* hin = F64(C.h64a);
  double* hout = F64(C.h64b);
  for (int l = 1; l < 5; ++l) {
    HiftConv c = conv_base(hin, fc, w[h->i_f0 + 2 * l], w[h->i_f0 + 2 * l + 1], fc, fc, 3, hout,
                           fc, C.frames);
    c.pad = causal_padding(3, 1);
    c.elu = 1;
    FCV_HIP(fcv::hift_conv_f64(c, T + 1, st));
    std::swap(hin, hout);
  }
  FCV_HIP(fcv::hift_f0_head(hin, fc, static_cast<const double*>(w[h->i_cls]),
                            static_cast<const double*>(w[h->i_cls + 1]), C.frames, F32(C.f0buf),
                            T + 1, st));

  // ---- harmonic source and its STFT ------------------------------------------------------
  fcv::HiftSource src{};
  src.f0 = F32(C.f0buf);
  src.rand_ini = static_cast<const float*>(w[h->i_ini]);
  src.table = static_cast<const float*>(w[h->i_tab]);
  src.max_samples = d.noise_samples;
  src.lin_w = static_cast<const float*>(w[h->i_lin]);
  src.lin_b = static_cast<const float*>(w[h->i_lin + 1]);
  src.H = H;
  src.scale = scale;
  src.sampling_rate = d.sampling_rate;
  src.sine_amp = d.nsf_alpha;
  src.noise_std = d.nsf_sigma;
  src.voiced_threshold = d.nsf_voiced_threshold;
  src.docs_cap = C.docs;
  src.samples_cap = C.src;
  src.sines = F32(C.sines);
  src.s = F32(C.srcbuf);
  FCV_HIP(fcv::hift_source(src, T + 2, st));
  if (source_out) FCV_HIP(fcv::hift_copy_live(F32(C.srcbuf), source_out, C.src, T + 2, st));
  const float* window = static_cast<const float*>(w[h->i_win]);
  FCV_HIP(fcv::hift_stft(F32(C.srcbuf), window, F32(C.specbuf), kSpecLd, C.spec, T + 3, st));

  // ---- conv_pre (lookahead on the right) -------------------------------------------------
  float* xp = F32(C.xa);
  float* xn = F32(C.xn);
  {
    HiftConv c = conv_base(mel, d.in_channels, w[h->i_pre], w[h->i_pre + 1], d.base_channels,
                           d.in_channels, d.conv_pre_look_right + 1, xp, d.base_channels,
                           C.frames);
    FCV_HIP(fcv::hift_conv_f32(c, T + 4, st));
  }

  // ---- upsampling stages -----------------------------------------------------------------
  int cprev = d.base_channels;
  const int rb_size = 8 * d.n_dilations;
  for (int s = 0; s < S; ++s) {
    const int Cs = stage_channels(d, s);
    const bool last = s == S - 1;
    const int nrows = C.stage_w[s];
    const HiftDocs* t_src = T + 5 + 3 * s;  // (spec, rows_w)
    const HiftDocs* t_w = T + 6 + 3 * s;    // (rows_w, rows_w)
    const HiftDocs* t_up = T + 7 + 3 * s;   // (previous rows, stage rows)

    // source branch: strided (or 1x1) conv of the STFT frames, then its resblock
    float* si = F32(C.si);
    {
      const auto kd = source_down(d, s);
      HiftConv c = conv_base(F32(C.specbuf), kSpecLd, w[h->i_down + 2 * s],
                             w[h->i_down + 2 * s + 1], Cs, kSpecLd, kd.first, si, Cs, nrows);
      c.stride = kd.second;
      c.pad = kd.second - 1;
      FCV_HIP(fcv::hift_conv_f32(c, t_src, st));
      if (int rc = run_resblock(d, w + h->i_srb + rb_size * s, d.source_kernels[s],
                                d.source_dilations[s], si, F32(C.r), F32(C.t1), F32(C.s1), si,
                                fcv::HIFT_ACC_WRITE, nullptr, 1.0f, Cs, nrows, t_w, st))
        return rc;
    }
    // upsampling conv on LeakyReLU(x), plus the source branch
    {
      HiftConv c = conv_base(xp, cprev, w[h->i_ups + 2 * s], w[h->i_ups + 2 * s + 1], Cs, cprev,
                             d.upsample_kernels[s], xn, Cs, C.stage[s]);
      c.up = d.upsample_rates[s];
      c.pad = d.upsample_kernels[s] - 1;
      c.pro = fcv::HIFT_PRO_LEAKY;
      c.slope = d.lrelu_slope;
      c.reflect = last ? 1 : 0;
      c.add = si;
      c.ld_add = Cs;
      FCV_HIP(fcv::hift_conv_f32(c, t_up, st));
    }
    // mean of the resblocks
    for (int j = 0; j < d.n_kernels; ++j) {
      const int K = d.n_kernels;
      int mode = fcv::HIFT_ACC_WRITE;
      float* out = F32(C.xs);
      const float* accin = nullptr;
      float div = 1.0f;
      if (K == 1) {
        out = xn;
      } else if (j == K - 1) {
        mode = fcv::HIFT_ACC_ADD_DIV;
        accin = F32(C.xs);
        out = xn;
        div = (float)K;
      } else if (j > 0) {
        mode = fcv::HIFT_ACC_ADD;
        accin = F32(C.xs);
      }
      if (int rc = run_resblock(d, w + h->i_rb + rb_size * (s * K + j), d.resblock_kernels[j],
                                d.resblock_dilations[j], xn, F32(C.r), F32(C.t1), F32(C.s1),
                                out, mode, accin, div, Cs, nrows, t_w, st))
        return rc;
    }
    cprev = Cs;
    std::swap(xp, xn);
  }

  // ---- conv_post on LeakyReLU(x) (slope 0.01), iSTFT, clamp ------------------------------
  {
    const int spec = d.n_fft + 2;
    HiftConv c = conv_base(xp, cprev, w[h->i_post], w[h->i_post + 1], spec, cprev, 7, F32(C.y),
                           kSpecLd, C.spec);
    c.pad = causal_padding(7, 1);
    c.pro = fcv::HIFT_PRO_LEAKY;
    c.slope = 0.01f;
    FCV_HIP(fcv::hift_conv_f32(c, T + 5 + 3 * S, st));
  }
  FCV_HIP(fcv::hift_istft(F32(C.y), kSpecLd, window, F32(C.fr), speech, d.audio_limit, C.spec,
                          C.samples, T + 6 + 3 * S, st));
  return FCV_OK;
}

// One vocoder call over capacity (frames_cap, docs_cap): the layout's tables go into the
// workspace, then the launches run eagerly or from the pooled graph of this key.
int infer(FcvHift* h, const float* mel, const int32_t* frames, const int32_t* finalize,
          int n_docs, int frames_cap, int docs_cap, float* speech, float* source_out,
          void* workspace, size_t workspace_bytes, int use_graph, hipStream_t st) {
  FCV_CHECK(h, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(mel && speech && workspace, FCV_ERR_INVALID, "null argument");
  Plan P;
  if (int rc = make_plan(h, frames, finalize, n_docs, &P)) return rc;
  FCV_CHECK(docs_cap >= 1 && docs_cap <= FCV_HIFT_MAX_DOCS, FCV_ERR_INVALID,
            "docs_cap must be in [1, 256]");
  FCV_CHECK(P.mel[n_docs] <= frames_cap && n_docs <= docs_cap, FCV_ERR_INVALID,
            "call of " + std::to_string(P.mel[n_docs]) + " frames in " +
                std::to_string(n_docs) + " documents exceeds the capacity (" +
                std::to_string(frames_cap) + " frames, " + std::to_string(docs_cap) +
                " documents)");
  FCV_CHECK((long)frames_cap * upsample_scale(h->d) < (1L << 30), FCV_ERR_INVALID,
            "capacity too large");
  const Capacity C = make_capacity(h->d, frames_cap, docs_cap);
  FCV_CHECK(workspace_bytes >= C.total, FCV_ERR_INVALID,
            "workspace too small: need " + std::to_string(C.total) + " bytes");
  FCV_CHECK(reinterpret_cast<uintptr_t>(workspace) % kAlign == 0, FCV_ERR_INVALID,
            "workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(workspace);
  const std::vector<HiftDocs> tables = make_tables(h->d, P);
  FCV_HIP(hipMemcpyAsync(ws + C.tables, tables.data(), tables.size() * sizeof(HiftDocs),
                         hipMemcpyHostToDevice, st));
  // the table copy reads pageable host memory: it is done once this call returns
  if (!use_graph) return run(h, mel, C, speech, source_out, ws, st);

  const std::vector<uintptr_t> key = {(uintptr_t)frames_cap, (uintptr_t)docs_cap,
                                      (uintptr_t)ws, (uintptr_t)mel, (uintptr_t)speech,
                                      (uintptr_t)source_out};
  auto hit = std::find_if(h->graphs.begin(), h->graphs.end(),
                          [&](const FcvHift::Graph& g) { return g.key == key; });
  if (hit == h->graphs.end()) {
    // a capture costs more than one eager call: a key is captured on its second call
    auto seen = std::find(h->seen.begin(), h->seen.end(), key);
    if (seen == h->seen.end()) {
      h->seen.insert(h->seen.begin(), key);
      if (h->seen.size() > kSeenKeys) h->seen.pop_back();
      return run(h, mel, C, speech, source_out, ws, st);
    }
    h->seen.erase(seen);
    FCV_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int r = run(h, mel, C, speech, source_out, ws, st);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(st, &graph);
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
    if (h->graphs.size() >= kGraphPool) {
      (void)hipGraphExecDestroy(h->graphs.back().exec);
      h->graphs.pop_back();
    }
    h->graphs.insert(h->graphs.begin(), FcvHift::Graph{key, exec});
    h->captures++;
  } else if (hit != h->graphs.begin()) {
    std::rotate(h->graphs.begin(), hit, hit + 1);
  }
  FCV_HIP(hipGraphLaunch(h->graphs.front().exec, st));
  return FCV_OK;
}

}  // namespace

extern "C" {

int32_t fcv_hift_weight_count(const FcvHiftDims* dims) {
  if (check_dims(dims) != FCV_OK) return 0;
  return weight_count(*dims);
}

int fcv_hift_create(const FcvHiftDims* dims, const void* const* weights, int32_t n_weights,
                    FcvHift** out) {
  if (int rc = check_dims(dims)) return rc;
  FCV_CHECK(weights && out, FCV_ERR_INVALID, "null argument");
  const int need = weight_count(*dims);
  FCV_CHECK(n_weights == need, FCV_ERR_INVALID,
            "expected " + std::to_string(need) + " weight pointers");
  for (int i = 0; i < need; ++i) {
    FCV_CHECK(weights[i] != nullptr, FCV_ERR_INVALID,
              "null weight pointer at index " + std::to_string(i));
    FCV_CHECK(reinterpret_cast<uintptr_t>(weights[i]) % 16 == 0, FCV_ERR_INVALID,
              "weight " + std::to_string(i) + " is not 16-byte aligned");
  }
  FcvHift* h = new FcvHift();
  h->d = *dims;
  h->w.assign(weights, weights + need);
  const int S = dims->n_stages, K = dims->n_kernels, D = dims->n_dilations;
  int i = 0;
  h->i_lin = i; i += 2;
  h->i_pre = i; i += 2;
  h->i_ups = i; i += 2 * S;
  h->i_down = i; i += 2 * S;
  h->i_srb = i; i += 8 * D * S;
  h->i_rb = i; i += 8 * D * S * K;
  h->i_post = i; i += 2;
  h->i_f0 = i; i += 10;
  h->i_cls = i; i += 2;
  h->i_win = i++;
  h->i_ini = i++;
  h->i_tab = i++;
  *out = h;
  return FCV_OK;
}

int fcv_hift_destroy(FcvHift* hift) {
  if (!hift) return FCV_OK;
  for (FcvHift::Graph& g : hift->graphs) (void)hipGraphExecDestroy(g.exec);
  delete hift;
  return FCV_OK;
}

int64_t fcv_hift_output_samples(const FcvHift* hift, int32_t frames, int32_t finalize) {
  if (!hift) return -1;
  DocLens L;
  if (!doc_lens(hift->d, frames, finalize != 0, &L)) return -1;
  return L.samples;
}

size_t fcv_hift_workspace_bytes(const FcvHift* hift, const int32_t* frames_host,
                                const int32_t* finalize_host, int32_t n_docs) {
  if (!hift) return 0;
  Plan P;
  if (make_plan(hift, frames_host, finalize_host, n_docs, &P) != FCV_OK) return 0;
  return make_capacity(hift->d, P.mel[n_docs], n_docs).total;
}

size_t fcv_hift_workspace_bytes_capacity(const FcvHift* hift, int32_t frames_cap,
                                         int32_t docs_cap) {
  if (!hift || frames_cap < 1 || docs_cap < 1 || docs_cap > FCV_HIFT_MAX_DOCS) return 0;
  if ((long)frames_cap * upsample_scale(hift->d) >= (1L << 30)) return 0;
  return make_capacity(hift->d, frames_cap, docs_cap).total;
}

int fcv_hift_inference(FcvHift* hift, const float* mel, const int32_t* frames_host,
                       const int32_t* finalize_host, int32_t n_docs, float* speech_out,
                       float* source_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  FCV_CHECK(hift, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(frames_host && n_docs >= 1 && n_docs <= FCV_HIFT_MAX_DOCS, FCV_ERR_INVALID,
            "n_docs must be in [1, 256]");
  long frames = 0;
  for (int i = 0; i < n_docs; ++i) frames += std::max(frames_host[i], 0);
  FCV_CHECK(frames < (1L << 26), FCV_ERR_INVALID, "too many frames in one call");
  return infer(hift, mel, frames_host, finalize_host, n_docs, (int)frames, n_docs, speech_out,
               source_out, workspace, workspace_bytes, 0, stream);
}

int fcv_hift_inference_capacity(FcvHift* hift, const float* mel, const int32_t* frames_host,
                                const int32_t* finalize_host, int32_t n_docs, int32_t frames_cap,
                                int32_t docs_cap, float* speech_out, float* source_out,
                                void* workspace, size_t workspace_bytes, int32_t use_graph,
                                hipStream_t stream) {
  return infer(hift, mel, frames_host, finalize_host, n_docs, frames_cap, docs_cap, speech_out,
               source_out, workspace, workspace_bytes, use_graph, stream);
}

int fcv_hift_graph_stats(const FcvHift* hift, int32_t* pooled, int32_t* captures) {
  FCV_CHECK(hift, FCV_ERR_INVALID, "null handle");
  if (pooled) *pooled = (int32_t)hift->graphs.size();
  if (captures) *captures = (int32_t)std::min<long>(hift->captures, 2147483647L);
  return FCV_OK;
}

}  // extern "C"
