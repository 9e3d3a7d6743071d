// C ABI of the HiFT vocoder (include/fcv_hift.h): validation, per-call document tables, the
// workspace carve-up and the launch sequence of CausalHiFTGenerator.inference over packed
// documents.
#include <algorithm>
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

struct Plan {
  int n_docs;
  std::vector<DocLens> lens;
  // prefix sums
  std::vector<int> mel, f0, x, spec, samples, src;
  std::vector<std::vector<int>> stage;  // compute rows of stage i (no reflection pad)
  // workspace carve-up (byte offsets)
  size_t mel64, h64a, h64b, f0buf, sines, srcbuf, specbuf, xa, xn, xs, r, t1, s1, si, y, fr,
      total;
  size_t stage_max;  // floats per stage buffer
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
  size_t smax = (size_t)P->x[n_docs] * d.base_channels;
  int rate = 1;
  for (int s = 0; s < d.n_stages; ++s) {
    rate *= d.upsample_rates[s];
    for (int i = 0; i < n_docs; ++i) P->stage[s][i + 1] = P->stage[s][i] + P->lens[i].x * rate;
    const size_t rows_w = (size_t)P->stage[s][n_docs] + (s == d.n_stages - 1 ? n_docs : 0);
    smax = std::max(smax, rows_w * stage_channels(d, s));
  }
  P->stage_max = smax;
  const int H = d.nb_harmonics + 1;
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += align_up(bytes); return o; };
  P->mel64 = take(sizeof(double) * P->mel[n_docs] * d.in_channels);
  P->h64a = take(sizeof(double) * P->f0[n_docs] * d.f0_channels);
  P->h64b = take(sizeof(double) * P->f0[n_docs] * d.f0_channels);
  P->f0buf = take(sizeof(float) * P->f0[n_docs]);
  P->sines = take(sizeof(float) * P->f0[n_docs] * H);
  P->srcbuf = take(sizeof(float) * P->src[n_docs]);
  P->specbuf = take(sizeof(float) * P->spec[n_docs] * kSpecLd);
  for (size_t* b : {&P->xa, &P->xn, &P->xs, &P->r, &P->t1, &P->s1, &P->si})
    *b = take(sizeof(float) * smax);
  P->y = take(sizeof(float) * P->spec[n_docs] * kSpecLd);
  P->fr = take(sizeof(float) * P->spec[n_docs] * kFrameLd);
  P->total = off;
  return FCV_OK;
}

HiftDocs docs_of(const std::vector<int>& a, const std::vector<int>& b) {
  HiftDocs t{};
  for (size_t i = 0; i < a.size(); ++i) t.a[i] = a[i];
  for (size_t i = 0; i < b.size(); ++i) t.b[i] = b[i];
  return t;
}

HiftConv conv_base(const void* x, int ldx, const void* w, const void* b, int cout, int cin_pad,
                   int k, void* out, int ldo, int rows_out, int n_docs) {
  HiftConv p{};
  p.x = x; p.ldx = ldx; p.w = w; p.bias = b; p.cout = cout; p.cin_pad = cin_pad; p.k = k;
  p.stride = 1; p.dil = 1; p.pad = 0; p.up = 1; p.rows_out = rows_out; p.n_docs = n_docs;
  p.out = out; p.ldo = ldo; p.div = 1.0f;
  return p;
}

// one ResBlock (generator.py:110-116) on x (rows by `docs`, C channels): for each dilation
// j: r = r + conv2(snake2(conv1(snake1(r)))); the last conv2 writes its result per `mode`
// (write / accin + y / (accin + y) / div) into `out`.  `wb` points at the block's 8 * D
// weight pointers.  x is read as the first residual; r holds the running value.
int run_resblock(const FcvHiftDims& d, const void* const* wb, int k, const int* dils,
                 const float* x, float* r, float* t1, float* s1, float* out, int mode,
                 const float* accin, float div, int C, int rows, const HiftDocs& docs,
                 int n_docs, hipStream_t st) {
  const int D = d.n_dilations;
  FCV_HIP(fcv::hift_snake(x, C, s1, C, rows, C, static_cast<const float*>(wb[4]),
                          static_cast<const float*>(wb[5]), st));
  for (int j = 0; j < D; ++j) {
    const void* const* q = wb + 8 * j;
    HiftConv c1 = conv_base(s1, C, q[0], q[1], C, C, k, t1, C, rows, n_docs);
    c1.dil = dils[j];
    c1.pad = causal_padding(k, dils[j]);
    c1.snake_out = 1;
    c1.alpha = static_cast<const float*>(q[6]);
    c1.inv_alpha = static_cast<const float*>(q[7]);
    FCV_HIP(fcv::hift_conv_f32(c1, docs, st));
    const bool last = j == D - 1;
    HiftConv c2 = conv_base(t1, C, q[2], q[3], C, C, k, last ? out : r, C, rows, n_docs);
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

int run(FcvHift* h, const float* mel, const Plan& P, float* speech, float* source_out,
        char* ws, hipStream_t st) {
  const FcvHiftDims& d = h->d;
  const int n = P.n_docs;
  const void* const* w = h->w.data();
  auto F32 = [&](size_t o) { return reinterpret_cast<float*>(ws + o); };
  auto F64 = [&](size_t o) { return reinterpret_cast<double*>(ws + o); };
  const int H = d.nb_harmonics + 1;
  const int scale = upsample_scale(d);

  // ---- F0 predictor (fp64) -------------------------------------------------------------
  FCV_HIP(fcv::hift_to_f64(mel, F64(P.mel64), (long)P.mel[n] * d.in_channels, st));
  const HiftDocs d_f0_in = docs_of(P.mel, P.f0);
  const HiftDocs d_f0 = docs_of(P.f0, P.f0);
  const int fc = d.f0_channels;
  HiftConv c0 = conv_base(F64(P.mel64), d.in_channels, w[h->i_f0], w[h->i_f0 + 1], fc,
                          d.in_channels, 4, F64(P.h64a), fc, P.f0[n], n);
  c0.elu = 1;  // right-side lookahead: no left padding, zero (or context) on the right
  FCV_HIP(fcv::hift_conv_f64(c0, d_f0_in, st));
  double* hin = F64(P.h64a);
  double* hout = F64(P.h64b);
  for (int l = 1; l < 5; ++l) {
    HiftConv c = conv_base(hin, fc, w[h->i_f0 + 2 * l], w[h->i_f0 + 2 * l + 1], fc, fc, 3, hout,
                           fc, P.f0[n], n);
    c.pad = causal_padding(3, 1);
    c.elu = 1;
    FCV_HIP(fcv::hift_conv_f64(c, d_f0, st));
    std::swap(hin, hout);
  }
  FCV_HIP(fcv::hift_f0_head(hin, fc, static_cast<const double*>(w[h->i_cls]),
                            static_cast<const double*>(w[h->i_cls + 1]), P.f0[n], F32(P.f0buf),
                            st));

  // ---- harmonic source and its STFT ------------------------------------------------------
  fcv::HiftSource src{};
  src.f0 = F32(P.f0buf);
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
  src.n_docs = n;
  src.sines = F32(P.sines);
  src.s = F32(P.srcbuf);
  FCV_HIP(fcv::hift_source(src, docs_of(P.f0, P.src), st));
  if (source_out)
    FCV_HIP(hipMemcpyAsync(source_out, F32(P.srcbuf), sizeof(float) * P.src[n],
                           hipMemcpyDeviceToDevice, st));
  const float* window = static_cast<const float*>(w[h->i_win]);
  FCV_HIP(fcv::hift_stft(F32(P.srcbuf), window, F32(P.specbuf), kSpecLd, n, P.spec[n],
                         docs_of(P.src, P.spec), st));

  // ---- conv_pre (lookahead on the right) -------------------------------------------------
  float* xp = F32(P.xa);
  float* xn = F32(P.xn);
  {
    HiftConv c = conv_base(mel, d.in_channels, w[h->i_pre], w[h->i_pre + 1], d.base_channels,
                           d.in_channels, d.conv_pre_look_right + 1, xp, d.base_channels,
                           P.x[n], n);
    FCV_HIP(fcv::hift_conv_f32(c, docs_of(P.mel, P.x), st));
  }

  // ---- upsampling stages -----------------------------------------------------------------
  std::vector<int> prev = P.x;
  int cprev = d.base_channels;
  const int rb_size = 8 * d.n_dilations;
  for (int s = 0; s < d.n_stages; ++s) {
    const int C = stage_channels(d, s);
    const bool last = s == d.n_stages - 1;
    // write layout: the last stage carries one reflection-pad row per document
    std::vector<int> rows_w = P.stage[s];
    if (last)
      for (int i = 0; i <= n; ++i) rows_w[i] += i;
    const int nrows = rows_w[n];
    const HiftDocs dw = docs_of(rows_w, rows_w);

    // source branch: strided (or 1x1) conv of the STFT frames, then its resblock
    float* si = F32(P.si);
    {
      const auto kd = source_down(d, s);
      HiftConv c = conv_base(F32(P.specbuf), kSpecLd, w[h->i_down + 2 * s],
                             w[h->i_down + 2 * s + 1], C, kSpecLd, kd.first, si, C, nrows, n);
      c.stride = kd.second;
      c.pad = kd.second - 1;
      FCV_HIP(fcv::hift_conv_f32(c, docs_of(P.spec, rows_w), st));
      if (int rc = run_resblock(d, w + h->i_srb + rb_size * s, d.source_kernels[s],
                                d.source_dilations[s], si, F32(P.r), F32(P.t1), F32(P.s1), si,
                                fcv::HIFT_ACC_WRITE, nullptr, 1.0f, C, nrows, dw, n, st))
        return rc;
    }
    // upsampling conv on LeakyReLU(x), plus the source branch
    {
      HiftConv c = conv_base(xp, cprev, w[h->i_ups + 2 * s], w[h->i_ups + 2 * s + 1], C, cprev,
                             d.upsample_kernels[s], xn, C, P.stage[s][n], n);
      c.up = d.upsample_rates[s];
      c.pad = d.upsample_kernels[s] - 1;
      c.pro = fcv::HIFT_PRO_LEAKY;
      c.slope = d.lrelu_slope;
      c.reflect = last ? 1 : 0;
      c.add = si;
      c.ld_add = C;
      FCV_HIP(fcv::hift_conv_f32(c, docs_of(prev, P.stage[s]), st));
    }
    // mean of the resblocks
    for (int j = 0; j < d.n_kernels; ++j) {
      const int K = d.n_kernels;
      int mode = fcv::HIFT_ACC_WRITE;
      float* out = F32(P.xs);
      const float* accin = nullptr;
      float div = 1.0f;
      if (K == 1) {
        out = xn;
      } else if (j == K - 1) {
        mode = fcv::HIFT_ACC_ADD_DIV;
        accin = F32(P.xs);
        out = xn;
        div = (float)K;
      } else if (j > 0) {
        mode = fcv::HIFT_ACC_ADD;
        accin = F32(P.xs);
      }
      if (int rc = run_resblock(d, w + h->i_rb + rb_size * (s * K + j), d.resblock_kernels[j],
                                d.resblock_dilations[j], xn, F32(P.r), F32(P.t1), F32(P.s1),
                                out, mode, accin, div, C, nrows, dw, n, st))
        return rc;
    }
    prev = rows_w;
    cprev = C;
    std::swap(xp, xn);
  }

  // ---- conv_post on LeakyReLU(x) (slope 0.01), iSTFT, clamp ------------------------------
  {
    const int spec = d.n_fft + 2;
    HiftConv c = conv_base(xp, cprev, w[h->i_post], w[h->i_post + 1], spec, cprev, 7, F32(P.y),
                           kSpecLd, P.spec[n], n);
    c.pad = causal_padding(7, 1);
    c.pro = fcv::HIFT_PRO_LEAKY;
    c.slope = 0.01f;
    FCV_HIP(fcv::hift_conv_f32(c, docs_of(prev, P.spec), st));
  }
  FCV_HIP(fcv::hift_istft(F32(P.y), kSpecLd, window, F32(P.fr), speech, d.audio_limit, n,
                          P.spec[n], P.samples[n], docs_of(P.spec, P.samples), st));
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
  return P.total;
}

int fcv_hift_inference(FcvHift* hift, const float* mel, const int32_t* frames_host,
                       const int32_t* finalize_host, int32_t n_docs, float* speech_out,
                       float* source_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  FCV_CHECK(hift, FCV_ERR_INVALID, "null handle");
  FCV_CHECK(mel && speech_out && workspace, FCV_ERR_INVALID, "null argument");
  Plan P;
  if (int rc = make_plan(hift, frames_host, finalize_host, n_docs, &P)) return rc;
  FCV_CHECK(workspace_bytes >= P.total, FCV_ERR_INVALID,
            "workspace too small: need " + std::to_string(P.total) + " bytes");
  FCV_CHECK(reinterpret_cast<uintptr_t>(workspace) % kAlign == 0, FCV_ERR_INVALID,
            "workspace must be 256-byte aligned");
  return run(hift, mel, P, speech_out, source_out, static_cast<char*>(workspace), stream);
}

}  // extern "C"
