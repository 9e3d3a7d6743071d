// Varlen flash attention over cu_seqlens for head_dim 64 on gfx950 (MFMA 32x32x16 f16).
//
// One workgroup = one tile of 128 queries of one document x one head; 4 waves x 32 queries.
// The kernel computes S^T = K Q^T so that the fp32 accumulator of S^T (lane l owns query
// l%32 and 16 keys) can be rounded in registers and fed straight back as the B operand of
// O^T = V^T P^T: no LDS round trip for P.  Each lane therefore owns a single query column,
// so the online-softmax rescale is a per-lane scalar; the row max / row sum need one
// cross-lane exchange (lane l <-> l^32, a v_permlane32_swap).
//
// K/V tiles of 64 keys go through LDS double buffers: K row-major [key][dim] and V already
// transposed [dim][key] (the QKV epilogue writes V transposed), both padded to 72 columns.
// Documents start at 8-row aligned rows of the internal layout, so every 16-byte V^T load is
// aligned and key tiles always start at the document start: a document's key partition, and
// hence its fp32 rounding, is the same wherever it sits in the batch.  Keys at or past kv_end
// and, in chunk mode, keys in a later chunk than the query are masked to -inf.  No split-KV:
// each (query, head) is reduced by exactly one wave in key order, so results do not depend on
// the batch composition.
#include "kernels.hpp"

namespace fcv {
namespace {

constexpr int TQ = kAttnTileQ;  // queries per workgroup
constexpr int TK = 64;          // keys per LDS tile
constexpr int HD = 64;          // head dim
constexpr int LDP = 72;         // padded LDS row (f16 elements)

// v_exp_f32 without the library's denormal range reduction: results below 2^-126 flush to 0,
// which only drops probabilities that are negligible next to the row maximum's 1.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine the two wave halves (lane l and lane l ^ 32) without an LDS round trip:
// v_permlane32_swap of v with itself leaves {v[l], v[l ^ 32]} in lower-half-first order on
// every lane, so both halves compute the same fp32 result.
__device__ __forceinline__ float2 half_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ float half_max(float v) {
  const float2 p = half_pair(v);
  return fmaxf(p.x, p.y);
}
__device__ __forceinline__ float half_sum(float v) {
  const float2 p = half_pair(v);
  return p.x + p.y;
}

__global__ __launch_bounds__(256, 2) void attention_kernel(
    const f16* __restrict__ Q, const f16* __restrict__ K, const f16* __restrict__ VT,
    f16* __restrict__ O, const int4* __restrict__ tiles, int rp, int heads, int chunk,
    float scale_log2, const int32_t* __restrict__ tiles_live) {
  __shared__ __attribute__((aligned(16))) f16 sK[2][TK][LDP];
  __shared__ __attribute__((aligned(16))) f16 sV[2][HD][LDP];

  const int tile = blockIdx.x / heads;
  const int head = blockIdx.x % heads;
  // the tile's entry and the live count are fetched together (an entry past the live count is
  // inside the capacity-sized list and is not used)
  const int4 td = tiles[tile];
  const int live = tiles_live ? *tiles_live : 0x7fffffff;
  if (tile >= live) return;  // past the live tiles of a capacity grid
  const int doc_start = td.x;
  const int doc_end = doc_start + td.y;
  const int q0 = td.z;
  const int q_last = min(q0 + TQ - 1, doc_end - 1);
  int kv_end = doc_end;
  if (chunk > 0) {
    int lim = ((q_last - doc_start) / chunk + 1) * chunk;
    kv_end = min(doc_end, doc_start + lim);
  }
  const int kv_begin = doc_start;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hl = lane >> 5;      // half of the wave
  const int ql = lane & 31;      // query column owned by this lane
  const int q_row = q0 + wave * 32 + ql;
  const int q_pos = q_row - doc_start;
  // last visible key (exclusive) for this lane's query
  const int key_lim =
      chunk > 0 ? min(kv_end, doc_start + (max(q_pos, 0) / chunk + 1) * chunk) : kv_end;

  const f16* Qh = Q + (long)head * rp * HD;
  const f16* Kh = K + (long)head * rp * HD;
  const f16* Vh = VT + (long)head * HD * rp;

  // Q^T fragments (B operand): query ql, dims 16*ks + 8*hl + 0..7
  f16x8 qf[4];
  {
    const int qr = min(q_row, doc_end - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[ks] = *reinterpret_cast<const f16x8*>(Qh + (long)qr * HD + ks * 16 + hl * 8);
  }

  // tile loaders: each thread moves 2 x 16 bytes of K and 2 x 16 bytes of V^T, through raw
  // buffer loads over this head's K rows and V^T block: 32-bit offsets, and chunks past the end
  // read as zeros (keys past the document are masked anyway).  A V^T chunk holds 8 keys from a
  // multiple of 8 (documents start 8-aligned); keys at or past kv_end are zeroed when the chunk
  // is stashed.  The next tile is fetched unconditionally (the surplus tile lands in the buffer
  // no later iteration reads), so the compiler never waits on a load before the stash that
  // consumes it.  (Descriptor word 3 = 0x00020000: 32-bit data format, no swizzle.)
  const int lr = tid >> 3;         // 0..31
  const int lc = (tid & 7) * 8;    // 0..56
  const __amdgpu_buffer_rsrc_t k_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(Kh), (short)0, rp * HD * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(Vh), (short)0, HD * rp * 2, 0x00020000);
  const uint32_t k_lane = (uint32_t)(lr * HD + lc) * 2, v_lane = (uint32_t)(lr * rp) * 2;
  f16x8 rk[2], rv[2];
  int vcnt = 8;  // keys of this thread's V^T chunks below kv_end
  auto fetch = [&](int kb) {
    const int k0 = kb + lc;
    vcnt = kv_end - k0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      rk[i] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                      k_rsrc, k_lane + (uint32_t)(kb + 32 * i) * HD * 2, 0, 0));
      rv[i] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                      v_rsrc, v_lane + (uint32_t)(32 * i * rp + k0) * 2, 0, 0));
    }
  };
  auto stash = [&](int buf) {
    if (vcnt < 8) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) rv[i][e] = e < vcnt ? rv[i][e] : (f16)0.0f;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<f16x8*>(&sK[buf][lr + 32 * i][lc]) = rk[i];
      *reinterpret_cast<f16x8*>(&sV[buf][lr + 32 * i][lc]) = rv[i];
    }
  };

  f32x16 acc_o[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  // keys below wave_lim are visible to every query of this wave: those tiles skip the mask
  int wave_lim = key_lim;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) wave_lim = min(wave_lim, __shfl_xor(wave_lim, off, kWave));

  const int n_kt = (kv_end - kv_begin + TK - 1) / TK;
  fetch(kv_begin);
  stash(0);
  __syncthreads();

  for (int it = 0; it < n_kt; ++it) {
    const int cur = it & 1;
    const int kb = kv_begin + it * TK;
    fetch(kb + TK);

    // S^T[key][query] for two 32-key halves (raw q.k)
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kt][e] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        f16x8 kf = *reinterpret_cast<const f16x8*>(&sK[cur][kt * 32 + ql][ks * 16 + hl * 8]);
        s[kt] = mfma32(kf, qf[ks], s[kt]);
      }
    }

    // online softmax in base 2: p = exp2(s * scale_log2 - m), m the running max of s * scale_log2
    float tmax = -INFINITY;
    if (kb + TK <= wave_lim) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[kt][e]);
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kb + kt * 32 + (e >> 2) * 8 + hl * 4 + (e & 3);
          s[kt][e] = key < key_lim ? s[kt][e] : -INFINITY;
          tmax = fmaxf(tmax, s[kt][e]);
        }
      }
    }
    tmax = half_max(tmax);
    const float m_new = fmaxf(m_run, tmax * scale_log2);
    if (__ballot(m_new > m_run)) {
      // some query of the wave has a new maximum: rescale its partial sums
      const float corr = fast_exp2(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[i][e] *= corr;
      m_run = m_new;
    }
    float psum = 0.0f;
    f16x8 pf[4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = fast_exp2(fmaf(s[kt][e], scale_log2, -m_new));
        psum += p;
        // a plain cast: p is an exponential, not a product, so no multiply can be fused into
        // the conversion here
        pf[kt * 2 + (e >> 3)][e & 7] = (f16)p;
      }
    }
    l_run += psum;

    // O^T[d][q] += V^T[d][key] P^T[key][q]; slot j of step s <-> key
    //   32*(s/2) + 16*(s%2) + 8*(j/4) + 4*hl + j%4  (same rule as the S^T accumulator)
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kbase = (st >> 1) * 32 + (st & 1) * 16 + hl * 4;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const f16* vrow = &sV[cur][dt * 32 + ql][0];
        f16x4 lo = *reinterpret_cast<const f16x4*>(vrow + kbase);
        f16x4 hi = *reinterpret_cast<const f16x4*>(vrow + kbase + 8);
        f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc_o[dt] = mfma32(vf, pf[st], acc_o[dt]);
      }
    }

    stash(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = half_sum(l_run);
  const float inv = 1.0f / l_tot;
  if (q_row < doc_end) {
    f16* dst = O + (long)q_row * heads * HD + head * HD;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = dt * 32 + a * 8 + hl * 4;
        f16x4 pk = f2h4(acc_o[dt][4 * a + 0] * inv, acc_o[dt][4 * a + 1] * inv,
                        acc_o[dt][4 * a + 2] * inv, acc_o[dt][4 * a + 3] * inv);
        *reinterpret_cast<f16x4*>(dst + d) = pk;
      }
    }
  }
}

}  // namespace

hipError_t attention_varlen(const f16* q, const f16* k, const f16* vt, f16* o,
                            const int32_t* tiles, int n_tiles, int rp, int heads, int chunk,
                            hipStream_t stream, const int32_t* tiles_live) {
  if (n_tiles <= 0) return hipSuccess;
  // per-head K rows and V^T blocks are addressed by 32-bit buffer offsets
  if ((long)HD * rp * 2 >= (1L << 31)) return hipErrorInvalidValue;
  const float scale_log2 = 0.125f * 1.4426950408889634f;  // 64^-0.5 * log2(e)
  if (reinterpret_cast<uintptr_t>(tiles) % 16 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel, dim3(n_tiles * heads), dim3(256), 0, stream, q, k, vt, o,
                     reinterpret_cast<const int4*>(tiles), rp, heads, chunk, scale_log2,
                     tiles_live);
  return hipGetLastError();
}

}  // namespace fcv
