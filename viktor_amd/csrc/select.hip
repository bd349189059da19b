// Fused LM head + token choice + decode-state update (one workgroup of 256 threads per sequence).
//
// Semantics (viktor/engine.py:79-116 and viktor/triton_ops.py:172-209):
//   z = logits + bias (bias = -inf at PAD and BOS);
//   greedy: first index of max(z); sampled: inverse CDF of softmax(z / T) at the supplied uniform, or
//   (gumbel) the reference's own formula, first index of max(z / T - log(-log(max(u_v, 1e-20)))) with one
//   supplied uniform per vocabulary entry -- the reference draws those uniforms from the device RNG
//   (viktor/engine.py:80-83), supplied ones make the stream reproducible;
//   grammar, in the reference's order: EOS after a tail token; homopolymer run counter and EOS when the
//   run reaches homo_stop tokens; PAD after EOS / PAD;
//   out[b, pos - plen] = token; tok = token; pos += 1 and the int32 mirrors pos32 = pos,
//   seqlens = pos + 1, rpos32 = pos + rope_off.
// The LM head is computed here from the final hidden state (bf16 x bf16 -> fp32, optionally rounded to
// bf16 as an nn.Linear in bf16 would) or read as fp32 logits.
#include <math.h>

#include "common.h"

namespace vk {

constexpr int SEL_THREADS = 256;
constexpr int SEL_MAXV = 512;

// Sum over the 64 lanes, every lane receiving it, with no LDS round trip: DPP lane swaps within quads (xor 1,
// xor 2), the mirrors within 8 and 16 lanes, then gfx950's permlane16 / permlane32 swaps. Each step adds two
// values that are also added, in the other order, on the partner lane, so all lanes hold the same bits.
__device__ __forceinline__ float sel_wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row mirror
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

// MAXC: 512-wide chunks of the hidden row per lane (d <= 512 MAXC). Every global load the choice needs is
// issued before the first use of any (the sequence state, the uniform, the hidden slice, the norm weight and
// the first two LM-head rows of each wave): loads in branches or after a use would each cost a round trip.
template <int MAXC>
__global__ __launch_bounds__(SEL_THREADS) void select_update_kernel(
    const float *__restrict__ logits, const bf16_t *__restrict__ h, const bf16_t *__restrict__ norm_w, float eps,
    const bf16_t *__restrict__ w_head, int d, int round_bf16, const float *__restrict__ bias, const uint8_t *__restrict__ is_tail,
    const uint8_t *__restrict__ is_homo, int homo_stop, float temperature, const float *__restrict__ uniforms,
    int64_t u_stride, int64_t u_cols, int gumbel, int64_t *__restrict__ tok, int64_t *__restrict__ run, int64_t *__restrict__ pos,
    const int64_t *__restrict__ plen, const int64_t *__restrict__ rope_off, const int64_t *__restrict__ cache_base,
    int64_t *__restrict__ out, int64_t out_stride, int64_t out_cols, int32_t *__restrict__ pos32,
    int32_t *__restrict__ seqlens, int32_t *__restrict__ rpos32, float *__restrict__ logp_out, int64_t logp_stride,
    int V, int eos, int pad) {
  __shared__ float z[SEL_MAXV];
  __shared__ float ez[SEL_MAXV];
  __shared__ uint8_t homo_s[SEL_MAXV];
  __shared__ float red_v[SEL_THREADS / 64];
  __shared__ int red_i[SEL_THREADS / 64];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const bool sample = temperature > 0.f;
  const float tdiv = sample ? temperature : 1.f;  // z / 1 is z: one expression for both modes

  // 0. the LM head's operands first (they depend on nothing the sequence's state holds): this lane's slice of the
  // hidden row (chunks of 8 at lane * 8 + 512 c; past d: column 0, unused), the norm weight and this wave's first
  // two LM-head rows (v = wid, wid + 4; past V: row V - 1, unused)
  const bool head = logits == nullptr;
  const int v0 = wid < V ? wid : V - 1, v1 = wid + 4 < V ? wid + 4 : V - 1;
  u32x4 hraw[MAXC], nraw[MAXC], w0raw[MAXC], w1raw[MAXC];
  float b0 = 0.f, b1 = 0.f;
  if (head) {
    const bf16_t *hr = h + b * d;
    const bf16_t *nw = norm_w ? norm_w : hr;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int k = lane * 8 + 512 * c, kk = k < d ? k : 0;
      hraw[c] = *reinterpret_cast<const u32x4 *>(hr + kk);
      nraw[c] = *reinterpret_cast<const u32x4 *>(nw + kk);
      w0raw[c] = *reinterpret_cast<const u32x4 *>(w_head + static_cast<int64_t>(v0) * d + kk);
      w1raw[c] = *reinterpret_cast<const u32x4 *>(w_head + static_cast<int64_t>(v1) * d + kk);
    }
    b0 = bias[v0];
    b1 = bias[v1];
  }
  // then the sequence's state (wave-uniform loads; an optional pointer that is NULL reads pos instead, discarded),
  // and the two loads that depend on it (the uniform at the output column, the previous token's tail flag), kept
  // as raw values until the choice, so no wait for them lands before the LM head
  const int64_t p = pos[b];
  const int64_t pl_raw = (plen ? plen : pos)[b];
  const int64_t prev = tok[b];
  const int64_t run_raw = (run ? run : pos)[b];
  const int64_t ro_raw = (rope_off ? rope_off : pos)[b];
  const int64_t cb_raw = (cache_base ? cache_base : pos)[b];
  const int64_t pl = plen ? pl_raw : 0;
  const int64_t ocol = p - pl;
  const int64_t uc = ocol < 0 ? 0 : (ocol >= u_cols ? u_cols - 1 : ocol);
  const float u_raw = (uniforms && !gumbel) ? uniforms[b * u_stride + uc] : 0.f;
  // gumbel: this thread's entries v = tid, tid + 256 of the column's V uniforms (past V: entry 0, unused)
  float ug[SEL_MAXV / SEL_THREADS] = {};
  if (gumbel && sample) {
#pragma unroll
    for (int i = 0; i < SEL_MAXV / SEL_THREADS; ++i) {
      const int v = tid + SEL_THREADS * i;
      ug[i] = uniforms[b * u_stride + uc * V + (v < V ? v : 0)];
    }
  }
  const int64_t pv = prev >= 0 && prev < V ? prev : 0;
  const uint8_t tail_raw = is_tail[pv];

  // 1. logits (+ bias), fp32
  if (!head) {
    for (int v = tid; v < V; v += SEL_THREADS) z[v] = (logits[b * V + v] + bias[v]) / tdiv;
  } else {
    float hv[MAXC][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const bool live = lane * 8 + 512 * c < d;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hv[c][2 * j] = live ? lo_bf(hraw[c][j]) : 0.f;
        hv[c][2 * j + 1] = live ? hi_bf(hraw[c][j]) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += hv[c][j] * hv[c][j];
    }
    if (norm_w != nullptr) {
      const float r = rsqrtf(sel_wave_sum(ss) / static_cast<float>(d) + eps);
#pragma unroll
      for (int c = 0; c < MAXC; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          hv[c][2 * j] = round_bf(hv[c][2 * j] * r * lo_bf(nraw[c][j]));
          hv[c][2 * j + 1] = round_bf(hv[c][2 * j + 1] * r * hi_bf(nraw[c][j]));
        }
    }
    auto dot = [&](const u32x4 (&wr)[MAXC]) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < MAXC; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += hv[c][2 * j] * lo_bf(wr[c][j]) + hv[c][2 * j + 1] * hi_bf(wr[c][j]);
      return sel_wave_sum(acc);
    };
    const float a0 = dot(w0raw), a1 = dot(w1raw);
    if (lane == 0 && wid < V) z[wid] = ((round_bf16 ? round_bf(a0) : a0) + b0) / tdiv;
    if (lane == 0 && wid + 4 < V) z[wid + 4] = ((round_bf16 ? round_bf(a1) : a1) + b1) / tdiv;
    // larger vocabularies: this wave's further rows v = wid + 8 + 4 i, eight rows' loads in flight per round trip
    // (rows past V load row V - 1 and are not written)
    constexpr int RB = 8;
    for (int v0b = wid + 8; v0b < V; v0b += RB * (SEL_THREADS / 64)) {
      u32x4 wr[RB][MAXC];
      float bv[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int v = v0b + r * (SEL_THREADS / 64), vc = v < V ? v : V - 1;
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
          const int k = lane * 8 + 512 * c, kk = k < d ? k : 0;
          wr[r][c] = *reinterpret_cast<const u32x4 *>(w_head + static_cast<int64_t>(vc) * d + kk);
        }
        bv[r] = bias[vc];
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int v = v0b + r * (SEL_THREADS / 64);
        const float acc = dot(wr[r]);
        if (lane == 0 && v < V) z[v] = ((round_bf16 ? round_bf(acc) : acc) + bv[r]) / tdiv;
      }
    }
  }
  if (homo_stop > 0)
    for (int v = tid; v < V; v += SEL_THREADS) homo_s[v] = is_homo[v];
  __syncthreads();

  // 2. max with first-index tie-break (greedy choice and softmax shift)
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int v = tid; v < V; v += SEL_THREADS) {
    const float zv = z[v];
    if (zv > best || (zv == best && v < bi)) {
      best = zv;
      bi = v;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    red_v[wid] = best;
    red_i[wid] = bi;
  }
  __syncthreads();
  // every thread merges the waves' (max, index) the same way, so all know the shift
  best = red_v[0];
  bi = red_i[0];
  for (int w = 1; w < SEL_THREADS / 64; ++w)
    if (red_v[w] > best || (red_v[w] == best && red_i[w] < bi)) {
      best = red_v[w];
      bi = red_i[w];
    }
  if (bi >= V) bi = 0;  // all -inf / NaN row: fall back to token 0 (PAD)
  const float zmax = best;
  // gumbel: the first index of the maximum of z / T - log(-log(max(u, 1e-20))), merged like the max above
  int gpick = bi;
  if (gumbel && sample) {
    float gb = -INFINITY;
    int gi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < SEL_MAXV / SEL_THREADS; ++i) {
      const int v = tid + SEL_THREADS * i;
      if (v < V) {
        const float zg = z[v] - logf(-logf(fmaxf(ug[i], 1e-20f)));
        if (zg > gb || (zg == gb && v < gi)) {
          gb = zg;
          gi = v;
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(gb, o, 64);
      const int oi = __shfl_xor(gi, o, 64);
      if (ov > gb || (ov == gb && oi < gi)) {
        gb = ov;
        gi = oi;
      }
    }
    __syncthreads();  // every thread has read the max's partials
    if (lane == 0) {
      red_v[wid] = gb;
      red_i[wid] = gi;
    }
    __syncthreads();
    gb = red_v[0];
    gi = red_i[0];
    for (int w = 1; w < SEL_THREADS / 64; ++w)
      if (red_v[w] > gb || (red_v[w] == gb && red_i[w] < gi)) {
        gb = red_v[w];
        gi = red_i[w];
      }
    gpick = gi < V ? gi : bi;
  }
  const bool need_e = sample || logp_out;
  if (need_e) {  // the exponentials, one token per thread (summed in token order below)
    for (int v = tid; v < V; v += SEL_THREADS) ez[v] = expf(z[v] - zmax);
    __syncthreads();
  }
  if (tid != 0) return;

  // 3. choice (single thread: the CDF is accumulated in token order)
  const float u = sample ? u_raw : 0.f;
  const bool prev_tail = prev >= 0 && prev < V && tail_raw != 0;
  int64_t nxt = bi;
  float sum = 0.f;
  if (need_e) {
    for (int v = 0; v < V; ++v) sum += ez[v];
  }
  if (sample && gumbel) {
    nxt = gpick;
  } else if (sample) {
    const float inv = 1.0f / sum;
    float cdf = 0.f;
    int64_t pick = -1, last_pos = bi;
    for (int v = 0; v < V; ++v) {
      const float pv = ez[v] * inv;
      if (pv > 0.f) last_pos = v;
      cdf += pv;
      if (pick < 0 && u < cdf) pick = v;
    }
    nxt = pick >= 0 ? pick : last_pos;
  }
  if (logp_out) {
    const float lp = z[nxt] - zmax - logf(sum);
    if (logp_stride == 0) logp_out[b] = lp;
    else if (ocol >= 0 && ocol < out_cols) logp_out[b * logp_stride + ocol] = lp;
  }

  // 4. grammar and bookkeeping
  if (prev_tail) nxt = eos;
  if (homo_stop > 0) {
    const bool same = nxt == prev && nxt >= 0 && nxt < V && homo_s[nxt];
    const int64_t r = same ? run_raw + 1 : 0;
    run[b] = r;
    if (r + 1 >= homo_stop) nxt = eos;
  }
  if (prev == eos || prev == pad) nxt = pad;
  if (ocol >= 0 && ocol < out_cols) out[b * out_stride + ocol] = nxt;
  tok[b] = nxt;
  const int64_t np = p + 1;
  pos[b] = np;
  // cache_base: the KV-cache row of position p is p - cache_base[b] (a per-sequence suffix cache)
  const int64_t cp = np - (cache_base ? cb_raw : 0);
  if (pos32) pos32[b] = static_cast<int32_t>(cp);
  if (seqlens) seqlens[b] = static_cast<int32_t>(cp + 1);
  if (rpos32) rpos32[b] = static_cast<int32_t>(np + (rope_off ? ro_raw : 0));
}

}  // namespace vk

using namespace vk;

extern "C" int vk_select_update(const float *logits, const void *h, const void *norm_w, float eps, const void *w_head,
                                int32_t d, int32_t round_bf16,
                                const float *bias, const uint8_t *is_tail, const uint8_t *is_homo, int32_t homo_stop,
                                float temperature, const float *uniforms, int64_t u_stride, int64_t u_cols,
                                int32_t gumbel, int64_t *tok, int64_t *run, int64_t *pos, const int64_t *plen, const int64_t *rope_off,
                                const int64_t *cache_base, int64_t *out, int64_t out_stride, int64_t out_cols, int32_t *pos32, int32_t *seqlens,
                                int32_t *rpos32, float *logp_out, int64_t logp_stride, int64_t B, int32_t V,
                                int32_t eos, int32_t pad, void *stream) {
  VK_CHECK_ARG(bias && is_tail && is_homo && tok && pos && out, "select_update: null pointer");
  VK_CHECK_ARG(V > 0 && V <= SEL_MAXV, "select_update: vocab must be in 1..%d (got %d)", SEL_MAXV, V);
  VK_CHECK_ARG(B >= 0 && B < (int64_t(1) << 31), "select_update: bad batch");
  VK_CHECK_ARG((logits != nullptr) != (h != nullptr && w_head != nullptr),
               "select_update: pass either logits or (h, w_head)");
  VK_CHECK_ARG(logits != nullptr || (d > 0 && d % 8 == 0 && d <= 2048 && vk_aligned16(h) && vk_aligned16(w_head) &&
                                      (!norm_w || vk_aligned16(norm_w))),
               "select_update: LM head needs d %% 8 == 0, d <= 2048 and 16-byte aligned h, w_head, norm_w");
  VK_CHECK_ARG(homo_stop <= 0 || run != nullptr, "select_update: homopolymer rule needs run");
  VK_CHECK_ARG(!(temperature > 0.f) || (uniforms != nullptr && u_cols > 0), "select_update: sampling needs uniforms");
  VK_CHECK_ARG(!gumbel || u_stride >= u_cols * V, "select_update: Gumbel uniforms are [B, u_cols, V] (row stride %lld)",
               static_cast<long long>(u_stride));
  VK_CHECK_ARG(out_cols > 0, "select_update: empty output buffer");
  VK_CHECK_ARG(logp_stride == 0 || logp_stride >= out_cols, "select_update: logp_stride must be 0 or >= out_cols");
  if (B == 0) return VK_OK;
  auto kern = (logits != nullptr || d <= 512) ? select_update_kernel<1> : select_update_kernel<4>;
  kern<<<static_cast<unsigned>(B), SEL_THREADS, 0, VK_STREAM(stream)>>>(
      logits, static_cast<const bf16_t *>(h), static_cast<const bf16_t *>(norm_w), eps,
      static_cast<const bf16_t *>(w_head), d, round_bf16, bias, is_tail,
      is_homo, homo_stop, temperature, uniforms, u_stride, u_cols, gumbel != 0, tok, run, pos, plen, rope_off,
      cache_base, out,
      out_stride,
      out_cols, pos32, seqlens, rpos32, logp_out, logp_stride, V, eos, pad);
  return launch_status("select_update");
}
