// GSPO scoring: per-token log-probabilities of the sampled tokens, the sequence-level importance ratio,
// the clipped objective and its gradient with respect to the logits, plus group-normalised advantages.
//
// Semantics: scripts/gspo.py:340-353 (token_logprobs: log_softmax over the fp32 logits, gathered at the
// PAD-clamped targets) and scripts/gspo.py:446-477 (advantages; s = exp(sum of masked (lp - old) /
// n_bases); pg = -min(s A, clamp(s, 1 - eps, 1 + eps) A); loss = sum(pg) / N). The gradient is the
// closed form of autograd through those ops:
//   dL/dz[b,t,v] = (1/N) g_b s_b mask[b,t] / n_bases[b] (onehot(y)[v] - softmax(z[b,t])[v]),
//   g_b = d pg_b / d s_b, with torch.minimum splitting ties evenly and clamp passing its gradient on
//   the closed interval.
// One workgroup per sequence; tokens are spread over threads (small vocabularies) or wavefronts
// (large ones); every reduction runs in a fixed order, so results are bitwise reproducible.
#include <math.h>

#include "common.h"

namespace vk {

constexpr int GS_THREADS = 256;

template <bool BF16>
__device__ __forceinline__ float logit_at(const void *p, int64_t i) {
  if (BF16) return bf2f(static_cast<const bf16_t *>(p)[i]);
  return static_cast<const float *>(p)[i];
}

// log-sum-exp and max of one token's logits, computed by one thread
template <bool BF16>
__device__ __forceinline__ void lse_thread(const void *lg, int64_t base, int V, float &mx, float &lse) {
  mx = -INFINITY;
  for (int v = 0; v < V; ++v) mx = fmaxf(mx, logit_at<BF16>(lg, base + v));
  float s = 0.f;
  for (int v = 0; v < V; ++v) s += expf(logit_at<BF16>(lg, base + v) - mx);
  lse = mx + logf(s);
}

// ... by one wavefront (every lane gets the result)
template <bool BF16>
__device__ __forceinline__ void lse_wave(const void *lg, int64_t base, int V, int lane, float &mx, float &lse) {
  mx = -INFINITY;
  for (int v = lane; v < V; v += 64) mx = fmaxf(mx, logit_at<BF16>(lg, base + v));
  mx = wave_max(mx);
  float s = 0.f;
  for (int v = lane; v < V; v += 64) s += expf(logit_at<BF16>(lg, base + v) - mx);
  s = wave_sum(s);
  lse = mx + logf(s);
}

__device__ __forceinline__ float block_sum(float v, float *scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < GS_THREADS / 64; ++w) t += scratch[w];
  return t;
}

template <bool BF16, bool WAVE_PER_TOKEN>
__global__ __launch_bounds__(GS_THREADS) void gspo_score_kernel(
    const void *__restrict__ logits, const int64_t *__restrict__ targets, const uint8_t *__restrict__ mask,
    const float *__restrict__ old_lp, const float *__restrict__ n_bases, const float *__restrict__ adv, float eps_lo,
    float eps_hi, float inv_n, float *__restrict__ lp_out, float *__restrict__ s_out, float *__restrict__ pg_out,
    float *__restrict__ dlogits, int64_t T, int V) {
  __shared__ float scratch[GS_THREADS / 64];
  __shared__ float coef_sh;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int stride = WAVE_PER_TOKEN ? GS_THREADS / 64 : GS_THREADS;
  const int first = WAVE_PER_TOKEN ? wid : tid;
  const bool ratio = old_lp != nullptr && adv != nullptr && n_bases != nullptr;

  // pass 1: lp and the masked sum of (lp - old)
  float part = 0.f;
  for (int64_t t = first; t < T; t += stride) {
    const int64_t row = b * T + t;
    int64_t y = targets[row];
    y = (y < 0 || y >= V) ? 0 : y;
    float mx, lse;
    if (WAVE_PER_TOKEN)
      lse_wave<BF16>(logits, row * V, V, lane, mx, lse);
    else
      lse_thread<BF16>(logits, row * V, V, mx, lse);
    const float lp = logit_at<BF16>(logits, row * V + y) - lse;
    if (!WAVE_PER_TOKEN || lane == 0) {
      lp_out[row] = lp;
      if (ratio && mask[row]) part += lp - old_lp[row];
    }
  }
  if (!ratio) return;
  const float tot = block_sum(part, scratch);
  if (tid == 0) {
    const float nb = n_bases[b];
    const float A = adv[b];
    const float s = expf(tot / nb);
    const float lo = 1.0f - eps_lo, hi = 1.0f + eps_hi;
    const float sc = fminf(fmaxf(s, lo), hi);
    const float a1 = s * A, a2 = sc * A;
    s_out[b] = s;
    pg_out[b] = -fminf(a1, a2);
    // d min(a1, a2) / ds: a1 branch slope A, a2 branch slope A * [lo <= s <= hi]; ties split evenly
    const float d2 = (s >= lo && s <= hi) ? A : 0.f;
    float dmin;
    if (a1 < a2)
      dmin = A;
    else if (a2 < a1)
      dmin = d2;
    else
      dmin = 0.5f * (A + d2);
    const float g = -dmin;
    coef_sh = inv_n * g * s / nb;
  }
  if (dlogits == nullptr) return;
  __syncthreads();
  const float coef = coef_sh;

  // pass 2: dL/dz = coef * mask * (onehot - softmax)
  for (int64_t t = first; t < T; t += stride) {
    const int64_t row = b * T + t;
    const float c = mask[row] ? coef : 0.f;
    int64_t y = targets[row];
    y = (y < 0 || y >= V) ? 0 : y;
    float mx, lse;
    if (WAVE_PER_TOKEN) {
      lse_wave<BF16>(logits, row * V, V, lane, mx, lse);
      for (int v = lane; v < V; v += 64) {
        const float sm = expf(logit_at<BF16>(logits, row * V + v) - lse);
        dlogits[row * V + v] = c * ((v == y ? 1.f : 0.f) - sm);
      }
    } else {
      lse_thread<BF16>(logits, row * V, V, mx, lse);
      for (int v = 0; v < V; ++v) {
        const float sm = expf(logit_at<BF16>(logits, row * V + v) - lse);
        dlogits[row * V + v] = c * ((v == y ? 1.f : 0.f) - sm);
      }
    }
  }
}

// loss = inv_n * sum_b pg[b], one workgroup, fixed order
__global__ __launch_bounds__(GS_THREADS) void gspo_loss_kernel(const float *__restrict__ pg, int64_t B, float inv_n,
                                                               float *__restrict__ loss) {
  __shared__ float scratch[GS_THREADS / 64];
  float part = 0.f;
  for (int64_t b = threadIdx.x; b < B; b += GS_THREADS) part += pg[b];
  const float tot = block_sum(part, scratch);
  if (threadIdx.x == 0) loss[0] = tot * inv_n;
}

__global__ void group_advantage_kernel(const float *__restrict__ reward, int64_t groups, int n, int mode, float param,
                                       float *__restrict__ adv, uint8_t *__restrict__ live) {
  const int64_t gi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const float *r = reward + gi * n;
  float mean = 0.f;
  for (int i = 0; i < n; ++i) mean += r[i];
  mean /= static_cast<float>(n);
  float var = 0.f;
  for (int i = 0; i < n; ++i) var += (r[i] - mean) * (r[i] - mean);
  const float sd = sqrtf(var / static_cast<float>(n));
  const float den = mode == 0 ? fmaxf(sd, param) : sd + param;
  for (int i = 0; i < n; ++i) adv[gi * n + i] = (r[i] - mean) / den;
  if (live) live[gi] = sd > 1e-6f ? 1 : 0;
}

}  // namespace vk

using namespace vk;

extern "C" int vk_gspo_score(const void *logits, int32_t logits_dtype, const int64_t *targets, const uint8_t *mask,
                             const float *old_lp, const float *n_bases, const float *adv, float eps_lo, float eps_hi,
                             float inv_n, float *lp, float *s, float *pg, float *loss, float *dlogits, int64_t B,
                             int64_t T, int32_t V, void *stream) {
  VK_CHECK_ARG(logits && targets && lp, "gspo_score: null pointer");
  VK_CHECK_ARG(logits_dtype == VK_DTYPE_BF16 || logits_dtype == VK_DTYPE_F32, "gspo_score: bad logits dtype");
  VK_CHECK_ARG(B >= 0 && B < (int64_t(1) << 31) && T >= 0 && V > 0, "gspo_score: bad sizes");
  const bool ratio = old_lp != nullptr || adv != nullptr;
  VK_CHECK_ARG(!ratio || (old_lp && adv && n_bases && mask && s && pg && loss),
               "gspo_score: the ratio / loss needs mask, old_lp, n_bases, adv, s, pg and loss");
  VK_CHECK_ARG(dlogits == nullptr || ratio, "gspo_score: dlogits needs the ratio inputs");
  if (B == 0 || T == 0) return VK_OK;
  hipStream_t st = VK_STREAM(stream);
  const bool wave = V > 32;
  const dim3 grid(static_cast<unsigned>(B));
#define VK_GSPO_LAUNCH(BF, WV)                                                                                    \
  gspo_score_kernel<BF, WV><<<grid, GS_THREADS, 0, st>>>(logits, targets, mask, ratio ? old_lp : nullptr, n_bases, \
                                                         ratio ? adv : nullptr, eps_lo, eps_hi, inv_n, lp, s, pg,   \
                                                         dlogits, T, V)
  if (logits_dtype == VK_DTYPE_BF16) {
    if (wave)
      VK_GSPO_LAUNCH(true, true);
    else
      VK_GSPO_LAUNCH(true, false);
  } else {
    if (wave)
      VK_GSPO_LAUNCH(false, true);
    else
      VK_GSPO_LAUNCH(false, false);
  }
#undef VK_GSPO_LAUNCH
  int rc = launch_status("gspo_score");
  if (rc != VK_OK || !ratio) return rc;
  gspo_loss_kernel<<<1, GS_THREADS, 0, st>>>(pg, B, inv_n, loss);
  return launch_status("gspo_loss");
}

extern "C" int vk_group_advantage(const float *reward, int64_t groups, int32_t n, int32_t mode, float param, float *adv,
                                  uint8_t *live, void *stream) {
  VK_CHECK_ARG(reward && adv && groups >= 0 && n > 0, "group_advantage: bad arguments");
  VK_CHECK_ARG(mode == 0 || mode == 1, "group_advantage: mode must be 0 (std floor) or 1 (std + eps)");
  if (groups == 0) return VK_OK;
  group_advantage_kernel<<<static_cast<unsigned>((groups + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
      reward, groups, n, mode, param, adv, live);
  return launch_status("group_advantage");
}
