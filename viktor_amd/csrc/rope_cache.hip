// QK-norm + RoPE + KV-cache write for packed tokens (prefill: many tokens of many sequences; decode:
// one token per sequence). One wavefront per token; each half-wave owns one head of D = 64 and each
// lane the RoPE pair (j, j + 32) of that head.
//
// Rounding follows viktor/triton_ops.py:43-91: RMSNorm over the head in fp32, the normalised value
// times the norm weight rounded to bf16, then the half-split rotation in fp32 with the cos/sin table
// entries as stored (bf16 tables when the module was cast to bf16), rounded to bf16 at the store. The norm weights
// are bf16 (the inference module) or fp32 (the fp32 master weights torch.autocast leaves in fp32 for nn.RMSNorm, which
// returns bf16(x / rms * w) for a bf16 head: the same rounding points).
#include "common.h"

namespace vk {

constexpr int kRopeD = 64;
constexpr int kHalf = kRopeD / 2;

template <bool TABLE_F32>
__device__ __forceinline__ float table_at(const void *t, int64_t i) {
  if (TABLE_F32) return static_cast<const float *>(t)[i];
  return bf2f(static_cast<const bf16_t *>(t)[i]);
}

template <bool TABLE_F32, typename WT>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(
    const bf16_t *__restrict__ qkv, const WT *__restrict__ qw, const WT *__restrict__ kw,
    const void *__restrict__ cos_t, const void *__restrict__ sin_t, int64_t table_rows,
    const int32_t *__restrict__ pos, const int32_t *__restrict__ rope_pos, const int32_t *__restrict__ seq,
    bf16_t *__restrict__ q, bf16_t *__restrict__ kc, bf16_t *__restrict__ vc, int64_t stride_cb, int64_t stride_cs,
    int64_t cache_rows, int64_t cache_len, bf16_t *__restrict__ ko, bf16_t *__restrict__ vo, int64_t n, float eps,
    int H, int HKV) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (t >= n) return;
  const int half = lane >> 5;  // which head of the pair this half-wave processes
  const int j = lane & 31;
  const int64_t p = pos[t];
  int64_t rp = rope_pos ? rope_pos[t] : p;
  rp = rp < 0 ? 0 : (rp >= table_rows ? table_rows - 1 : rp);
  const float c = table_at<TABLE_F32>(cos_t, rp * kHalf + j);
  const float s = table_at<TABLE_F32>(sin_t, rp * kHalf + j);
  const int64_t sq = seq ? seq[t] : 0;
  const bool cache_ok = kc != nullptr && sq >= 0 && sq < cache_rows && p >= 0 && p < cache_len;
  const int nh = H + 2 * HKV;
  const bf16_t *row = qkv + t * nh * kRopeD;

  // heads 0..H+HKV-1 get norm + rope; the remaining HKV (v) heads are copied.
  for (int h0 = 0; h0 < H + HKV; h0 += 2) {
    const int hd = h0 + half;
    if (hd >= H + HKV) break;
    const bool is_q = hd < H;
    const float x1 = bf2f(row[hd * kRopeD + j]);
    const float x2 = bf2f(row[hd * kRopeD + kHalf + j]);
    const float ss = group_sum<32>(x1 * x1 + x2 * x2);
    const float r = rsqrtf(ss / static_cast<float>(kRopeD) + eps);
    const WT *wn = is_q ? qw : kw;
    float w1, w2;
    if constexpr (sizeof(WT) == 4) {
      w1 = wn[j];
      w2 = wn[kHalf + j];
    } else {
      w1 = bf2f(wn[j]);
      w2 = bf2f(wn[kHalf + j]);
    }
    const float y1 = round_bf(x1 * r * w1);
    const float y2 = round_bf(x2 * r * w2);
    const bf16_t o1 = f2bf(y1 * c - y2 * s);
    const bf16_t o2 = f2bf(y1 * s + y2 * c);
    if (is_q) {
      bf16_t *qo = q + (t * H + hd) * kRopeD;
      qo[j] = o1;
      qo[kHalf + j] = o2;
    } else {
      const int hk = hd - H;
      if (cache_ok) {
        bf16_t *dst = kc + sq * stride_cb + p * stride_cs + hk * kRopeD;
        dst[j] = o1;
        dst[kHalf + j] = o2;
      }
      if (ko) {
        bf16_t *dst = ko + (t * HKV + hk) * kRopeD;
        dst[j] = o1;
        dst[kHalf + j] = o2;
      }
    }
  }
  // v heads: straight copy
  for (int hk = half; hk < HKV; hk += 2) {
    const bf16_t *src = row + (H + HKV + hk) * kRopeD;
    const bf16_t a = src[j], b = src[kHalf + j];
    if (cache_ok) {
      bf16_t *dst = vc + sq * stride_cb + p * stride_cs + hk * kRopeD;
      dst[j] = a;
      dst[kHalf + j] = b;
    }
    if (vo) {
      bf16_t *dst = vo + (t * HKV + hk) * kRopeD;
      dst[j] = a;
      dst[kHalf + j] = b;
    }
  }
}

}  // namespace vk

using namespace vk;

extern "C" int vk_qkv_rope_cache(const void *qkv, const void *q_norm_w, const void *k_norm_w, int32_t norm_w_dtype,
                                 const void *cos_t,
                                 const void *sin_t, int32_t table_dtype, int64_t table_rows, const int32_t *pos,
                                 const int32_t *rope_pos, const int32_t *seq, void *q, void *k_cache, void *v_cache,
                                 int64_t stride_cb, int64_t stride_cs, int64_t cache_rows, int64_t cache_len,
                                 void *k_out, void *v_out, int64_t n, float eps, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, void *stream) {
  VK_CHECK_ARG(qkv && q_norm_w && k_norm_w && cos_t && sin_t && pos && q, "qkv_rope_cache: null pointer");
  VK_CHECK_ARG(head_dim == kRopeD, "qkv_rope_cache: built for head_dim 64 (got %d)", head_dim);
  VK_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, "qkv_rope_cache: bad head counts");
  VK_CHECK_ARG(table_dtype == VK_DTYPE_BF16 || table_dtype == VK_DTYPE_F32, "qkv_rope_cache: bad table dtype");
  VK_CHECK_ARG(norm_w_dtype == VK_DTYPE_BF16 || norm_w_dtype == VK_DTYPE_F32, "qkv_rope_cache: bad norm weight dtype");
  VK_CHECK_ARG(table_rows > 0, "qkv_rope_cache: empty rope table");
  VK_CHECK_ARG((k_cache == nullptr) == (v_cache == nullptr), "qkv_rope_cache: k_cache and v_cache go together");
  VK_CHECK_ARG(k_cache == nullptr || seq != nullptr, "qkv_rope_cache: cache writes need seq");
  VK_CHECK_ARG((k_out == nullptr) == (v_out == nullptr), "qkv_rope_cache: k_out and v_out go together");
  if (n == 0) return VK_OK;
  const dim3 grid(static_cast<unsigned>((n + 3) / 4));
  hipStream_t s = VK_STREAM(stream);
#define VK_ROPE_LAUNCH(F32, WT)                                                                             \
  qkv_rope_cache_kernel<F32, WT><<<grid, 256, 0, s>>>(                                                     \
      static_cast<const bf16_t *>(qkv), static_cast<const WT *>(q_norm_w),                                 \
      static_cast<const WT *>(k_norm_w), cos_t, sin_t, table_rows, pos, rope_pos, seq,                     \
      static_cast<bf16_t *>(q), static_cast<bf16_t *>(k_cache), static_cast<bf16_t *>(v_cache), stride_cb, \
      stride_cs, cache_rows, cache_len, static_cast<bf16_t *>(k_out), static_cast<bf16_t *>(v_out), n, eps, \
      n_heads, n_kv_heads)
  if (norm_w_dtype == VK_DTYPE_F32) {
    if (table_dtype == VK_DTYPE_F32)
      VK_ROPE_LAUNCH(true, float);
    else
      VK_ROPE_LAUNCH(false, float);
  } else {
    if (table_dtype == VK_DTYPE_F32)
      VK_ROPE_LAUNCH(true, bf16_t);
    else
      VK_ROPE_LAUNCH(false, bf16_t);
  }
#undef VK_ROPE_LAUNCH
  return launch_status("qkv_rope_cache");
}
