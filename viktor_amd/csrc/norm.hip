// Row-wise kernels of the packed token layout [n, d]: fused residual add + RMSNorm and the
// embedding lookup + first RMSNorm of a decode step. One wavefront per row, 16-byte accesses.
//
// Rounding follows the reference's fused path (viktor/triton_ops.py:17-40, 149-169): the residual
// sum is stored in bf16 and the norm is taken over that stored value; the normalised output is
// (x * rsqrt(mean(x^2) + eps)) * w in fp32, rounded once to bf16. The teacher-forced scoring forward runs
// under torch.autocast over fp32 master weights (scripts/gspo.py:345-347): its residual stream and norm
// weights are fp32, and rmsnorm_f32_kernel / the fp32 forms of rmsnorm_apply_ss_kernel normalise them with
// one rounding, to the bf16 operand of the next product.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace vk {

// Thread-local message of the last failure, returned by vk_last_error().
static thread_local char g_msg[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(VK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return VK_OK;
}

// CH = number of 8-element chunks each lane owns (d <= 512 * CH). Every load (row, delta, weight) is
// issued before the reduction, unconditionally (chunk indices clamped, surplus chunks masked), so a row
// costs one memory round trip.
template <int CH, bool EMBED>
__global__ __launch_bounds__(256) void rmsnorm_rows(bf16_t *__restrict__ x, const bf16_t *__restrict__ delta,
                                                    const int64_t *__restrict__ tok, const bf16_t *__restrict__ emb,
                                                    int64_t vocab, const bf16_t *__restrict__ w,
                                                    bf16_t *__restrict__ h, int64_t n, int d, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= n) return;
  const int nch = d >> 3;
  const bf16_t *src = x + row * d;
  bool zero_row = false;
  if (EMBED) {
    const int64_t t = tok[row];
    zero_row = t < 0 || t >= vocab;
    src = emb + (zero_row ? 0 : t) * d;
  }
  u32x4 a[CH], b[CH], wv[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    int ci = lane + c * kWave;
    ci = ci < nch ? ci : nch - 1;
    a[c] = *reinterpret_cast<const u32x4 *>(src + ci * 8);
    if (!EMBED && delta != nullptr) b[c] = *reinterpret_cast<const u32x4 *>(delta + row * d + ci * 8);
    wv[c] = *reinterpret_cast<const u32x4 *>(w + ci * 8);
  }
  float v[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ci = lane + c * kWave;
    if (EMBED && zero_row) a[c] = u32x4{0u, 0u, 0u, 0u};
    if (!EMBED && delta != nullptr) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a[c][j] = pack_bf(lo_bf(a[c][j]) + lo_bf(b[c][j]), hi_bf(a[c][j]) + hi_bf(b[c][j]));
    }
    if ((EMBED || delta != nullptr) && ci < nch) *reinterpret_cast<u32x4 *>(x + row * d + ci * 8) = a[c];
    const float keep = ci < nch ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[c][2 * j] = lo_bf(a[c][j]);
      v[c][2 * j + 1] = hi_bf(a[c][j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += keep * (v[c][j] * v[c][j]);
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ci = lane + c * kWave;
    if (ci < nch) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf(v[c][2 * j] * r * lo_bf(wv[c][j]), v[c][2 * j + 1] * r * hi_bf(wv[c][j]));
      *reinterpret_cast<u32x4 *>(h + row * d + ci * 8) = o;
    }
  }
}

template <bool EMBED>
static int launch_rows(bf16_t *x, const bf16_t *delta, const int64_t *tok, const bf16_t *emb, int64_t vocab,
                       const bf16_t *w, bf16_t *h, int64_t n, int d, float eps, hipStream_t s, const char *name) {
  if (n == 0) return VK_OK;
  const int rows_per_block = 4;
  const dim3 grid(static_cast<unsigned>((n + rows_per_block - 1) / rows_per_block));
  const int ch = (d / 8 + kWave - 1) / kWave;
  if (ch <= 1)
    rmsnorm_rows<1, EMBED><<<grid, 256, 0, s>>>(x, delta, tok, emb, vocab, w, h, n, d, eps);
  else if (ch <= 2)
    rmsnorm_rows<2, EMBED><<<grid, 256, 0, s>>>(x, delta, tok, emb, vocab, w, h, n, d, eps);
  else
    rmsnorm_rows<4, EMBED><<<grid, 256, 0, s>>>(x, delta, tok, emb, vocab, w, h, n, d, eps);
  return launch_status(name);
}

__device__ __forceinline__ u32x4 norm8(const float (&x)[8], float r, const float (&w)[8]) {
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = pack_bf(x[2 * k] * r * w[2 * k], x[2 * k + 1] * r * w[2 * k + 1]);
  return o;
}

// h = bf16(x * rsqrt(sum(ss[row]) / d + eps) * w) with the row's sum of squares handed over in nb block partials
// (ss [n, nb] fp32, summed in block order); 8 columns per lane. x is the bf16 residual stream of the inference path
// or the fp32 one of the autocast forward (XT), w bf16 or fp32 (WT); h bf16 may be x when XT is bf16 (each lane
// rewrites the chunk it read).
// d = 512 (one 8-column chunk per lane per row): a wavefront takes RN_ROWS rows and issues all their loads before
// the first use, so 4 KB per wavefront are in flight rather than one row's 1 KB (the kernel streams 2 x n x 1 KB
// and, with one row per wavefront, was bound by the loads in flight at about 4.3 TB/s). Other d: one row per
// wavefront.
constexpr int RN_ROWS = 4;
template <typename XT, typename WT>
__global__ __launch_bounds__(256) void rmsnorm_apply_ss_kernel(const XT *x, const float *__restrict__ ss, int nb,
                                                               const WT *__restrict__ w, bf16_t *h, int64_t n,
                                                               int d, float eps, bool vec_ss) {
  const int lane = threadIdx.x & 63;
  if (d == 512) {
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RN_ROWS;
    if (row0 >= n) return;
    Raw8<XT> xv[RN_ROWS];
#pragma unroll
    for (int i = 0; i < RN_ROWS; ++i) {
      const int64_t row = row0 + i < n ? row0 + i : n - 1;
      xv[i].load(x + row * 512 + lane * 8);
    }
    Raw8<WT> wr;
    wr.load(w + lane * 8);
    float r[RN_ROWS];
    if (vec_ss) {  // nb % 4 == 0, nb <= 16, ss 16-byte aligned: the partials as 16-byte loads, all issued before the
                   // sums (block order kept)
      f32x4 sv[RN_ROWS][4];
#pragma unroll
      for (int i = 0; i < RN_ROWS; ++i) {
        const int64_t row = row0 + i < n ? row0 + i : n - 1;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (4 * q < nb) sv[i][q] = *reinterpret_cast<const f32x4 *>(ss + row * nb + 4 * q);
      }
#pragma unroll
      for (int i = 0; i < RN_ROWS; ++i) {
        float tot = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (4 * q < nb) tot = (((tot + sv[i][q][0]) + sv[i][q][1]) + sv[i][q][2]) + sv[i][q][3];
        r[i] = rsqrtf(tot / static_cast<float>(d) + eps);
      }
    } else {
#pragma unroll
      for (int i = 0; i < RN_ROWS; ++i) {
        const int64_t row = row0 + i < n ? row0 + i : n - 1;
        float tot = 0.f;
        for (int b = 0; b < nb; ++b) tot += ss[row * nb + b];
        r[i] = rsqrtf(tot / static_cast<float>(d) + eps);
      }
    }
    float wv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) wv[k] = wr.get(k);
#pragma unroll
    for (int i = 0; i < RN_ROWS; ++i) {
      if (row0 + i >= n) break;
      float xf[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) xf[k] = xv[i].get(k);
      *reinterpret_cast<u32x4 *>(h + (row0 + i) * 512 + lane * 8) = norm8(xf, r[i], wv);
    }
    return;
  }
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  float tot = 0.f;
  for (int b = 0; b < nb; ++b) tot += ss[row * nb + b];
  const float r = rsqrtf(tot / static_cast<float>(d) + eps);
  for (int c = lane * 8; c < d; c += 64 * 8) {
    Raw8<XT> xr;
    Raw8<WT> wr;
    xr.load(x + row * d + c);
    wr.load(w + c);
    float xf[8], wv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xf[k] = xr.get(k);
      wv[k] = wr.get(k);
    }
    *reinterpret_cast<u32x4 *>(h + row * d + c) = norm8(xf, r, wv);
  }
}

// The RMSNorm of an fp32 residual stream with fp32 weights, rounded once to bf16: nn.RMSNorm (fp32 input and
// weight, computed in fp32) followed by the bf16 cast torch.autocast applies at the next product's input
// (viktor/decoder.py:118-119, 144 under autocast). One wavefront per row, every chunk's loads issued before the sum.
template <int CH>
__global__ __launch_bounds__(256) void rmsnorm_f32_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                          bf16_t *__restrict__ h, int64_t n, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const int nch = d >> 3;
  Raw8<float> xr[CH], wr[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    int ci = lane + c * 64;
    ci = ci < nch ? ci : nch - 1;
    xr[c].load(x + row * d + ci * 8);
    wr[c].load(w + ci * 8);
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const float keep = lane + c * 64 < nch ? 1.f : 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += keep * (xr[c].get(k) * xr[c].get(k));
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ci = lane + c * 64;
    if (ci >= nch) continue;
    float xf[8], wv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xf[k] = xr[c].get(k);
      wv[k] = wr[c].get(k);
    }
    *reinterpret_cast<u32x4 *>(h + row * d + ci * 8) = norm8(xf, r, wv);
  }
}

// Whether every member of every group of G equal-size members equals the group's first member, bit for bit:
// a thread per 16-byte chunk of a group's first member, which it loads once and compares with the same chunk
// of members 1..G-1 (every byte of the group read once); a difference stores 1 to *flag (every writer stores
// the same value).
__global__ __launch_bounds__(256) void group_rows_equal_kernel(const u32x4 *__restrict__ x, int64_t groups, int G,
                                                               int64_t chunks_per_member, int32_t *__restrict__ flag) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= groups * chunks_per_member) return;
  const int64_t grp = i / chunks_per_member, c = i - grp * chunks_per_member;
  const u32x4 *g0 = x + grp * G * chunks_per_member + c;
  const u32x4 a = g0[0];
  uint32_t diff = 0;
  for (int m = 1; m < G; ++m) {
    const u32x4 b = g0[static_cast<int64_t>(m) * chunks_per_member];
    diff |= (a[0] ^ b[0]) | (a[1] ^ b[1]) | (a[2] ^ b[2]) | (a[3] ^ b[3]);
  }
  if (diff != 0) *flag = 1;
}

}  // namespace vk

using namespace vk;

extern "C" int vk_group_rows_equal(const void *x, int64_t groups, int32_t G, int64_t member_bytes, int32_t *flag,
                                   void *stream) {
  VK_CHECK_ARG(x && flag, "group_rows_equal: null pointer");
  VK_CHECK_ARG(groups >= 0 && G >= 1 && member_bytes >= 0 && member_bytes % 16 == 0 && vk_aligned16(x),
               "group_rows_equal: need 16-byte aligned members of a multiple of 16 bytes");
  const int64_t total = G > 1 ? groups * (member_bytes / 16) : 0;
  if (total == 0) return VK_OK;
  group_rows_equal_kernel<<<static_cast<unsigned>((total + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
      static_cast<const u32x4 *>(x), groups, G, member_bytes / 16, flag);
  return launch_status("group_rows_equal");
}

extern "C" int vk_rmsnorm_apply_ss(const void *x, int32_t x_dtype, const float *ss, int32_t nb, const void *w,
                                   int32_t w_dtype, void *h, int64_t n, int32_t d, float eps, void *stream) {
  VK_CHECK_ARG(x && ss && w && h, "rmsnorm_apply_ss: null pointer");
  VK_CHECK_ARG(n >= 0 && d > 0 && d % 8 == 0 && nb > 0, "rmsnorm_apply_ss: bad sizes (d=%d nb=%d)", d, nb);
  VK_CHECK_ARG((x_dtype == VK_DTYPE_BF16 || x_dtype == VK_DTYPE_F32) && (w_dtype == VK_DTYPE_BF16 || w_dtype == VK_DTYPE_F32),
               "rmsnorm_apply_ss: bad dtypes");
  VK_CHECK_ARG(x_dtype == VK_DTYPE_BF16 || x != h, "rmsnorm_apply_ss: an fp32 x cannot be overwritten by h");
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(h), "rmsnorm_apply_ss: pointers must be 16-byte aligned");
  if (n == 0) return VK_OK;
  const int64_t waves = d == 512 ? (n + RN_ROWS - 1) / RN_ROWS : n;
  const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
  const bool vec = nb % 4 == 0 && nb <= 16 && vk_aligned16(ss);
  hipStream_t s = VK_STREAM(stream);
  auto hb = static_cast<bf16_t *>(h);
  if (x_dtype == VK_DTYPE_BF16) {
    const auto xb = static_cast<const bf16_t *>(x);
    if (w_dtype == VK_DTYPE_BF16)
      rmsnorm_apply_ss_kernel<bf16_t, bf16_t><<<grid, 256, 0, s>>>(xb, ss, nb, static_cast<const bf16_t *>(w), hb, n, d, eps, vec);
    else
      rmsnorm_apply_ss_kernel<bf16_t, float><<<grid, 256, 0, s>>>(xb, ss, nb, static_cast<const float *>(w), hb, n, d, eps, vec);
  } else {
    const auto xf = static_cast<const float *>(x);
    if (w_dtype == VK_DTYPE_BF16)
      rmsnorm_apply_ss_kernel<float, bf16_t><<<grid, 256, 0, s>>>(xf, ss, nb, static_cast<const bf16_t *>(w), hb, n, d, eps, vec);
    else
      rmsnorm_apply_ss_kernel<float, float><<<grid, 256, 0, s>>>(xf, ss, nb, static_cast<const float *>(w), hb, n, d, eps, vec);
  }
  return launch_status("rmsnorm_apply_ss");
}

extern "C" int vk_rmsnorm_f32(const float *x, const float *w, void *h, int64_t n, int32_t d, float eps, void *stream) {
  VK_CHECK_ARG(x && w && h, "rmsnorm_f32: null pointer");
  VK_CHECK_ARG(n >= 0 && d > 0 && d % 8 == 0 && d <= 2048, "rmsnorm_f32: need 0 < d <= 2048, d %% 8 == 0 (d=%d)", d);
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(h), "rmsnorm_f32: pointers must be 16-byte aligned");
  if (n == 0) return VK_OK;
  const dim3 grid(static_cast<unsigned>((n + 3) / 4));
  hipStream_t s = VK_STREAM(stream);
  auto hb = static_cast<bf16_t *>(h);
  const int ch = (d / 8 + 63) / 64;
  if (ch <= 1)
    rmsnorm_f32_kernel<1><<<grid, 256, 0, s>>>(x, w, hb, n, d, eps);
  else if (ch <= 2)
    rmsnorm_f32_kernel<2><<<grid, 256, 0, s>>>(x, w, hb, n, d, eps);
  else
    rmsnorm_f32_kernel<4><<<grid, 256, 0, s>>>(x, w, hb, n, d, eps);
  return launch_status("rmsnorm_f32");
}

extern "C" int vk_version(void) { return 100; }

extern "C" const char *vk_last_error(void) { return vk::g_msg; }

extern "C" int vk_device_cus(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

extern "C" int vk_add_rmsnorm(void *x, const void *delta, const void *w, void *h, int64_t n, int32_t d, float eps,
                              void *stream) {
  VK_CHECK_ARG(x && w && h, "add_rmsnorm: null pointer");
  VK_CHECK_ARG(n >= 0 && d > 0 && d % 8 == 0 && d <= 2048, "add_rmsnorm: need 0 < d <= 2048, d %% 8 == 0 (d=%d)", d);
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(h) && (!delta || vk_aligned16(delta)),
               "add_rmsnorm: pointers must be 16-byte aligned");
  return launch_rows<false>(static_cast<bf16_t *>(x), static_cast<const bf16_t *>(delta), nullptr, nullptr, 0,
                            static_cast<const bf16_t *>(w), static_cast<bf16_t *>(h), n, d, eps, VK_STREAM(stream),
                            "add_rmsnorm");
}

extern "C" int vk_embed_rmsnorm(const int64_t *tok, const void *emb, int64_t vocab, const void *w, void *x, void *h,
                                int64_t n, int32_t d, float eps, void *stream) {
  VK_CHECK_ARG(tok && emb && w && x && h, "embed_rmsnorm: null pointer");
  VK_CHECK_ARG(n >= 0 && d > 0 && d % 8 == 0 && d <= 2048 && vocab > 0, "embed_rmsnorm: bad sizes (d=%d)", d);
  VK_CHECK_ARG(vk_aligned16(emb) && vk_aligned16(w) && vk_aligned16(x) && vk_aligned16(h),
               "embed_rmsnorm: pointers must be 16-byte aligned");
  return launch_rows<true>(static_cast<bf16_t *>(x), nullptr, tok, static_cast<const bf16_t *>(emb), vocab,
                           static_cast<const bf16_t *>(w), static_cast<bf16_t *>(h), n, d, eps, VK_STREAM(stream),
                           "embed_rmsnorm");
}
