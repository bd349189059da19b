// The GSPO update's kernels at the two ends of the decoder stack (scripts/gspo.py:477 differentiating
// Basecaller.logits, viktor/model.py:55-60, 72-86):
//
//   * bias_act_kernel: the epilogue of the per-frame projector's linears (viktor/model.py:35, nn.Linear ->
//     nn.GELU() -> nn.Linear under torch.autocast bf16): pre = bf16(y + b) over an fp32 product y, and for the
//     first linear out = bf16(gelu(pre)) with the exact erf GELU, 0.5 x (1 + erf(x / sqrt 2)).
//   * act_bwd_kernel: the projector's backward rows: din = bf16(dout gelu'(pre)) with
//     gelu'(x) = Phi(x) + x phi(x), and per-workgroup column sums of the bias gradient (of din, or of dout
//     itself for the second linear's bias); vk_colsum sums the partials in a fixed order.
//   * embed_grad_kernel + embed_reduce_kernel: the token-embedding table's gradient (nn.Embedding backward,
//     viktor/decoder.py:127 gathered at viktor/model.py:77): out[v, c] = sum of d_rows[r, c] over rows r with
//     tokens[r] = v, in fp32. Rows are split into slices; a wavefront owns 8 columns per lane of a 512-column
//     block and a chunk of <= 32 token ids, and keeps that chunk's sums in LDS, each lane touching only its own
//     columns (no atomics, no races); the slices' partials are then summed in a fixed order -- deterministic.
// All of these are HBM-bound row sweeps (a few bytes per element): 16-byte loads and stores, fp32 math.
#include <math.h>

#include "common.h"

namespace vk {

__device__ __forceinline__ float gelu_f(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }
// d gelu / dx = Phi(x) + x phi(x), Phi the normal CDF and phi its density
__device__ __forceinline__ float gelu_grad_f(float x) {
  const float cdf = 0.5f * (1.f + erff(x * 0.70710678118654752f));
  return cdf + x * (0.39894228040143268f * expf(-0.5f * x * x));
}

// 8 consecutive columns per thread over [n, d] (d % 8 == 0)
__global__ __launch_bounds__(256) void bias_act_kernel(const float *__restrict__ y, const float *__restrict__ bias,
                                                       bf16_t *__restrict__ pre, bf16_t *__restrict__ out,
                                                       int64_t total8, int d8, int gelu) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total8) return;
  const int c8 = static_cast<int>(i % d8);
  const f32x4 y0 = *reinterpret_cast<const f32x4 *>(y + 8 * i), y1 = *reinterpret_cast<const f32x4 *>(y + 8 * i + 4);
  const f32x4 b0 = *reinterpret_cast<const f32x4 *>(bias + 8 * c8), b1 = *reinterpret_cast<const f32x4 *>(bias + 8 * c8 + 4);
  float z[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    z[e] = round_bf(y0[e] + b0[e]);
    z[4 + e] = round_bf(y1[e] + b1[e]);
  }
  if (!gelu) {
    *reinterpret_cast<u32x4 *>(out + 8 * i) =
        u32x4{pack_bf(z[0], z[1]), pack_bf(z[2], z[3]), pack_bf(z[4], z[5]), pack_bf(z[6], z[7])};
    return;
  }
  *reinterpret_cast<u32x4 *>(pre + 8 * i) =
      u32x4{pack_bf(z[0], z[1]), pack_bf(z[2], z[3]), pack_bf(z[4], z[5]), pack_bf(z[6], z[7])};
  float a[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = gelu_f(z[e]);
  *reinterpret_cast<u32x4 *>(out + 8 * i) =
      u32x4{pack_bf(a[0], a[1]), pack_bf(a[2], a[3]), pack_bf(a[4], a[5]), pack_bf(a[6], a[7])};
}

// Workgroup of 256 threads: rpi = 256 / d8 row lanes x d8 column groups (d8 = d / 8 <= 256; threads past
// rpi d8 idle); the grid strides over rows. GELU: din = bf16(dout gelu'(pre)) and the column sums are of din; otherwise the column sums of dout.
// part [gridDim.x, d]: this workgroup's sums, rows in a fixed order.
template <bool GELU>
__global__ __launch_bounds__(256) void act_bwd_kernel(const bf16_t *__restrict__ pre, const bf16_t *__restrict__ dout,
                                                      bf16_t *__restrict__ din, float *__restrict__ part, int64_t n,
                                                      int d8) {
  extern __shared__ float red[];  // [rpi][d]
  const int rpi = 256 / d8, c8 = threadIdx.x % d8, rl = threadIdx.x / d8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int64_t r_first = rl < rpi ? static_cast<int64_t>(blockIdx.x) * rpi + rl : n;
  for (int64_t r = r_first; r < n; r += static_cast<int64_t>(gridDim.x) * rpi) {
    const int64_t o = r * d8 * 8 + 8 * c8;
    const u32x4 g = *reinterpret_cast<const u32x4 *>(dout + o);
    float v[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      v[2 * w] = lo_bf(g[w]);
      v[2 * w + 1] = hi_bf(g[w]);
    }
    if (GELU) {
      const u32x4 p = *reinterpret_cast<const u32x4 *>(pre + o);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        v[2 * w] = round_bf(v[2 * w] * gelu_grad_f(lo_bf(p[w])));
        v[2 * w + 1] = round_bf(v[2 * w + 1] * gelu_grad_f(hi_bf(p[w])));
      }
      *reinterpret_cast<u32x4 *>(din + o) =
          u32x4{pack_bf(v[0], v[1]), pack_bf(v[2], v[3]), pack_bf(v[4], v[5]), pack_bf(v[6], v[7])};
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
  }
  const int d = 8 * d8;
  if (rl < rpi)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[rl * d + 8 * c8 + e] = acc[e];
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += 256) {
    float s = 0.f;
    for (int q = 0; q < rpi; ++q) s += red[q * d + c];
    part[static_cast<int64_t>(blockIdx.x) * d + c] = s;
  }
}

constexpr int EG_VC = 32;     // token ids per workgroup chunk
constexpr int EG_COLS = 512;  // columns per workgroup: 8 per lane
constexpr int EG_UNROLL = 8;  // rows whose loads are in flight together

// grid (slices, vocab chunks, column blocks), one wavefront; bins: min(V, 32) x 512 fp32 of dynamic LDS.
// part [slices, V, d]: slice s's sums of its rows. d_rows bf16 (the inference-precision residual's gradient) or
// fp32 (the autocast forward's fp32 residual gradient: the embedding rows enter it unrounded). A token id is tested
// against this workgroup's vocabulary chunk as an int64, before it is narrowed.
template <typename DT>
__global__ __launch_bounds__(64) void embed_grad_kernel(const DT *__restrict__ drows, int64_t ld,
                                                        const int64_t *__restrict__ tokens, int64_t n, int V, int d,
                                                        float *__restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) float bins[];
  const int lane = threadIdx.x;
  const int slices = gridDim.x, sl = blockIdx.x;
  const int v0 = blockIdx.y * EG_VC, vc = min(EG_VC, V - v0);
  const int c0 = blockIdx.z * EG_COLS + 8 * lane;
  const bool live = c0 < d;
  for (int i = lane; i < vc * EG_COLS; i += 64) bins[i] = 0.f;
  __syncthreads();
  const int64_t r0 = n * sl / slices, r1 = n * (sl + 1) / slices;
  for (int64_t r = r0; r < r1; r += EG_UNROLL) {
    int t[EG_UNROLL];
    Raw8<DT> x[EG_UNROLL];
#pragma unroll
    for (int u = 0; u < EG_UNROLL; ++u) {
      const bool in = r + u < r1;
      const int64_t rel = in ? tokens[r + u] - v0 : -1;
      t[u] = (rel >= 0 && rel < vc) ? static_cast<int>(rel) : -1;
      if (live && t[u] >= 0)
        x[u].load(drows + (r + u) * ld + c0);
      else
        x[u].zero();
    }
#pragma unroll
    for (int u = 0; u < EG_UNROLL; ++u) {
      if (t[u] < 0) continue;  // wave-uniform: every lane reads the same token
      float *b = bins + t[u] * EG_COLS + 8 * lane;
      f32x4 lo = *reinterpret_cast<f32x4 *>(b), hi = *reinterpret_cast<f32x4 *>(b + 4);
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = x[u].get(e);
      lo += f32x4{v[0], v[1], v[2], v[3]};
      hi += f32x4{v[4], v[5], v[6], v[7]};
      *reinterpret_cast<f32x4 *>(b) = lo;
      *reinterpret_cast<f32x4 *>(b + 4) = hi;
    }
  }
  if (!live) return;
  for (int v = 0; v < vc; ++v) {
    float *dst = part + (static_cast<int64_t>(sl) * V + v0 + v) * d + c0;
    const float *b = bins + v * EG_COLS + 8 * lane;
    *reinterpret_cast<f32x4 *>(dst) = *reinterpret_cast<const f32x4 *>(b);
    *reinterpret_cast<f32x4 *>(dst + 4) = *reinterpret_cast<const f32x4 *>(b + 4);
  }
}

// out[i] = sum over slices of part[s, i] (i over V x d, vd % 4 == 0) in a fixed order: thread (g, q) of a
// workgroup sums slices g, g + 16, g + 32, ... of elements i0 + 4 q .. + 3 (i0 = 64 blockIdx.x), then the 16
// group sums are added in g order.
__global__ __launch_bounds__(256) void embed_reduce_kernel(const float *__restrict__ part, int slices, int64_t vd,
                                                           float *__restrict__ out) {
  __shared__ f32x4 red[16][16];
  const int g = threadIdx.x >> 4, q = threadIdx.x & 15;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 64 + 4 * q;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (i < vd)
    for (int s = g; s < slices; s += 16) acc += *reinterpret_cast<const f32x4 *>(part + static_cast<int64_t>(s) * vd + i);
  red[g][q] = acc;
  __syncthreads();
  if (g == 0 && i < vd) {
    f32x4 t = red[0][q];
    for (int k = 1; k < 16; ++k) t += red[k][q];
    *reinterpret_cast<f32x4 *>(out + i) = t;
  }
}

static int embed_slices(int64_t n, int V, int d) {
  const int64_t chunks = static_cast<int64_t>((V + EG_VC - 1) / EG_VC) * ((d + EG_COLS - 1) / EG_COLS);
  int64_t s = (n + 63) / 64;                             // >= 64 rows a slice
  const int64_t cap = 8 * device_cus_cached() / chunks;  // about 8 wavefronts per CU in all
  if (s > cap) s = cap;
  if (s > (int64_t(64) << 20) / (static_cast<int64_t>(V) * d * 4)) s = (int64_t(64) << 20) / (static_cast<int64_t>(V) * d * 4);
  return static_cast<int>(s < 1 ? 1 : s);  // partials stay under 64 MB
}

}  // namespace vk

using namespace vk;

extern "C" int vk_bias_act(const float *y, const float *bias, void *pre, void *out, int64_t n, int32_t d, int32_t gelu,
                           void *stream) {
  VK_CHECK_ARG(bias && (n == 0 || (y && out && (!gelu || pre))), "bias_act: null pointer");
  VK_CHECK_ARG(n >= 0 && d > 0 && d % 8 == 0, "bias_act: need d %% 8 == 0 (got %d)", d);
  VK_CHECK_ARG(vk_aligned16(y) && vk_aligned16(bias) && vk_aligned16(out) && (!gelu || vk_aligned16(pre)),
               "bias_act: 16-byte aligned tensors");
  const int64_t total8 = n * d / 8;
  if (total8 == 0) return VK_OK;
  bias_act_kernel<<<static_cast<unsigned>((total8 + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
      y, bias, static_cast<bf16_t *>(pre), static_cast<bf16_t *>(out), total8, d / 8, gelu != 0);
  return launch_status("bias_act");
}

extern "C" int vk_act_backward_blocks(int64_t n, int32_t d, int32_t *blocks) {
  VK_CHECK_ARG(blocks && n >= 0 && d > 0 && d % 8 == 0 && d <= 2048, "act_backward_blocks: bad arguments");
  const int64_t rpi = 256 / (d / 8), need = (n + rpi - 1) / rpi, cap = 2 * device_cus_cached();
  *blocks = static_cast<int32_t>(need < 1 ? 1 : (need < cap ? need : cap));
  return VK_OK;
}

extern "C" int vk_act_backward(const void *pre, const void *dout, void *din, float *part, int32_t blocks, int64_t n,
                               int32_t d, int32_t gelu, void *stream) {
  VK_CHECK_ARG(part && (n == 0 || (dout && (!gelu || (pre && din)))), "act_backward: null pointer");
  VK_CHECK_ARG(n >= 0 && d > 0 && d % 8 == 0 && d <= 2048 && blocks > 0,
               "act_backward: need d %% 8 == 0 and d <= 2048 (got %d)", d);
  VK_CHECK_ARG(vk_aligned16(dout) && (!gelu || (vk_aligned16(pre) && vk_aligned16(din))),
               "act_backward: 16-byte aligned tensors");
  const int d8 = d / 8;
  const size_t lds = static_cast<size_t>(256 / d8) * d * sizeof(float);  // <= 8 KB
  hipStream_t s = VK_STREAM(stream);
  if (gelu)
    act_bwd_kernel<true><<<static_cast<unsigned>(blocks), 256, lds, s>>>(
        static_cast<const bf16_t *>(pre), static_cast<const bf16_t *>(dout), static_cast<bf16_t *>(din), part, n, d8);
  else
    act_bwd_kernel<false><<<static_cast<unsigned>(blocks), 256, lds, s>>>(
        nullptr, static_cast<const bf16_t *>(dout), nullptr, part, n, d8);
  return launch_status("act_backward");
}

extern "C" int vk_embed_grad_workspace(int64_t n, int32_t V, int32_t d, int64_t *bytes) {
  VK_CHECK_ARG(bytes && n >= 0 && V > 0 && d > 0, "embed_grad_workspace: bad arguments");
  *bytes = static_cast<int64_t>(embed_slices(n, V, d)) * V * d * static_cast<int64_t>(sizeof(float));
  return VK_OK;
}

extern "C" int vk_embed_grad(const void *d_rows, int32_t d_dtype, int64_t ld, const int64_t *tokens, int64_t n, int32_t V,
                             int32_t d, float *out, void *workspace, int64_t workspace_bytes, void *stream) {
  VK_CHECK_ARG(out && workspace && (n == 0 || (d_rows && tokens)), "embed_grad: null pointer");
  VK_CHECK_ARG(d_dtype == VK_DTYPE_BF16 || d_dtype == VK_DTYPE_F32, "embed_grad: bad row dtype");
  VK_CHECK_ARG(n >= 0 && V > 0 && d > 0 && d % 8 == 0 && ld >= d && ld % 8 == 0,
               "embed_grad: need d %% 8 == 0 and a row stride >= d, multiple of 8");
  VK_CHECK_ARG(vk_aligned16(d_rows) && vk_aligned16(out) && vk_aligned16(workspace), "embed_grad: alignment");
  const int slices = embed_slices(n, V, d);
  const int64_t vd = static_cast<int64_t>(V) * d;
  VK_CHECK_ARG(workspace_bytes >= slices * vd * static_cast<int64_t>(sizeof(float)),
               "embed_grad: workspace of %lld bytes needed", static_cast<long long>(slices * vd * 4));
  hipStream_t s = VK_STREAM(stream);
  float *part = static_cast<float *>(workspace);
  const dim3 grid(static_cast<unsigned>(slices), static_cast<unsigned>((V + EG_VC - 1) / EG_VC),
                  static_cast<unsigned>((d + EG_COLS - 1) / EG_COLS));
  const size_t lds = static_cast<size_t>(V < EG_VC ? V : EG_VC) * EG_COLS * sizeof(float);  // <= 64 KB
  if (d_dtype == VK_DTYPE_F32)
    embed_grad_kernel<float><<<grid, 64, lds, s>>>(static_cast<const float *>(d_rows), ld, tokens, n, V, d, part);
  else
    embed_grad_kernel<bf16_t><<<grid, 64, lds, s>>>(static_cast<const bf16_t *>(d_rows), ld, tokens, n, V, d, part);
  const int rc = launch_status("embed_grad");
  if (rc != VK_OK) return rc;
  embed_reduce_kernel<<<static_cast<unsigned>((vd + 63) / 64), 256, 0, s>>>(part, slices, vd, out);
  return launch_status("embed_grad reduce");
}
