// Backward passes of the decoder's element-wise stages and the optimizer step of the GSPO update
// (scripts/gspo.py:477-493: loss.backward() through Basecaller.logits, clip_grad_norm_, AdamW(fused) step).
//
//   * rmsnorm_bwd_kernel: y = x r w with r = (mean x^2 + eps)^-1/2 over d = 512 (nn.RMSNorm,
//     viktor/decoder.py:110-124): dx = r (w dy) - x r^3 mean(w dy x) (+ the residual's incoming gradient),
//     dw = sum_rows dy x r (per-workgroup partial rows, reduced by colsum_kernel). One wavefront per row.
//   * qknorm_rope_bwd_kernel: the per-head QK-norm (d = 64) followed by the half-split RoPE rotation
//     (viktor/decoder.py:62-66, viktor/encoder.py:36-40): the rotation is undone on the gradient
//     (dy1 = c do1 + s do2, dy2 = -s do1 + c do2), then the 64-wide norm backward; v heads pass through.
//     Writes the qkv-projection output gradient [n, 768] in bf16 (the operand of its weight / input GEMMs).
//   * swiglu_bwd_kernel: silu(g) u (viktor/decoder.py:127): dg = do u s (1 + g (1 - s)), du = do g s.
//   * sumsq_kernel + clip_coef_kernel: the global gradient norm and min(1, max_norm / (norm + 1e-6)) of
//     clip_grad_norm_, kept on the device.
//   * adamw_kernel: torch's AdamW update with the clip coefficient applied to the gradient:
//     m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g^2, p = p (1 - lr wd) - lr / bc1 * m / (sqrt(v) / sqrt(bc2) + eps).
// All math in fp32; every reduction runs in a fixed order (deterministic).
#include <math.h>

#include <type_traits>

#include "common.h"

namespace vk {

constexpr int TR_D = 512;  // d_model of the norm kernels

template <typename T>
__device__ __forceinline__ float ld(const T *p, int64_t i);
template <>
__device__ __forceinline__ float ld<float>(const float *p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<bf16_t>(const bf16_t *p, int64_t i) { return bf2f(p[i]); }

// one wavefront per row; lane l owns columns 8 l .. 8 l + 7. Workgroup = 4 waves; the grid strides over rows.
// dw_part [gridDim.x, 512]: this workgroup's sum over its rows of dy x r.
// x, w: bf16 (the inference-precision residual stream) or fp32 (the autocast forward's fp32 stream and master
// norm weights); dy bf16 or fp32.
template <typename XT, typename WT, typename DT>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const XT *__restrict__ x, const WT *__restrict__ w,
                                                         const DT *__restrict__ dy, const float *__restrict__ dres,
                                                         float *__restrict__ dx, bf16_t *__restrict__ dx_bf,
                                                         float *__restrict__ dw_part, int64_t n, float eps) {
  __shared__ float red[4][TR_D];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float wv[8], dwa[8];
  {
    Raw8<WT> wr;
    wr.load(w + 8 * lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[e] = wr.get(e);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) dwa[j] = 0.f;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wid; row < n; row += static_cast<int64_t>(gridDim.x) * 4) {
    Raw8<XT> xr;
    Raw8<DT> gr;
    xr.load(x + row * TR_D + 8 * lane);
    gr.load(dy + row * TR_D + 8 * lane);
    float xv[8], gv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xv[e] = xr.get(e);
      gv[e] = gr.get(e);
    }
    f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
    if (dres) {
      d0 = *reinterpret_cast<const f32x4 *>(dres + row * TR_D + 8 * lane);
      d1 = *reinterpret_cast<const f32x4 *>(dres + row * TR_D + 8 * lane + 4);
    }
    float ss = 0.f, dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss += xv[j] * xv[j];
      dot += gv[j] * wv[j] * xv[j];
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    const float r = rsqrtf(ss * (1.0f / TR_D) + eps);
    const float c = r * r * r * dot * (1.0f / TR_D);
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[j] = r * gv[j] * wv[j] - xv[j] * c;
      if (dres) o[j] += j < 4 ? d0[j] : d1[j - 4];
      dwa[j] += gv[j] * xv[j] * r;
    }
    float *dst = dx + row * TR_D + 8 * lane;
    *reinterpret_cast<f32x4 *>(dst) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4 *>(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
    if (dx_bf)  // the bf16 copy the next products take (round to nearest even, as a tensor cast)
      *reinterpret_cast<u32x4 *>(dx_bf + row * TR_D + 8 * lane) =
          u32x4{pack_bf(o[0], o[1]), pack_bf(o[2], o[3]), pack_bf(o[4], o[5]), pack_bf(o[6], o[7])};
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) red[wid][8 * lane + j] = dwa[j];
  __syncthreads();
  for (int c = threadIdx.x; c < TR_D; c += 256)
    dw_part[static_cast<int64_t>(blockIdx.x) * TR_D + c] = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
}

// sum over the rows of part [rows, cols], out[c] = sum (+ out[c] when accumulate). Workgroup = 16 columns x
// 16 row slices (slice s: rows s, s + 16, ...), then the 16 slice sums added in a fixed order: a short
// dependency chain per thread and cols / 16 workgroups.
__global__ __launch_bounds__(256) void colsum_kernel(const float *__restrict__ part, float *__restrict__ out, int rows,
                                                    int cols, int accumulate) {
  __shared__ float red[16][16];
  const int ci = threadIdx.x & 15, sl = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + ci;
  float s = 0.f;
  if (c < cols)
    for (int r = sl; r < rows; r += 16) s += part[static_cast<int64_t>(r) * cols + c];
  red[sl][ci] = s;
  __syncthreads();
  if (sl == 0 && c < cols) {
    float t = red[0][ci];
#pragma unroll
    for (int k = 1; k < 16; ++k) t += red[k][ci];
    out[c] = accumulate ? out[c] + t : t;
  }
}

// The (row, head) items of qkv [n, (H + 2 HKV) 64] bf16 (the forward's projection output), flattened as
// row (H + 2 HKV) + head: q heads 0..H-1 and k heads get the norm + RoPE backward from dq / dk [n, H|HKV, 64] fp32,
// v heads pass dv through (rounded to bf16). cos/sin [S, 32] fp32 (or bf16) at row position rpos.
// Eight lanes per item: lane j of a group owns dims 8 j .. 8 j + 7 (16-byte loads and stores; it loads its
// rotation partners, dims d ^ 32, itself), so a wavefront takes 8 items at a time and a head's two sums over 64
// dims are 8 lane partials and three lane swaps inside the group. Every lane runs the same code for every kind
// of head (no divergent branches around the swaps); the kind selects the gradient source and the result.
// dw_part [gridDim.x, 128]: this workgroup's q-norm weight gradient (0..63) and k-norm (64..127), summed over
// its items in a fixed order (a lane's items in sequence, the wavefront's 8 groups by lane swaps, the 4
// wavefronts in order).
// HT / HKVT > 0: the head counts as compile-time constants (the decoder's 8 / 2); 0: the run-time H / HKV.
// WT: the norm weights' type (bf16, or the fp32 master weights of the autocast forward).
template <typename TT, typename WT, int HT, int HKVT>
__global__ __launch_bounds__(256) void qknorm_rope_bwd_kernel(
    const bf16_t *__restrict__ qkv, const WT *__restrict__ qw, const WT *__restrict__ kw,
    const TT *__restrict__ cos_t, const TT *__restrict__ sin_t, int64_t table_rows, const int32_t *__restrict__ rpos,
    const float *__restrict__ dq, const float *__restrict__ dk, const float *__restrict__ dv,
    bf16_t *__restrict__ dqkv, float *__restrict__ dw_part, int64_t n, int H_rt, int HKV_rt, float eps) {
  const int H = HT > 0 ? HT : H_rt, HKV = HKVT > 0 ? HKVT : HKV_rt;
  const int NH = H + 2 * HKV;
  __shared__ float red[4][128];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int j = lane & 7, slot = lane >> 3;
  const int d0 = 8 * j, dp = d0 ^ 32, fi = d0 & 31;  // own dims, partner dims, rotary frequency index
  const float rsign = d0 < 32 ? 1.f : -1.f;          // dy1 = c do1 + s do2, dy2 = c do2 - s do1
  using TV = typename std::remove_cv<TT>::type;
  using WV = typename std::remove_cv<WT>::type;
  float wq[8], wk[8], dwq[8], dwk[8];
  {
    Raw8<WV> a, b;
    a.load(qw + d0);
    b.load(kw + d0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      wq[e] = a.get(e);
      wk[e] = b.get(e);
      dwq[e] = dwk[e] = 0.f;
    }
  }
  const int64_t total = n * NH;
  // a wavefront's items of one pass: 8 at t0 + u step (u < QB_U), loaded together before any is computed, so a
  // pass keeps QB_U items' loads (and their dependent rotary-table loads) in flight per lane
  constexpr int QB_U = 4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * 32;  // items per sweep of the grid (4 waves x 8)
  for (int64_t t0 = (static_cast<int64_t>(blockIdx.x) * 4 + wid) * 8; t0 < total; t0 += QB_U * step) {
    bool live[QB_U], isq[QB_U], isk[QB_U];
    int64_t obase[QB_U];
    Raw8<float> go[QB_U], gp[QB_U];
    Raw8<bf16_t> xr[QB_U];
    int64_t p[QB_U];
#pragma unroll
    for (int u = 0; u < QB_U; ++u) {
      live[u] = t0 + u * step + slot < total;
      const int64_t t = live[u] ? t0 + u * step + slot : total - 1;
      const int64_t row = t / NH;
      const int h = static_cast<int>(t - row * NH);
      isq[u] = h < H;
      isk[u] = !isq[u] && h < H + HKV;
      const float *g = isq[u] ? dq + (row * H + h) * 64
                              : (isk[u] ? dk + (row * HKV + (h - H)) * 64 : dv + (row * HKV + (h - H - HKV)) * 64);
      go[u].load(g + d0);
      gp[u].load(g + dp);
      obase[u] = row * NH * 64 + h * 64 + d0;
      xr[u].load(qkv + obase[u]);
      p[u] = rpos[row];
    }
    Raw8<TV> cr[QB_U], sr[QB_U];
#pragma unroll
    for (int u = 0; u < QB_U; ++u) {
      const int64_t pc = p[u] < 0 ? 0 : (p[u] >= table_rows ? table_rows - 1 : p[u]);
      cr[u].load(cos_t + pc * 32 + fi);
      sr[u].load(sin_t + pc * 32 + fi);
    }
#pragma unroll
    for (int u = 0; u < QB_U; ++u) {
      float gy[8], xv[8], ss = 0.f, dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gy[e] = cr[u].get(e) * go[u].get(e) + rsign * (sr[u].get(e) * gp[u].get(e));
        xv[e] = xr[u].get(e);
        ss += xv[e] * xv[e];
        dot += gy[e] * (isq[u] ? wq[e] : wk[e]) * xv[e];
      }
      ss = group_sum<8>(ss);
      dot = group_sum<8>(dot);
      const float r = rsqrtf(ss * (1.0f / 64) + eps);
      const float c3 = r * r * r * dot * (1.0f / 64);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dx = r * gy[e] * (isq[u] ? wq[e] : wk[e]) - xv[e] * c3;
        o[e] = (isq[u] || isk[u]) ? dx : go[u].get(e);
        const float gw = live[u] ? gy[e] * xv[e] * r : 0.f;
        dwq[e] += isq[u] ? gw : 0.f;
        dwk[e] += isk[u] ? gw : 0.f;
      }
      if (live[u])
        *reinterpret_cast<u32x4 *>(dqkv + obase[u]) =
            u32x4{pack_bf(o[0], o[1]), pack_bf(o[2], o[3]), pack_bf(o[4], o[5]), pack_bf(o[6], o[7])};
    }
  }
  // the 8 groups of the wavefront (lanes j, j + 8, ..., j + 56 own the same dims), then the 4 wavefronts
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
      dwq[e] += __shfl_xor(dwq[e], off, 64);
      dwk[e] += __shfl_xor(dwk[e], off, 64);
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      red[wid][d0 + e] = dwq[e];
      red[wid][64 + d0 + e] = dwk[e];
    }
  }
  __syncthreads();
  if (threadIdx.x < 128)
    dw_part[static_cast<int64_t>(blockIdx.x) * 128 + threadIdx.x] =
        (red[0][threadIdx.x] + red[1][threadIdx.x]) + (red[2][threadIdx.x] + red[3][threadIdx.x]);
}

// gu [n, 2F] (gate | up, bf16), dout [n, F] (bf16) -> dgu [n, 2F] bf16; 8 columns per thread
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const bf16_t *__restrict__ gu, const bf16_t *__restrict__ dout,
                                                        bf16_t *__restrict__ dgu, int64_t n, int F) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (row, 8-column group)
  const int groups = F / 8;
  if (i >= n * groups) return;
  const int64_t row = i / groups;
  const int c0 = static_cast<int>(i - row * groups) * 8;
  const u32x4 gr = *reinterpret_cast<const u32x4 *>(gu + row * 2 * F + c0);
  const u32x4 ur = *reinterpret_cast<const u32x4 *>(gu + row * 2 * F + F + c0);
  const u32x4 dr = *reinterpret_cast<const u32x4 *>(dout + row * F + c0);
  u32x4 dg, du;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float o[2][2];
#pragma unroll
    for (int hlf = 0; hlf < 2; ++hlf) {
      const float g = hlf ? hi_bf(gr[e]) : lo_bf(gr[e]);
      const float u = hlf ? hi_bf(ur[e]) : lo_bf(ur[e]);
      const float d = hlf ? hi_bf(dr[e]) : lo_bf(dr[e]);
      const float sg = 1.0f / (1.0f + __expf(-g));
      o[0][hlf] = d * u * sg * (1.0f + g * (1.0f - sg));
      o[1][hlf] = d * g * sg;
    }
    dg[e] = pack_bf(o[0][0], o[0][1]);
    du[e] = pack_bf(o[1][0], o[1][1]);
  }
  *reinterpret_cast<u32x4 *>(dgu + row * 2 * F + c0) = dg;
  *reinterpret_cast<u32x4 *>(dgu + row * 2 * F + F + c0) = du;
}

// per-workgroup partial sums of squares of x [n] (grid-stride, fixed order)
__global__ __launch_bounds__(256) void sumsq_kernel(const float *__restrict__ x, int64_t n, float *__restrict__ part) {
  __shared__ float red[4];
  float s = 0.f;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    s += x[i] * x[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// norm_out[0] = sqrt(sum of the parts), norm_out[1] = min(1, max_norm / (norm + 1e-6)) (clip_grad_norm_)
__global__ __launch_bounds__(64) void clip_coef_kernel(const float *__restrict__ part, int nparts, float max_norm,
                                                       float *__restrict__ norm_out) {
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 64) s += part[i];
  s = wave_sum(s);
  if (threadIdx.x == 0) {
    const float nrm = sqrtf(s);
    norm_out[0] = nrm;
    norm_out[1] = fminf(1.0f, max_norm / (nrm + 1e-6f));
  }
}

__global__ __launch_bounds__(256) void adamw_kernel(float *__restrict__ p, const float *__restrict__ g,
                                                   float *__restrict__ m, float *__restrict__ v, int64_t n,
                                                   const float *__restrict__ coef, float lr, float b1, float b2,
                                                   float eps, float wd, float bc1, float bc2_sqrt) {
  const float cs = coef ? coef[1] : 1.0f;
  const float step = lr / bc1;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    const float gi = g[i] * cs;
    const float mi = b1 * m[i] + (1.0f - b1) * gi;
    const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    float pi = p[i] * (1.0f - lr * wd);
    pi -= step * mi / (sqrtf(vi) / bc2_sqrt + eps);
    p[i] = pi;
  }
}

static unsigned row_grid(int64_t n) {
  const int64_t cus = device_cus_cached();
  int64_t b = (n + 3) / 4;
  return static_cast<unsigned>(b < 2 * cus ? (b > 0 ? b : 1) : 2 * cus);
}

}  // namespace vk

using namespace vk;

extern "C" int vk_rmsnorm_backward_blocks(int64_t n, int32_t *blocks) {
  VK_CHECK_ARG(blocks && n >= 0, "rmsnorm_backward_blocks: bad arguments");
  *blocks = static_cast<int32_t>(row_grid(n));
  return VK_OK;
}

extern "C" int vk_rmsnorm_backward(const void *x, int32_t x_dtype, const void *w, int32_t w_dtype, const void *dy,
                                   int32_t dy_dtype, const float *dres, float *dx, void *dx_bf16, float *dw_part,
                                   int64_t n, int32_t d, float eps, void *stream) {
  VK_CHECK_ARG(x && w && dy && dx && dw_part, "rmsnorm_backward: null pointer");
  if (d != TR_D) return fail(VK_ERR_UNSUPPORTED, "rmsnorm_backward: built for d = %d (got %d)", TR_D, d);
  VK_CHECK_ARG(n >= 0 && (dy_dtype == VK_DTYPE_BF16 || dy_dtype == VK_DTYPE_F32), "rmsnorm_backward: bad arguments");
  VK_CHECK_ARG((x_dtype == VK_DTYPE_BF16 || x_dtype == VK_DTYPE_F32) && (w_dtype == VK_DTYPE_BF16 || w_dtype == VK_DTYPE_F32),
               "rmsnorm_backward: bad dtypes");
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(dx) && vk_aligned16(dy) &&
                   (!dres || vk_aligned16(dres)) && (!dx_bf16 || vk_aligned16(dx_bf16)),
               "rmsnorm_backward: alignment");
  bf16_t *const dxb = static_cast<bf16_t *>(dx_bf16);
  if (n == 0) return VK_OK;
  const unsigned grid = row_grid(n);
  hipStream_t s = VK_STREAM(stream);
  // the inference-precision combination (bf16 x and w) and the autocast one (fp32 x and w), each with either dy
  if (x_dtype == VK_DTYPE_BF16 && w_dtype == VK_DTYPE_BF16) {
    const auto xb = static_cast<const bf16_t *>(x);
    const auto wb = static_cast<const bf16_t *>(w);
    if (dy_dtype == VK_DTYPE_F32)
      rmsnorm_bwd_kernel<bf16_t, bf16_t, float><<<grid, 256, 0, s>>>(xb, wb, static_cast<const float *>(dy), dres, dx, dxb, dw_part, n, eps);
    else
      rmsnorm_bwd_kernel<bf16_t, bf16_t, bf16_t><<<grid, 256, 0, s>>>(xb, wb, static_cast<const bf16_t *>(dy), dres, dx, dxb, dw_part, n, eps);
  } else if (x_dtype == VK_DTYPE_F32 && w_dtype == VK_DTYPE_F32) {
    const auto xf = static_cast<const float *>(x);
    const auto wf = static_cast<const float *>(w);
    if (dy_dtype == VK_DTYPE_F32)
      rmsnorm_bwd_kernel<float, float, float><<<grid, 256, 0, s>>>(xf, wf, static_cast<const float *>(dy), dres, dx, dxb, dw_part, n, eps);
    else
      rmsnorm_bwd_kernel<float, float, bf16_t><<<grid, 256, 0, s>>>(xf, wf, static_cast<const bf16_t *>(dy), dres, dx, dxb, dw_part, n, eps);
  } else {
    return fail(VK_ERR_UNSUPPORTED, "rmsnorm_backward: x and w are both bf16 or both fp32");
  }
  return launch_status("rmsnorm_backward");
}

extern "C" int vk_colsum(const float *part, float *out, int32_t rows, int32_t cols, int32_t accumulate, void *stream) {
  VK_CHECK_ARG(part && out && rows >= 0 && cols >= 0, "colsum: bad arguments");
  if (cols == 0) return VK_OK;
  colsum_kernel<<<static_cast<unsigned>((cols + 15) / 16), 256, 0, VK_STREAM(stream)>>>(part, out, rows, cols,
                                                                                      accumulate);
  return launch_status("colsum");
}

extern "C" int vk_qknorm_rope_backward(const void *qkv, const void *q_norm_w, const void *k_norm_w, int32_t norm_w_dtype,
                                       const void *cos_t, const void *sin_t, int32_t table_dtype, int64_t table_rows,
                                       const int32_t *rope_pos, const float *dq, const float *dk, const float *dv,
                                       void *dqkv, float *dw_part, int64_t n, int32_t H, int32_t HKV, int32_t D,
                                       float eps, void *stream) {
  VK_CHECK_ARG(qkv && q_norm_w && k_norm_w && cos_t && sin_t && rope_pos && dq && dk && dv && dqkv && dw_part,
               "qknorm_rope_backward: null pointer");
  if (D != 64) return fail(VK_ERR_UNSUPPORTED, "qknorm_rope_backward: built for head_dim 64 (got %d)", D);
  VK_CHECK_ARG(n >= 0 && H > 0 && HKV > 0 && table_rows > 0 &&
                   (table_dtype == VK_DTYPE_F32 || table_dtype == VK_DTYPE_BF16) &&
                   (norm_w_dtype == VK_DTYPE_F32 || norm_w_dtype == VK_DTYPE_BF16),
               "qknorm_rope_backward: bad arguments");
  VK_CHECK_ARG(vk_aligned16(qkv) && vk_aligned16(q_norm_w) && vk_aligned16(k_norm_w) && vk_aligned16(cos_t) &&
                   vk_aligned16(sin_t) && vk_aligned16(dq) && vk_aligned16(dk) && vk_aligned16(dv) && vk_aligned16(dqkv),
               "qknorm_rope_backward: pointers must be 16-byte aligned");
  if (n == 0) return VK_OK;
  const unsigned grid = row_grid(n);
  hipStream_t s = VK_STREAM(stream);
  const auto qb = static_cast<const bf16_t *>(qkv);
  auto out = static_cast<bf16_t *>(dqkv);
  const bool fixed = H == 8 && HKV == 2;
  // table and weight types, then the head counts as constants (8 / 2) or at run time
  auto run = [&](auto ct, auto wt) {
    using TT = typename std::remove_pointer<decltype(ct)>::type;
    using WT = typename std::remove_pointer<decltype(wt)>::type;
    const auto c = static_cast<const TT *>(cos_t), sn = static_cast<const TT *>(sin_t);
    const auto qw = static_cast<const WT *>(q_norm_w), kw = static_cast<const WT *>(k_norm_w);
    if (fixed)
      qknorm_rope_bwd_kernel<TT, WT, 8, 2><<<grid, 256, 0, s>>>(qb, qw, kw, c, sn, table_rows, rope_pos, dq, dk, dv,
                                                                out, dw_part, n, H, HKV, eps);
    else
      qknorm_rope_bwd_kernel<TT, WT, 0, 0><<<grid, 256, 0, s>>>(qb, qw, kw, c, sn, table_rows, rope_pos, dq, dk, dv,
                                                                out, dw_part, n, H, HKV, eps);
  };
  const float *f = nullptr;
  const bf16_t *b = nullptr;
  if (table_dtype == VK_DTYPE_F32) {
    if (norm_w_dtype == VK_DTYPE_F32)
      run(f, f);
    else
      run(f, b);
  } else {
    if (norm_w_dtype == VK_DTYPE_F32)
      run(b, f);
    else
      run(b, b);
  }
  return launch_status("qknorm_rope_backward");
}

extern "C" int vk_swiglu_backward(const void *gu, const void *dout, void *dgu, int64_t n, int32_t F, void *stream) {
  VK_CHECK_ARG(gu && dout && dgu && n >= 0 && F > 0 && F % 8 == 0, "swiglu_backward: bad arguments");
  VK_CHECK_ARG(vk_aligned16(gu) && vk_aligned16(dout) && vk_aligned16(dgu), "swiglu_backward: alignment");
  if (n == 0) return VK_OK;
  const int64_t work = n * (F / 8);
  swiglu_bwd_kernel<<<static_cast<unsigned>((work + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
      static_cast<const bf16_t *>(gu), static_cast<const bf16_t *>(dout), static_cast<bf16_t *>(dgu), n, F);
  return launch_status("swiglu_backward");
}

extern "C" int vk_grad_norm_clip(const float *g, int64_t n, float max_norm, float *partials, int32_t n_partials,
                                 float *norm_out, void *stream) {
  VK_CHECK_ARG(g && partials && norm_out && n >= 0 && n_partials > 0 && max_norm > 0.f, "grad_norm_clip: bad arguments");
  hipStream_t s = VK_STREAM(stream);
  sumsq_kernel<<<static_cast<unsigned>(n_partials), 256, 0, s>>>(g, n, partials);
  int rc = launch_status("grad_norm_clip sumsq");
  if (rc != VK_OK) return rc;
  clip_coef_kernel<<<1, 64, 0, s>>>(partials, n_partials, max_norm, norm_out);
  return launch_status("grad_norm_clip coef");
}

extern "C" int vk_adamw(float *p, const float *g, float *m, float *v, int64_t n, const float *coef, float lr, float b1,
                        float b2, float eps, float wd, int64_t step, void *stream) {
  VK_CHECK_ARG(p && g && m && v && n >= 0 && step >= 1, "adamw: bad arguments");
  if (n == 0) return VK_OK;
  const float bc1 = static_cast<float>(1.0 - pow(static_cast<double>(b1), static_cast<double>(step)));
  const float bc2 = static_cast<float>(1.0 - pow(static_cast<double>(b2), static_cast<double>(step)));
  const int64_t cus = device_cus_cached();
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8 * cus) blocks = 8 * cus;
  adamw_kernel<<<static_cast<unsigned>(blocks), 256, 0, VK_STREAM(stream)>>>(p, g, m, v, n, coef, lr, b1, b2, eps, wd,
                                                                           bc1, sqrtf(bc2));
  return launch_status("adamw");
}
