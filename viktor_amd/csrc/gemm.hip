// y[M, N] = x[M, K] @ w[N, K]^T on gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
// Both operands are K-contiguous (activations [M, K] row-major, PyTorch Linear weights [N, K]), which
// is the operand order the MFMA wants: every lane's A and B fragment is 8 consecutive K values, one
// 16-byte read. A workgroup of 4 wavefronts (2 x 2) owns a BM x BN output tile; K advances in BK
// slices staged through LDS (double buffered: the next slice's global loads are in flight while the
// current slice feeds the MFMAs), rows padded by 16 bytes against bank conflicts.
//
// Epilogues: bf16 or fp32 store; SwiGLU (w = [gate; up] of 2N rows): the tile loads the matching gate
// and up rows, and stores bf16(bf16(silu(bf16(g))) * bf16(u)) -- the rounding points of an unfused
// bf16 linear followed by viktor/triton_ops.py:212-229 (and of the fused epilogue at :132-134).
#include "common.h"

namespace vk {

template <int BM, int BN, int BK, bool SWIGLU, bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const bf16_t *__restrict__ x, const bf16_t *__restrict__ w,
                                                        void *__restrict__ y, int64_t M, int N, int K) {
  constexpr int NB = SWIGLU ? 2 * BN : BN;  // rows of w staged per tile
  constexpr int PITCH = BK + 8;             // bf16 elements per LDS row (16-byte pad)
  constexpr int WM = BM / 2, WN = BN / 2;   // per-wave tile
  constexpr int TM = WM / 16, TN = WN / 16; // MFMA tiles per wave
  constexpr int CPR = BK / 8;               // 16-byte chunks per row of a K slice
  constexpr int A_CHUNKS = BM * CPR / 256;  // per thread
  constexpr int B_CHUNKS = NB * CPR / 256;
  static_assert(BM * CPR % 256 == 0 && NB * CPR % 256 == 0, "tile / thread mismatch");

  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][NB * PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int wm = wid >> 1, wn = wid & 1;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int n0 = blockIdx.x * BN;

  // global source rows of this thread's chunks (clamped in range: rows past M / N load valid memory
  // whose results are never stored)
  const bf16_t *a_src[A_CHUNKS];
  int a_dst[A_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = tid + 256 * i;
    const int r = c / CPR, k8 = c % CPR;
    int64_t gr = m0 + r;
    gr = gr < M ? gr : M - 1;
    a_src[i] = x + gr * K + k8 * 8;
    a_dst[i] = r * PITCH + k8 * 8;
  }
  const bf16_t *b_src[B_CHUNKS];
  int b_dst[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = tid + 256 * i;
    const int r = c / CPR, k8 = c % CPR;
    int gr;
    if (SWIGLU) {
      const int col = n0 + (r < BN ? r : r - BN);
      gr = (col < N ? col : N - 1) + (r < BN ? 0 : N);
    } else {
      gr = n0 + r;
      gr = gr < N ? gr : N - 1;
    }
    b_src[i] = w + static_cast<int64_t>(gr) * K + k8 * 8;
    b_dst[i] = r * PITCH + k8 * 8;
  }

  u32x4 ra[A_CHUNKS], rb[B_CHUNKS];
  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(a_src[i] + k0);
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) rb[i] = *reinterpret_cast<const u32x4 *>(b_src[i] + k0);
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) *reinterpret_cast<u32x4 *>(&As[buf][a_dst[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) *reinterpret_cast<u32x4 *>(&Bs[buf][b_dst[i]]) = rb[i];
  };

  f32x4 acc[TM][TN];
  f32x4 acc2[SWIGLU ? TM : 1][SWIGLU ? TN : 1];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (SWIGLU) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc2[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int frag_row = lane & 15;       // row of A / column of B this lane feeds
  const int frag_k = (lane >> 4) * 8;   // first of its 8 K values
  const int nk = K / BK;

  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_global((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8 *>(&As[buf][(wm * WM + i * 16 + frag_row) * PITCH + ks * 32 + frag_k]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][(wn * WN + j * 16 + frag_row) * PITCH + ks * 32 + frag_k]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      if (SWIGLU) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8 *>(
              &Bs[buf][(BN + wn * WN + j * 16 + frag_row) * PITCH + ks * 32 + frag_k]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc2[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc2[i][j], 0, 0, 0);
      }
    }
    if (kt + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds rows 4*(lane/16) + r (r = 0..3), column lane % 16 of each 16 x 16 tile
  const int out_col = lane & 15;
  const int out_row = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WN + j * 16 + out_col;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm * WM + i * 16 + out_row + r;
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (SWIGLU) {
          const float g = round_bf(v);
          const float u = round_bf(acc2[i][j][r]);
          const float act = round_bf(g / (1.0f + __expf(-g)));
          v = act * u;
        }
        if (OUT_F32)
          static_cast<float *>(y)[row * N + col] = v;
        else
          static_cast<bf16_t *>(y)[row * N + col] = f2bf(v);
      }
    }
  }
}

template <int BM, int BN, int BK, bool SWIGLU, bool OUT_F32>
static void launch_gemm(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, hipStream_t s) {
  const dim3 grid((N + BN - 1) / BN, static_cast<unsigned>((M + BM - 1) / BM));
  gemm_bf16_kernel<BM, BN, BK, SWIGLU, OUT_F32><<<grid, 256, 0, s>>>(x, w, y, M, N, K);
}

template <int BK>
static void dispatch_gemm(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, bool swiglu,
                          bool out_f32, hipStream_t s) {
  const bool big = M >= 4096;
  if (swiglu) {
    if (big)
      launch_gemm<128, 64, BK, true, false>(x, w, y, M, N, K, s);
    else
      launch_gemm<64, 32, BK, true, false>(x, w, y, M, N, K, s);
  } else if (out_f32) {
    if (big)
      launch_gemm<128, 128, BK, false, true>(x, w, y, M, N, K, s);
    else
      launch_gemm<64, 64, BK, false, true>(x, w, y, M, N, K, s);
  } else {
    if (big)
      launch_gemm<128, 128, BK, false, false>(x, w, y, M, N, K, s);
    else
      launch_gemm<64, 64, BK, false, false>(x, w, y, M, N, K, s);
  }
}

int gemm_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, bool swiglu, bool out_f32,
             hipStream_t s);
int gemm_big_swiglu_keep(const bf16_t *x, const bf16_t *w, void *y, bf16_t *gu, int64_t M, int N, int K,
                         hipStream_t s);

}  // namespace vk

using namespace vk;

extern "C" int vk_linear(const void *x, const void *w, void *y, int64_t M, int32_t N, int32_t K, int32_t swiglu,
                         int32_t out_dtype, void *gu_out, void *stream) {
  VK_CHECK_ARG(x && w && y, "linear: null pointer");
  VK_CHECK_ARG(gu_out == nullptr || swiglu, "linear: gu_out goes with the SwiGLU epilogue");
  VK_CHECK_ARG(M >= 0 && N > 0 && K > 0 && K % 32 == 0, "linear: need K %% 32 == 0 (M=%lld N=%d K=%d)",
               static_cast<long long>(M), N, K);
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w), "linear: x and w must be 16-byte aligned");
  VK_CHECK_ARG(out_dtype == VK_DTYPE_BF16 || out_dtype == VK_DTYPE_F32, "linear: bad out dtype");
  VK_CHECK_ARG(!(swiglu && out_dtype == VK_DTYPE_F32), "linear: the SwiGLU epilogue stores bf16");
  VK_CHECK_ARG(M < (int64_t(1) << 31) / 128 * 128, "linear: M too large");
  if (M == 0) return VK_OK;
  const auto xs = static_cast<const bf16_t *>(x);
  const auto ws = static_cast<const bf16_t *>(w);
  // large M: the direct-to-LDS pipeline of gemm_big (SwiGLU included: 778 against 626 TFLOP/s for the 128 x 64
  // tile kernel below at M = 131072)
  if (M >= 4096 && K % 64 == 0 && N % 8 == 0 && vk_aligned16(y) && (gu_out == nullptr || vk_aligned16(gu_out))) {
    const int rc = gu_out != nullptr
                       ? gemm_big_swiglu_keep(xs, ws, y, static_cast<bf16_t *>(gu_out), M, N, K, VK_STREAM(stream))
                       : gemm_big(xs, ws, y, M, N, K, swiglu != 0, out_dtype == VK_DTYPE_F32, VK_STREAM(stream));
    if (rc != VK_OK) return rc;
    return launch_status("linear");
  }
  if (gu_out != nullptr) {  // smaller M: the gate | up rows from the plain product, then the SwiGLU product
    if (K % 64 == 0)
      dispatch_gemm<64>(xs, ws, gu_out, M, 2 * N, K, false, false, VK_STREAM(stream));
    else
      dispatch_gemm<32>(xs, ws, gu_out, M, 2 * N, K, false, false, VK_STREAM(stream));
  }
  if (K % 64 == 0)
    dispatch_gemm<64>(xs, ws, y, M, N, K, swiglu != 0, out_dtype == VK_DTYPE_F32, VK_STREAM(stream));
  else
    dispatch_gemm<32>(xs, ws, y, M, N, K, swiglu != 0, out_dtype == VK_DTYPE_F32, VK_STREAM(stream));
  return launch_status("linear");
}

// ---- standalone SwiGLU over [n, 2F] (prefill path of the reference; fused into vk_linear here) ----
__global__ __launch_bounds__(256) void swiglu_kernel(const bf16_t *__restrict__ gu, bf16_t *__restrict__ out,
                                                     int64_t total, int F) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t row = i / F;
  const int col = static_cast<int>(i - row * F);
  const float g = bf2f(gu[row * 2 * F + col]);
  const float u = bf2f(gu[row * 2 * F + F + col]);
  const float act = round_bf(g / (1.0f + __expf(-g)));
  out[i] = f2bf(act * u);
}

// 8 columns per thread (16-byte loads of gate and up, one 16-byte store) when F % 8 == 0
__global__ __launch_bounds__(256) void swiglu8_kernel(const bf16_t *__restrict__ gu, bf16_t *__restrict__ out,
                                                      int64_t total8, int F8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total8) return;
  const int64_t row = i / F8;
  const int c8 = static_cast<int>(i - row * F8);
  const u32x4 g = *reinterpret_cast<const u32x4 *>(gu + (row * 2 * F8 + c8) * 8);
  const u32x4 u = *reinterpret_cast<const u32x4 *>(gu + (row * 2 * F8 + F8 + c8) * 8);
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float g0 = lo_bf(g[w]), g1 = hi_bf(g[w]);
    const float a0 = round_bf(g0 / (1.0f + __expf(-g0))), a1 = round_bf(g1 / (1.0f + __expf(-g1)));
    o[w] = pack_bf(a0 * lo_bf(u[w]), a1 * hi_bf(u[w]));
  }
  *reinterpret_cast<u32x4 *>(out + i * 8) = o;
}

extern "C" int vk_swiglu(const void *gu, void *out, int64_t n, int32_t f, void *stream) {
  VK_CHECK_ARG(gu && out && n >= 0 && f > 0, "swiglu: bad arguments");
  const int64_t total = n * f;
  if (total == 0) return VK_OK;
  if (f % 8 == 0 && vk_aligned16(gu) && vk_aligned16(out)) {
    const int64_t total8 = total / 8;
    swiglu8_kernel<<<static_cast<unsigned>((total8 + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
        static_cast<const bf16_t *>(gu), static_cast<bf16_t *>(out), total8, f / 8);
    return launch_status("swiglu");
  }
  swiglu_kernel<<<static_cast<unsigned>((total + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
      static_cast<const bf16_t *>(gu), static_cast<bf16_t *>(out), total, f);
  return launch_status("swiglu");
}
