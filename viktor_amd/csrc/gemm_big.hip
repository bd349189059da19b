// Large-M GEMMs of the prefill / scoring forward: y[M, N] = x[M, K] @ w[N, K]^T, bf16 in, fp32 accumulate.
//
// MI355X design (the M = tokens x N = 512..3072 x K = 512 / 1536 shapes of a packed prefill):
//   * 256 x 256 output tile per workgroup of 4 wavefronts, each wavefront 128 x 128 (64 fp32 MFMA tiles,
//     256 accumulator registers, held in AGPRs). Per 32-wide K step a wavefront reads 16 fragments
//     (16 KB) from LDS for 64 v_mfma_f32_16x16x32_bf16, half the LDS bytes per MFMA of a 64 x 64 tile.
//   * Operands reach LDS with gfx950's direct global->LDS loads (global_load_lds_dwordx4: lane l of an
//     instruction lands at LDS base + 16 l), so the prefetch costs no registers and the pipeline runs a
//     4-stage ring of 32-wide K slices (3 slices in flight while one feeds the MFMAs). LDS rows are 64 B
//     without padding; the 16-byte slot of K chunk c in row r is c ^ ((r >> 2) & 3), which makes every
//     fragment read (16 consecutive rows, one chunk) hit 16 distinct bank groups.
//   * Tiles are ordered XCD-aware: workgroup p runs on XCD p % 8, so each XCD gets a contiguous range of
//     tiles and the N-tiles that share a block of x rows share that XCD's L2.
//   * The product is formed transposed, C^T = W X^T (the weight fragment is the MFMA A operand), so each
//     lane ends with 4 consecutive output columns of one row: 8-byte stores.
//   * SwiGLU: the tile's W rows are 128 gate rows and the matching 128 up rows; both land in the same lane,
//     and the epilogue stores bf16(bf16(silu(bf16(g))) * bf16(u)) over 128 output columns.
#include "common.h"

namespace vk {

constexpr int GB_BM = 256;   // rows of x per workgroup
constexpr int GB_BW = 256;   // rows of w per workgroup
constexpr int GB_BK = 32;    // K per stage
constexpr int GB_STAGES = 4;
constexpr int GB_ROWB = GB_BK * 2;                   // bytes per LDS row
constexpr int GB_TILEB = GB_BM * GB_ROWB;            // bytes of one operand tile (16 KB)
constexpr int GB_STAGEB = 2 * GB_TILEB;              // x + w
constexpr size_t GB_SMEM = static_cast<size_t>(GB_STAGES) * GB_STAGEB;  // 128 KB

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate that waits for vmcnt <= n and leaves expcnt / lgkmcnt unconstrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt in 6:4, lgkmcnt in 11:8)
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

template <bool SWIGLU, bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_big_kernel(const bf16_t *__restrict__ x, const bf16_t *__restrict__ w,
                                                       void *__restrict__ y, int64_t M, int N, int K, int tiles_n,
                                                       int tiles_total) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  constexpr int OUT_COLS = SWIGLU ? 128 : 256;

  // XCD-aware tile order: physical workgroup p runs on XCD p % 8; XCD x owns the contiguous logical
  // range [x q + min(x, r), ...) of q + (x < r) tiles (q = total / 8, r = total % 8) -- a bijection
  const int p = blockIdx.x;
  const int xcd = p & 7, idx = p >> 3;
  const int q8 = tiles_total >> 3, r8 = tiles_total & 7;
  const int tile = xcd * q8 + min(xcd, r8) + idx;
  const int mt = tile / tiles_n, nt = tile % tiles_n;
  const int64_t m0 = static_cast<int64_t>(mt) * GB_BM;
  const int n0 = nt * OUT_COLS;

  // direct-load sources: instruction q (0..15) of an operand tile covers rows 16 q .. 16 q + 15; wave w
  // issues q = w, w + 4, w + 8, w + 12. Lane l -> row 16 q + l / 4, LDS slot l % 4, K chunk slot ^ swizzle.
  const bf16_t *xsrc[4];
  const bf16_t *wsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = wid + 4 * i;
    const int r = 16 * q + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    int64_t gr = m0 + r;
    gr = gr < M ? gr : M - 1;
    xsrc[i] = x + gr * K + 8 * c;
    int wr;
    if (SWIGLU) {
      int colr = n0 + (r & 127);
      colr = colr < N ? colr : N - 1;
      wr = colr + (r >= 128 ? N : 0);
    } else {
      wr = n0 + r;
      wr = wr < N ? wr : N - 1;
    }
    wsrc[i] = w + static_cast<int64_t>(wr) * K + 8 * c;
  }
  auto issue = [&](int stage, int k0) {
    char *base = smem + (stage % GB_STAGES) * GB_STAGEB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = wid + 4 * i;
      __builtin_amdgcn_global_load_lds(xsrc[i] + k0, (lds_void *)(base + q * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(wsrc[i] + k0, (lds_void *)(base + GB_TILEB + q * 1024), 16, 0, 0);
    }
  };

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, fg = lane >> 4;
  // fragment byte offsets inside a tile: row R, chunk fg -> R * 64 + 16 * (fg ^ ((R >> 2) & 3))
  int xoff[8], woff[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int R = wm * 128 + 16 * j + fr;
    xoff[j] = R * GB_ROWB + 16 * (fg ^ ((R >> 2) & 3));
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int R = SWIGLU ? ((i < 4 ? 0 : 128) + wn * 64 + 16 * (i & 3) + fr) : (wn * 128 + 16 * i + fr);
    woff[i] = GB_TILEB + R * GB_ROWB + 16 * (fg ^ ((R >> 2) & 3));
  }

  const int nk = K / GB_BK;
#pragma unroll
  for (int s = 0; s < GB_STAGES - 1; ++s)
    if (s < nk) issue(s, s * GB_BK);
  for (int kt = 0; kt < nk; ++kt) {
    // this thread's loads of stage kt are done once at most (stages issued after it) x 8 remain
    const int ahead = min(nk - 1 - kt, GB_STAGES - 2);
    if (ahead >= 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // Every thread's slice of stage kt has landed (the wait above), so after the barrier the whole stage is
    // in LDS and stage kt - 1's slot is free. A bare s_barrier: __syncthreads() would add a release fence
    // that drains every outstanding load, the prefetched stages included.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + GB_STAGES - 1 < nk) issue(kt + GB_STAGES - 1, (kt + GB_STAGES - 1) * GB_BK);
    const char *base = smem + (kt % GB_STAGES) * GB_STAGEB;
    bf16x8 xf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xf[j] = *reinterpret_cast<const bf16x8 *>(base + xoff[j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bf16x8 wf = *reinterpret_cast<const bf16x8 *>(base + woff[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xf[j], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: acc[i][j] lane holds C^T[w row 16 i + 4 g + e][x row 16 j + lane % 16], e = 0..3
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t row = m0 + wm * 128 + 16 * j + fr;
    if (row >= M) continue;
    if (SWIGLU) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = n0 + wn * 64 + 16 * i + 4 * fg;
        if (col >= N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gt = round_bf(acc[i][j][e]);
          const float up = round_bf(acc[i + 4][j][e]);
          o[e] = round_bf(gt / (1.0f + __expf(-gt))) * up;
        }
        *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(y) + row * N + col) =
            u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int col = n0 + wn * 128 + 16 * i + 4 * fg;
        if (col >= N) continue;
        if (OUT_F32) {
          *reinterpret_cast<f32x4 *>(static_cast<float *>(y) + row * N + col) = acc[i][j];
        } else {
          *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(y) + row * N + col) =
              u32x2{pack_bf(acc[i][j][0], acc[i][j][1]), pack_bf(acc[i][j][2], acc[i][j][3])};
        }
      }
    }
  }
}

template <bool SWIGLU, bool OUT_F32>
static int launch_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, hipStream_t s) {
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_big_kernel<SWIGLU, OUT_F32>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(GB_SMEM)) != hipSuccess)
      return fail(VK_ERR_LAUNCH, "linear: cannot reserve %zu bytes of LDS", GB_SMEM);
    configured = true;
  }
  constexpr int OUT_COLS = SWIGLU ? 128 : 256;
  const int tiles_n = (N + OUT_COLS - 1) / OUT_COLS;
  const int64_t tiles_m = (M + GB_BM - 1) / GB_BM;
  const int64_t total = tiles_m * tiles_n;
  if (total >= (int64_t(1) << 31)) return fail(VK_ERR_ARG, "linear: too many tiles");
  gemm_big_kernel<SWIGLU, OUT_F32><<<static_cast<unsigned>(total), 256, GB_SMEM, s>>>(
      x, w, y, M, N, K, tiles_n, static_cast<int>(total));
  return VK_OK;
}

// Entry used by vk_linear for large M (K % 32 == 0, N % 4 == 0).
int gemm_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, bool swiglu, bool out_f32,
             hipStream_t s) {
  if (swiglu) return launch_big<true, false>(x, w, y, M, N, K, s);
  if (out_f32) return launch_big<false, true>(x, w, y, M, N, K, s);
  return launch_big<false, false>(x, w, y, M, N, K, s);
}

}  // namespace vk
