// Large-M GEMMs of the prefill / scoring forward: y[M, N] = x[M, K] @ w[N, K]^T, bf16 in, fp32 accumulate.
//
// MI355X design (M = tokens or frames x N = 512..4096 x K = 512..2048):
//   * 256 x 128 output tile per workgroup of 4 wavefronts, each wavefront 128 x 64 (32 fp32 MFMA tiles, 128
//     accumulator registers), so a wavefront fits in 256 registers and two workgroups share a CU: one
//     workgroup's barriers, LDS phases and epilogue overlap the other's MFMAs (with 256 x 256 tiles of
//     128 x 128 per wavefront, one wavefront per SIMD left all of those exposed).
//   * Operands reach LDS with gfx950's direct global->LDS loads (global_load_lds_dwordx4: lane l of an
//     instruction lands at LDS base + 16 l), so the prefetch costs no registers; a 3-stage ring of 32-wide K
//     slices (72 KB) keeps two slices in flight while one feeds the MFMAs. LDS rows are 64 B without padding;
//     the 16-byte slot of K chunk c in row r is c ^ ((r >> 1) & 3), so the 8 lanes of a fragment-read phase
//     (8 consecutive rows, one chunk) hit 8 distinct bank groups. A wavefront reads its 12 fragments of a
//     slice before its 32 MFMAs (pinned with sched_group_barrier).
//   * Tiles are ordered XCD-aware: workgroup p runs on XCD p % 8, so each XCD gets a contiguous range of
//     tiles and the N-tiles that share a block of x rows share that XCD's L2.
//   * The product is formed transposed, C^T = W X^T (the weight fragment is the MFMA A operand), so each
//     lane ends with 4 consecutive output columns of one row; the epilogue stages each wavefront's quadrant
//     through LDS and stores whole rows in 16-byte chunks.
//   * SwiGLU: the tile's W rows are 64 gate rows and the matching 64 up rows; both land in the same lane,
//     and the epilogue stores bf16(bf16(silu(bf16(g))) * bf16(u)) over 64 output columns.
//   * Every row of y is computed by the same code whatever M is (no split of K), so a row's result does not
//     depend on the other rows of the product.
#include "common.h"

namespace vk {

constexpr int GB_BM = 256;   // rows of x per workgroup
constexpr int GB_BW = 128;   // rows of w per workgroup
constexpr int GB_BK = 32;    // K per stage
constexpr int GB_STAGES = 3;
constexpr int GB_ROWB = GB_BK * 2;                   // bytes per LDS row
constexpr int GB_XTILEB = GB_BM * GB_ROWB;           // 16 KB
constexpr int GB_WTILEB = GB_BW * GB_ROWB;           // 8 KB
constexpr int GB_STAGEB = GB_XTILEB + GB_WTILEB;     // 24 KB
constexpr size_t GB_SMEM = static_cast<size_t>(GB_STAGES) * GB_STAGEB;  // 72 KB: two workgroups per CU
constexpr int GB_LOADS = 6;                          // direct loads per thread per stage (4 x + 2 w)

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate that waits for vmcnt <= n and leaves expcnt / lgkmcnt unconstrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt in 6:4, lgkmcnt in 11:8)
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

template <bool SWIGLU, bool OUT_F32>
__global__ __launch_bounds__(256, 2) void gemm_big_kernel(const bf16_t *__restrict__ x, const bf16_t *__restrict__ w,
                                                          void *__restrict__ y, int64_t M, int N, int K, int tiles_n,
                                                          int tiles_total) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  constexpr int OUT_COLS = SWIGLU ? 64 : 128;

  // XCD-aware tile order: physical workgroup p runs on XCD p % 8; XCD x owns the contiguous logical
  // range [x q + min(x, r), ...) of q + (x < r) tiles (q = total / 8, r = total % 8) -- a bijection
  const int p = blockIdx.x;
  const int xcd = p & 7, idx = p >> 3;
  const int q8 = tiles_total >> 3, r8 = tiles_total & 7;
  const int tile = xcd * q8 + min(xcd, r8) + idx;
  const int mt = tile / tiles_n, nt = tile % tiles_n;
  const int64_t m0 = static_cast<int64_t>(mt) * GB_BM;
  const int n0 = nt * OUT_COLS;

  // direct-load sources: instruction q of an operand tile covers its rows 16 q .. 16 q + 15 (x: q < 16,
  // w: q < 8); wave w issues q = w + 4 i. Lane l -> row 16 q + l / 4, LDS slot l % 4, K chunk slot ^ swizzle.
  const bf16_t *xsrc[4];
  const bf16_t *wsrc[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * (wid + 4 * i) + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 1) & 3);
    int64_t gr = m0 + r;
    gr = gr < M ? gr : M - 1;
    xsrc[i] = x + gr * K + 8 * c;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 16 * (wid + 4 * i) + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 1) & 3);
    int wr;
    if (SWIGLU) {  // tile rows 0..63: gate rows n0.., rows 64..127: the matching up rows N + n0..
      int colr = n0 + (r & 63);
      colr = colr < N ? colr : N - 1;
      wr = colr + (r >= 64 ? N : 0);
    } else {
      wr = n0 + r;
      wr = wr < N ? wr : N - 1;
    }
    wsrc[i] = w + static_cast<int64_t>(wr) * K + 8 * c;
  }
  auto issue = [&](int stage, int k0) {
    char *base = smem + (stage % GB_STAGES) * GB_STAGEB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(xsrc[i] + k0, (lds_void *)(base + (wid + 4 * i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(wsrc[i] + k0, (lds_void *)(base + GB_XTILEB + (wid + 4 * i) * 1024), 16, 0, 0);
  };

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, fg = lane >> 4;
  // fragment byte offsets inside a tile: row R, chunk fg -> R * 64 + 16 * (fg ^ ((R >> 1) & 3))
  int xoff[8], woff[4];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int R = wm * 128 + 16 * j + fr;
    xoff[j] = R * GB_ROWB + 16 * (fg ^ ((R >> 1) & 3));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int R = SWIGLU ? ((i < 2 ? 0 : 64) + wn * 32 + 16 * (i & 1) + fr) : (wn * 64 + 16 * i + fr);
    woff[i] = GB_XTILEB + R * GB_ROWB + 16 * (fg ^ ((R >> 1) & 3));
  }

  const int nk = K / GB_BK;
#pragma unroll
  for (int s = 0; s < GB_STAGES - 1; ++s)
    if (s < nk) issue(s, s * GB_BK);
  for (int kt = 0; kt < nk; ++kt) {
    // this thread's loads of stage kt are done once at most (stages issued after it) x GB_LOADS remain
    if (kt + 1 < nk)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(GB_LOADS));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // Every thread's slice of stage kt has landed (the wait above), so after the barrier the whole stage is
    // in LDS and stage kt - 1's slot is free. A bare s_barrier: __syncthreads() would add a release fence
    // that drains every outstanding load, the prefetched stage included.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + GB_STAGES - 1 < nk) issue(kt + GB_STAGES - 1, (kt + GB_STAGES - 1) * GB_BK);
    const char *base = smem + (kt % GB_STAGES) * GB_STAGEB;
    bf16x8 xf[8], wf[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) xf[j] = *reinterpret_cast<const bf16x8 *>(base + xoff[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) wf[i] = *reinterpret_cast<const bf16x8 *>(base + woff[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
    // keep that order: the scheduler would otherwise sink each W read next to its 8 MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // 12 LDS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);  // then the 32 MFMAs
  }

  // Epilogue through LDS: a lane holds 4 consecutive columns of one row per (i, j), so direct stores would
  // write 16 rows x 16-32 B per instruction. Each wavefront instead stages its 128-row quadrant in its own
  // quarter of the (now idle) ring, a pass of rows at a time (row pitch + 16 B against bank conflicts), and
  // stores 16-byte chunks whose lanes cover whole rows.
  __syncthreads();  // every wavefront has finished reading the ring
  constexpr int ESZ = OUT_F32 ? 4 : 2;                // output element bytes
  constexpr int QCOLS = SWIGLU ? 32 : 64;             // output columns of a wavefront
  constexpr int RB = QCOLS * ESZ;                     // bytes of one quadrant row
  constexpr int PITCH = RB + 16;
  constexpr int PASS_ROWS = OUT_F32 ? 64 : 128;       // rows staged per pass (<= GB_SMEM / 4 bytes)
  constexpr int CPR = RB / 16;                        // 16-byte chunks per row
  static_assert(PASS_ROWS * PITCH <= static_cast<int>(GB_SMEM / 4), "epilogue staging exceeds a quarter of LDS");
  char *stg = smem + wid * (GB_SMEM / 4);
  const int64_t qrow0 = m0 + wm * 128;
  const int qcol0 = n0 + wn * QCOLS;
#pragma unroll
  for (int pass = 0; pass < 128 / PASS_ROWS; ++pass) {
#pragma unroll
    for (int jj = 0; jj < PASS_ROWS / 16; ++jj) {
      const int j = pass * (PASS_ROWS / 16) + jj;
      char *rowp = stg + (16 * jj + fr) * PITCH;
      if (SWIGLU) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gt = round_bf(acc[i][j][e]);
            const float up = round_bf(acc[i + 2][j][e]);
            o[e] = round_bf(gt / (1.0f + __expf(-gt))) * up;
          }
          *reinterpret_cast<u32x2 *>(rowp + (16 * i + 4 * fg) * 2) = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (OUT_F32)
            *reinterpret_cast<f32x4 *>(rowp + (16 * i + 4 * fg) * 4) = acc[i][j];
          else
            *reinterpret_cast<u32x2 *>(rowp + (16 * i + 4 * fg) * 2) =
                u32x2{pack_bf(acc[i][j][0], acc[i][j][1]), pack_bf(acc[i][j][2], acc[i][j][3])};
        }
      }
    }
    // same wavefront reads back (LDS keeps a wavefront's accesses in order): chunk id -> (row, chunk)
#pragma unroll
    for (int it = 0; it < PASS_ROWS * CPR / 64; ++it) {
      const int id = it * 64 + lane;
      const int r = id / CPR, c = id % CPR;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + r * PITCH + c * 16);
      const int64_t row = qrow0 + pass * PASS_ROWS + r;
      const int col = qcol0 + c * (16 / ESZ);
      if (row < M && col < N)
        *reinterpret_cast<u32x4 *>(static_cast<char *>(y) + (row * N + col) * ESZ) = v;
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
  constexpr int OUT_COLS = SWIGLU ? 64 : 128;
  const int tiles_n = (N + OUT_COLS - 1) / OUT_COLS;
  const int64_t tiles_m = (M + GB_BM - 1) / GB_BM;
  const int64_t total = tiles_m * tiles_n;
  if (total >= (int64_t(1) << 31)) return fail(VK_ERR_ARG, "linear: too many tiles");
  gemm_big_kernel<SWIGLU, OUT_F32><<<static_cast<unsigned>(total), 256, GB_SMEM, s>>>(
      x, w, y, M, N, K, tiles_n, static_cast<int>(total));
  return VK_OK;
}

// Entry used by vk_linear for large M and by vk_gemm_rows (K % 64 == 0: an even number of K slices; N % 8 == 0:
// whole 16-byte output chunks).
int gemm_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, bool swiglu, bool out_f32,
             hipStream_t s) {
  if (swiglu) return launch_big<true, false>(x, w, y, M, N, K, s);
  if (out_f32) return launch_big<false, true>(x, w, y, M, N, K, s);
  return launch_big<false, false>(x, w, y, M, N, K, s);
}

}  // namespace vk
