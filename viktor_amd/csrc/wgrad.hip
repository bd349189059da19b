// Weight gradients of the GSPO update's linear layers: C[Ka, Kb] = A^T B = sum over packed rows r of
// A[r, ka] B[r, kb] (A = the output gradient [N, Ka], B = the layer input [N, Kb], both bf16 row-major), the
// products autograd forms for nn.Linear weights under autocast (viktor/decoder.py:58-59, 114-115 through
// loss.backward() at scripts/gspo.py:477), rounded to bf16 once as the autocast matmul output is.
//
// MI355X design:
//   * The reduction runs over ~10^5 rows into a small output (at most 3072 x 1536), so the rows are split into
//     S slices (split-K); each workgroup computes one 256 (ka) x 128 (kb) output tile over one slice and writes
//     its fp32 partial; a second kernel sums the S partials in slice order (deterministic) and rounds.
//   * The reduction index is the row index of both operands, so an MFMA operand (8 consecutive rows of one
//     column per lane) is a column segment of a row-major tile. Tiles reach LDS row-major by direct
//     global->LDS loads (global_load_lds_dwordx4, no registers), and the fragments are formed by gfx950's LDS
//     transpose read ds_read_b64_tr_b16: within each 16-lane group, source lane s reads 4 consecutive columns
//     4 (s % 4) .. + 3 of row R0 + s / 4, and output lane 4 a + b receives element b of source lanes a,
//     a + 4, a + 8, a + 12 -- i.e. column 4 a + b at rows R0 .. R0 + 3. Two reads (R0 = 8 g and 8 g + 4 for
//     lane group g) give the 16x16x32 operand layout: column = lane % 16, rows 8 g .. 8 g + 7.
//   * The product is formed transposed, C^T = B^T A (the B tile feeds the MFMA A operand), so a lane ends
//     with 4 consecutive kb of one ka: 16-byte partial stores.
//   * 8 consumer wavefronts (two per SIMD), each 64 (kb) x 64 (ka) = 16 fp32 MFMA tiles, and 2
//     producer wavefronts that only issue the direct loads, 3 stages ahead through a 4-slot ring of 32-row
//     stages (16 KB A + 8 KB B; 96 KB, one workgroup per CU); 16-byte chunk c of LDS row r sits in slot
//     c ^ 2 (r % 4), so the 4 rows x 32 bytes of one transpose read hit 8 distinct bank groups.
//   * XCD-aware order: the tiles of one slice are consecutive in the logical order and an XCD owns a
//     contiguous logical range, so they share the slice's rows in that XCD's L2.
#include "common.h"

namespace vk {

constexpr int WG_BJ = 256;  // ka (output rows) per workgroup: MFMA B operand columns
constexpr int WG_BI = 128;  // kb (output columns) per workgroup: MFMA A operand rows
constexpr int WG_BR = 32;   // packed rows (the reduction) per stage
constexpr int WG_NS = 4;    // ring slots
constexpr int WG_AHEAD = 3; // stages in flight ahead of the one being consumed
constexpr int WG_CONS = 8;  // consumer wavefronts (MFMA): two per SIMD
constexpr int WG_PROD = 2;  // producer wavefronts (direct loads)
constexpr int WG_AROWB = WG_BJ * 2;                   // 512 B: one row of the A tile
constexpr int WG_BROWB = WG_BI * 2;                   // 256 B: one row of the B tile
constexpr int WG_ATILEB = WG_BR * WG_AROWB;           // 16 KB
constexpr int WG_BTILEB = WG_BR * WG_BROWB;           // 8 KB
constexpr int WG_STAGEB = WG_ATILEB + WG_BTILEB;      // 24 KB
constexpr size_t WG_SMEM = static_cast<size_t>(WG_NS) * WG_STAGEB;  // 96 KB
constexpr int WG_PLOADS = (WG_ATILEB + WG_BTILEB) / 1024 / WG_PROD;  // direct loads per producer per stage (12)

typedef __attribute__((address_space(3))) void wg_lds_void;
typedef short wg_s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) wg_s4 wg_lds_s4;

constexpr int wg_vmcnt(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }
static_assert(WG_AHEAD * WG_PLOADS <= 63, "a producer's loads in flight must fit the 6-bit vmcnt counter");

// byte offset of (row r, 16-byte chunk c) in a tile with row_bytes per row
__device__ __forceinline__ int wg_slot(int r, int c, int row_bytes) { return r * row_bytes + 16 * (c ^ (2 * (r & 3))); }

// The 8-row x 16-column fragment for lane group g of column block cb in a tile (row_bytes per row) as one
// bf16x8: two transpose reads, rows 8 g .. 8 g + 3 and 8 g + 4 .. 8 g + 7.
__device__ __forceinline__ bf16x8 wg_frag(const char *tile, int row_bytes, int cb, int g, int s) {
  const int a = s & 3, t = s >> 2;
  const int c = 2 * cb + (a >> 1), half = 8 * (a & 1);
  const char *p0 = tile + wg_slot(8 * g + t, c, row_bytes) + half;
  const char *p1 = tile + wg_slot(8 * g + 4 + t, c, row_bytes) + half;
  const wg_s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((wg_lds_s4 *)(const __attribute__((address_space(3))) char *)p0);
  const wg_s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((wg_lds_s4 *)(const __attribute__((address_space(3))) char *)p1);
  typedef short s8 __attribute__((ext_vector_type(8)));
  const s8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Wave roles: waves 0..7 consume (fragments + MFMAs), waves 8..9 produce (direct loads). The compiler treats a
// transpose read as aliasing every direct load in flight in the same wave and would wait for all of them, so no
// wave does both: each role runs a loop of its own, and the two meet at one s_barrier per stage. At barrier kt,
// stage kt is in LDS (the producers waited for it) and every consumer is done with stage kt - 1, whose slot the
// producers then refill with stage kt + 3.
__global__ __launch_bounds__((WG_CONS + WG_PROD) * 64, 1) void wgrad_kernel(
    const bf16_t *__restrict__ A, int64_t lda, const bf16_t *__restrict__ B, int64_t ldb, int64_t N, int Ka, int Kb,
    int tiles_kb, int tiles, int slices, int64_t steps, float *__restrict__ ws) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);

  // XCD-aware order over (slice, tile), tile fastest: workgroup p runs on XCD p % 8, which owns a contiguous
  // logical range (a bijection for any count)
  const int total = tiles * slices;
  const int p = blockIdx.x, xcd = p & 7, idx = p >> 3;
  const int q8 = total >> 3, r8 = total & 7;
  const int lt = xcd * q8 + min(xcd, r8) + idx;
  const int sl = lt / tiles, tile = lt % tiles;
  const int ka0 = (tile / tiles_kb) * WG_BJ, kb0 = (tile % tiles_kb) * WG_BI;
  // this slice's 32-row steps [st0, st1); rows past N (the last step of the last slice) are masked
  const int64_t st0 = steps * sl / slices, st1 = steps * (sl + 1) / slices;
  const int64_t r_end = st1 * WG_BR < N ? st1 * WG_BR : N;
  const int nst = static_cast<int>(st1 - st0);

  if (wid >= WG_CONS) {
    // ---- producer: instructions of a stage are A0..A15 (tile rows 2 q, 2 q + 1) then B0..B7 (rows 4 q ..
    // 4 q + 3); producer w takes every other one. Lane -> (row, LDS slot) and the chunk that belongs in it.
    const int pw = wid - WG_CONS;
    const bf16_t *src[WG_PLOADS];
    int row[WG_PLOADS], dst[WG_PLOADS];
#pragma unroll
    for (int i = 0; i < WG_PLOADS; ++i) {
      const int q = pw + WG_PROD * i;  // 0 .. 23
      if (q < 16) {
        const int r = 2 * q + (lane >> 5), sl32 = lane & 31;
        row[i] = r;
        src[i] = A + ka0 + 8 * (sl32 ^ (2 * (r & 3)));
        dst[i] = q * 1024;
      } else {
        const int qb = q - 16, r = 4 * qb + (lane >> 4), sl16 = lane & 15;
        row[i] = r;
        src[i] = B + kb0 + 8 * (sl16 ^ (2 * (r & 3)));
        dst[i] = WG_ATILEB + qb * 1024;
      }
    }
    auto issue = [&](int st) {
      char *base = smem + (st % WG_NS) * WG_STAGEB;
      const int64_t r0 = (st0 + st) * WG_BR;
#pragma unroll
      for (int i = 0; i < WG_PLOADS; ++i) {
        int64_t r = r0 + row[i];
        r = r < N ? r : N - 1;
        const int64_t ld = i < 8 ? lda : ldb;  // producer w: 8 A instructions, then 4 B instructions
        __builtin_amdgcn_global_load_lds(src[i] + r * ld, (wg_lds_void *)(base + dst[i]), 16, 0, 0);
      }
    };
#pragma unroll
    for (int st = 0; st < WG_AHEAD; ++st)
      if (st < nst) issue(st);
    for (int kt = 0; kt < nst; ++kt) {
      // stage kt complete: at most the loads of stages kt + 1 .. min(kt + 2, nst - 1) still in flight
      const int later = min(kt + WG_AHEAD - 1, nst - 1) - kt;
      if (later >= 2)
        __builtin_amdgcn_s_waitcnt(wg_vmcnt(2 * WG_PLOADS));
      else if (later == 1)
        __builtin_amdgcn_s_waitcnt(wg_vmcnt(WG_PLOADS));
      else
        __builtin_amdgcn_s_waitcnt(wg_vmcnt(0));
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (kt + WG_AHEAD < nst) issue(kt + WG_AHEAD);  // into stage kt - 1's slot, which every consumer has left
    }
    return;
  }

  // ---- consumers: wave w covers kb half w % 2 (64 of 128) and ka quarter w / 2 (64 of 256); the two consumer
  // waves of a SIMD overlap one's transpose reads with the other's MFMAs
  const int wi = wid & 1, wj = wid >> 1;
  const int g = lane >> 4, s16 = lane & 15;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kt = 0; kt < nst; ++kt) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // B_kt: stage kt is in LDS
    asm volatile("" ::: "memory");
    const char *base = smem + (kt % WG_NS) * WG_STAGEB;
    bf16x8 bfr[4], afr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) bfr[i] = wg_frag(base + WG_ATILEB, WG_BROWB, 4 * wi + i, g, s16);
#pragma unroll
    for (int j = 0; j < 4; ++j) afr[j] = wg_frag(base, WG_AROWB, 4 * wj + j, g, s16);
    const int64_t r0 = (st0 + kt) * WG_BR;
    if (r0 + WG_BR > r_end) {  // the last, partial step: rows r0 + 8 g + e at or past r_end add nothing
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (r0 + 8 * g + e >= r_end) bfr[i][e] = static_cast<__bf16>(0.f);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[i], afr[j], acc[i][j], 0, 0, 0);
  }

  // acc[i][j]: C^T block (kb block 4 wi + i, ka block 4 wj + j); lane -> ka = 16 block + lane % 16, kb = 16 block
  // + 4 (lane / 16) .. + 3: one 16-byte store of the slice's partial per (i, j)
  float *out = ws + static_cast<int64_t>(sl) * Ka * Kb;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ka = ka0 + 16 * (4 * wj + j) + s16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kb = kb0 + 16 * (4 * wi + i) + 4 * g;
      *reinterpret_cast<f32x4 *>(out + static_cast<int64_t>(ka) * Kb + kb) = acc[i][j];
    }
  }
}

// out[c] = sum over slices s (in order) of ws[s, c], rounded to bf16 (out_bf16) or kept fp32; 4 columns a thread.
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float *__restrict__ ws, int slices, int64_t n,
                                                           void *__restrict__ out, int out_bf16) {
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (c >= n) return;
  f32x4 acc = *reinterpret_cast<const f32x4 *>(ws + c);
  for (int s = 1; s < slices; ++s) acc += *reinterpret_cast<const f32x4 *>(ws + static_cast<int64_t>(s) * n + c);
  if (out_bf16)
    *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(out) + c) = u32x2{pack_bf(acc[0], acc[1]), pack_bf(acc[2], acc[3])};
  else
    *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + c) = acc;
}

static int wgrad_slices(int64_t N, int tiles, int cus) {
  const int64_t steps = (N + WG_BR - 1) / WG_BR;
  // one workgroup per CU and one round of them: a partial second round would double the time of its slices
  int64_t s = static_cast<int64_t>(cus > 0 ? cus : 256) / tiles;
  if (s > steps / 8) s = steps / 8;  // at least 8 steps (256 rows) per slice
  if (s < 1) s = 1;
  if (s > 1024) s = 1024;
  return static_cast<int>(s);
}

}  // namespace vk

using namespace vk;

extern "C" int vk_wgrad_workspace(int64_t N, int32_t Ka, int32_t Kb, int64_t *bytes) {
  VK_CHECK_ARG(bytes && N > 0 && Ka > 0 && Kb > 0, "wgrad_workspace: bad arguments");
  const int tiles = (Ka / WG_BJ) * (Kb / WG_BI);
  *bytes = static_cast<int64_t>(wgrad_slices(N, tiles > 0 ? tiles : 1, device_cus_cached())) * Ka * Kb *
           static_cast<int64_t>(sizeof(float));
  return VK_OK;
}

extern "C" int vk_wgrad(const void *a, int64_t lda, const void *b, int64_t ldb, int64_t N, int32_t Ka, int32_t Kb,
                        void *out, int32_t out_dtype, void *workspace, int64_t workspace_bytes, void *stream) {
  VK_CHECK_ARG(a && b && out && workspace, "wgrad: null pointer");
  VK_CHECK_ARG(N > 0 && Ka > 0 && Kb > 0 && Ka % WG_BJ == 0 && Kb % WG_BI == 0,
               "wgrad: need Ka %% 256 == 0 and Kb %% 128 == 0 (got N=%lld Ka=%d Kb=%d)", static_cast<long long>(N), Ka,
               Kb);
  VK_CHECK_ARG(lda >= Ka && ldb >= Kb && lda % 8 == 0 && ldb % 8 == 0, "wgrad: row strides (multiples of 8, >= width)");
  VK_CHECK_ARG(vk_aligned16(a) && vk_aligned16(b) && vk_aligned16(out) && vk_aligned16(workspace),
               "wgrad: 16-byte aligned operands");
  VK_CHECK_ARG(out_dtype == VK_DTYPE_BF16 || out_dtype == VK_DTYPE_F32, "wgrad: bad out dtype");
  const int tiles_kb = Kb / WG_BI, tiles = (Ka / WG_BJ) * tiles_kb;
  const int slices = wgrad_slices(N, tiles, device_cus_cached());
  const int64_t need = static_cast<int64_t>(slices) * Ka * Kb * static_cast<int64_t>(sizeof(float));
  VK_CHECK_ARG(workspace_bytes >= need, "wgrad: workspace of %lld bytes needed", static_cast<long long>(need));
  VK_CHECK_ARG(static_cast<int64_t>(tiles) * slices < (int64_t(1) << 31), "wgrad: too many workgroups");
  const int64_t steps = (N + WG_BR - 1) / WG_BR;
  VK_RAISE_LDS_ONCE(wgrad_kernel, WG_SMEM, "wgrad");  // 96 KB of dynamic LDS is above the default limit
  hipStream_t s = VK_STREAM(stream);
  wgrad_kernel<<<static_cast<unsigned>(tiles * slices), (WG_CONS + WG_PROD) * 64, WG_SMEM, s>>>(
      static_cast<const bf16_t *>(a), lda, static_cast<const bf16_t *>(b), ldb, N, Ka, Kb, tiles_kb, tiles, slices,
      steps, static_cast<float *>(workspace));
  const int rc = launch_status("wgrad");
  if (rc != VK_OK) return rc;
  const int64_t n = static_cast<int64_t>(Ka) * Kb;
  wgrad_reduce_kernel<<<static_cast<unsigned>((n / 4 + 255) / 256), 256, 0, s>>>(
      static_cast<const float *>(workspace), slices, n, out, out_dtype == VK_DTYPE_BF16);
  return launch_status("wgrad reduce");
}
