// Large-M GEMMs of the prefill / scoring forward: y[M, N] = x[M, K] @ w[N, K]^T, bf16 in, fp32 accumulate.
//
// MI355X design (M = tokens or frames x N = 512..4096 x K = 512..2048):
//   * 256 x 128 output tile per workgroup of 4 wavefronts, each wavefront 128 x 64 (32 fp32 MFMA tiles, 128
//     accumulator registers), so a wavefront fits in 256 registers and two workgroups share a CU: one
//     workgroup's barriers, LDS phases and epilogue overlap the other's MFMAs (with 256 x 256 tiles of
//     128 x 128 per wavefront, one wavefront per SIMD left all of those exposed). Plain products use 256 x 256
//     tiles of 8 such wavefronts instead (one workgroup per CU, a third fewer global->LDS bytes per flop).
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
#include <type_traits>

#include "common.h"

namespace vk {

constexpr int GB_BM = 256;   // rows of x per workgroup
constexpr int GB_BK = 32;    // K per stage
constexpr int GB_GM = 8;     // row blocks per group of the tile order
constexpr int GB_STAGES = 3;
constexpr int GB_ROWB = GB_BK * 2;                   // bytes per LDS row
constexpr int GB_XTILEB = GB_BM * GB_ROWB;           // 16 KB

// GW wavefronts along the weight rows, each 64 of them; 2 GW wavefronts per workgroup, every one a 128 x 64 block.
// GW = 2: 256 x 128 tiles, 4 wavefronts, 72 KB of ring (two workgroups per CU); GW = 4: 256 x 256 tiles, 8
// wavefronts, 96 KB (one workgroup per CU): a third fewer global->LDS bytes per flop.
template <int GW>
struct GbShape {
  static constexpr int WAVES = 2 * GW;
  static constexpr int BW = 64 * GW;                                   // rows of w per workgroup
  static constexpr int WTILEB = BW * GB_ROWB;                          // 8 / 16 KB
  static constexpr int STAGEB = GB_XTILEB + WTILEB;                    // 24 / 32 KB
  static constexpr size_t SMEM = static_cast<size_t>(GB_STAGES) * STAGEB;  // 72 / 96 KB
  static constexpr int XLOADS = 16 / WAVES;                            // x instructions per wave per stage
  static constexpr int LOADS = XLOADS + 2;                             // + 2 w instructions
  static constexpr int WG_PER_CU = GW == 2 ? 2 : 1;
};

typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte direct global->LDS load per lane (lane l lands at dst + 16 l). A plain device function: written in
// a kernel template with arguments that depend on its parameters, the builtin makes the host pass drop the
// kernel's launch stub.
__device__ __forceinline__ void gb_load_lds(const bf16_t *src, char *dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 16, 0, 0);
}

// s_waitcnt immediate that waits for vmcnt <= n and leaves expcnt / lgkmcnt unconstrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt in 6:4, lgkmcnt in 11:8)
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

// Epilogues: bf16 out, fp32 out, SwiGLU, or the attention input stage of a Wqkv product (GB_QKV): the
// product's 64-column heads (H q heads, HKV k heads, HKV v heads) are rounded to bf16 as the unfused product
// stores them; q and k heads then get the per-head RMSNorm (when qw / kw are given: bf16(x / rms * w)) and
// the half-split rotary embedding at the row's position (bf16(y1 c - y2 s), bf16(y1 s + y2 c), with the
// table entries as stored), the rounding points of vk_qkv_rope_cache; then every head goes to its
// destination -- q rows, the KV cache and / or k / v rows.
//
// GB_RESID: y is a bf16 residual stream updated in place, y = bf16(bf16(acc + bias) + bf16(alpha y)) (alpha = 1,
// no bias: add_rmsnorm's x += bf16(delta); the encoder's DeepNorm sum with its out_proj bias and alpha), and
// ss_out[row, col / 64] receives the fp32 sum of squares of the row's new bf16 values over each 64-column block
// (the RMSNorm that follows reads them instead of a pass of its own over the row).
// GB_QKV reads fp32 rotary tables, GB_QKV_BF16 bf16 ones (the table type is a compile-time choice, so the epilogue's
// prefetched table registers are not merged across two load shapes); both take bf16 QK-norm weights. GB_QKV_W32 is
// GB_QKV with fp32 QK-norm weights: nn.RMSNorm under torch.autocast bf16 with fp32 master weights, which returns
// bf16(x / rms * w) for a bf16 head (the multiply by w in fp32, one rounding), before the fp32 rotation.
//
// GB_RESID_F32: y is an fp32 residual stream updated in place, y = alpha y + bf16(acc + bias): the autocast residual
// add x + sublayer(x) of an fp32 stream and a bf16 product (viktor/decoder.py:118-120 under torch.autocast bf16);
// ss_out as GB_RESID, over the new fp32 values.
// Both residual forms read the old residual from resid_in instead when it is given (out of place: y is then only
// written, and resid_in keeps the previous layer's stream, as a backward pass needs it).
enum GbEpi { GB_BF16 = 0, GB_F32 = 1, GB_SWIGLU = 2, GB_QKV = 3, GB_RESID = 4, GB_QKV_BF16 = 5, GB_RESID_F32 = 6,
             GB_QKV_W32 = 7 };

struct GbQkv {
  const void *qw, *kw;  // per-head RMSNorm weights [64], bf16 (fp32 for GB_QKV_W32); both NULL: no norm
  float eps;
  const void *cos_t, *sin_t;  // [table_rows, 32], fp32 (table_f32) or bf16
  int table_f32;
  int64_t table_rows;
  const int32_t *pos, *rope_pos, *seq;  // per row: cache position, rotary position (NULL: pos), cache row
  bf16_t *q;                            // q head h of row t at q + t q_ld + 64 h
  int64_t q_ld;
  bf16_t *kc, *vc;  // cache row (seq, pos) head h at kc + seq stride_cb + pos stride_cs + 64 h (NULL: none)
  int64_t stride_cb, stride_cs, cache_rows, cache_len;
  bf16_t *ko, *vo;  // k / v head h of row t at ko + t kv_ld + 64 h (NULL: none)
  int64_t kv_ld;
  bf16_t *raw;      // the product itself, rounded to bf16, rows [M, N] before the QK-norm and rotation (NULL: none)
  int H, HKV;
  // GB_RESID
  const float *bias;  // [N] or NULL
  float alpha;
  float *ss_out;         // [M, N / 64]
  const void *resid_in;  // the old residual rows [M, N] (NULL: the output itself, updated in place)
};

template <int EPI, int GW>
__global__ __launch_bounds__(128 * GW, 4 / GW) void gemm_big_kernel(
    const bf16_t *__restrict__ x, const bf16_t *__restrict__ w, void *__restrict__ y, int64_t M, int N, int K,
    int tiles_n, int tiles_total, const GbQkv qa) {
  using SH = GbShape<GW>;
  constexpr int GB_STAGEB = SH::STAGEB, GB_LOADS = SH::LOADS, NWAVES = SH::WAVES;
  constexpr size_t GB_SMEM = SH::SMEM;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr bool SWIGLU = EPI == GB_SWIGLU, OUT_F32 = EPI == GB_F32, RESID = EPI == GB_RESID;
  constexpr bool RESID32 = EPI == GB_RESID_F32;
  constexpr bool QKV = EPI == GB_QKV || EPI == GB_QKV_BF16 || EPI == GB_QKV_W32;
  constexpr bool TAB_F32 = EPI == GB_QKV || EPI == GB_QKV_W32, W32 = EPI == GB_QKV_W32;
  // wid through readfirstlane: wave-uniform for the compiler, so branches on the wavefront's quadrant or head are scalar
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / GW, wn = wid % GW;
  constexpr int OUT_COLS = SWIGLU ? 32 * GW : 64 * GW;

  // XCD-aware tile order: physical workgroup p runs on XCD p % 8; XCD x owns the contiguous logical
  // range [x q + min(x, r), ...) of q + (x < r) tiles (q = total / 8, r = total % 8) -- a bijection
  const int p = blockIdx.x;
  const int xcd = p & 7, idx = p >> 3;
  const int q8 = tiles_total >> 3, r8 = tiles_total & 7;
  const int tile = xcd * q8 + min(xcd, r8) + idx;
  // logical order: groups of GB_GM row blocks, each walked column block by column block (GB_GM row blocks
  // per column block), so an XCD's resident workgroups share GB_GM A blocks and a few weight blocks in its
  // L2 instead of every weight block (a bijection: the last group has the remaining row blocks)
  const int tiles_m = tiles_total / tiles_n;
  const int grp = tile / (GB_GM * tiles_n), first_m = grp * GB_GM;
  const int gm = min(tiles_m - first_m, GB_GM), in_grp = tile - grp * GB_GM * tiles_n;
  const int mt = first_m + in_grp % gm, nt = in_grp / gm;
  const int64_t m0 = static_cast<int64_t>(mt) * GB_BM;
  const int n0 = nt * OUT_COLS;

  // direct-load sources: instruction q of an operand tile covers its rows 16 q .. 16 q + 15 (x: q < 16,
  // w: q < 4 GW); wave w issues q = w + NWAVES i. Lane l -> row 16 q + l / 4, LDS slot l % 4, K chunk slot ^ swizzle.
  const bf16_t *xsrc[SH::XLOADS];
  const bf16_t *wsrc[2];
#pragma unroll
  for (int i = 0; i < SH::XLOADS; ++i) {
    const int r = 16 * (wid + NWAVES * i) + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 1) & 3);
    int64_t gr = m0 + r;
    gr = gr < M ? gr : M - 1;
    xsrc[i] = x + gr * K + 8 * c;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 16 * (wid + NWAVES * i) + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 1) & 3);
    int wr;
    if (SWIGLU) {  // tile rows 0..32 GW - 1: gate rows n0.., the next 32 GW: the matching up rows N + n0..
      int colr = n0 + (r & (32 * GW - 1));
      colr = colr < N ? colr : N - 1;
      wr = colr + (r >= 32 * GW ? N : 0);
    } else {
      wr = n0 + r;
      wr = wr < N ? wr : N - 1;
    }
    wsrc[i] = w + static_cast<int64_t>(wr) * K + 8 * c;
  }
  auto issue = [&](int stage, int k0) {
    char *base = smem + (stage % GB_STAGES) * GB_STAGEB;
#pragma unroll
    for (int i = 0; i < SH::XLOADS; ++i) gb_load_lds(xsrc[i] + k0, base + (wid + NWAVES * i) * 1024);
#pragma unroll
    for (int i = 0; i < 2; ++i) gb_load_lds(wsrc[i] + k0, base + GB_XTILEB + (wid + NWAVES * i) * 1024);
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
    const int R = SWIGLU ? ((i < 2 ? 0 : 32 * GW) + wn * 32 + 16 * (i & 1) + fr) : (wn * 64 + 16 * i + fr);
    woff[i] = GB_XTILEB + R * GB_ROWB + 16 * (fg ^ ((R >> 1) & 3));
  }

  // The plain, fp32 and SwiGLU epilogues (whose values live across the loop leave room for a second set of
  // fragment registers) run a software-pipelined K loop: a wavefront reads its 12 fragments of slice kt + 1
  // while its 32 MFMAs of slice kt run, from two register sets (the loop unrolled by two). Slice kt + 1 must
  // then be whole in LDS one slice earlier, and slice kt + 3 goes into slice kt's slot once every wavefront has
  // its fragments of slice kt in registers, so two slices stay in flight during the MFMAs, as with reads right
  // before them. The other epilogues would spill with the second set; they read a slice's fragments right
  // before its MFMAs.
  constexpr bool PIPE = EPI == GB_BF16 || EPI == GB_F32 || EPI == GB_SWIGLU;
  const int nk = K / GB_BK;
#pragma unroll
  for (int s = 0; s < GB_STAGES - 1; ++s)
    if (s < nk) issue(s, s * GB_BK);
  auto read_frags = [&](int kt, bf16x8(&xf)[8], bf16x8(&wf)[4]) {
    const char *base = smem + (kt % GB_STAGES) * GB_STAGEB;
#pragma unroll
    for (int j = 0; j < 8; ++j) xf[j] = *reinterpret_cast<const bf16x8 *>(base + xoff[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) wf[i] = *reinterpret_cast<const bf16x8 *>(base + woff[i]);
  };
  auto mfmas = [&](const bf16x8(&xf)[8], const bf16x8(&wf)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
  };
  if constexpr (PIPE) {
    // this thread's loads of slice kt + 1 are done once at most slice kt + 2's remain, and its fragment reads
    // of slice kt are done; after the barrier slice kt + 1 is whole in LDS and slice kt's slot is free for
    // kt + 3. A bare s_barrier: __syncthreads() would add a release fence that drains every outstanding load,
    // the prefetched slices included.
    auto next_slice = [&](int kt) {
      if (kt + 2 < nk)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(GB_LOADS));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (kt + GB_STAGES < nk) issue(kt + GB_STAGES, (kt + GB_STAGES) * GB_BK);
    };
    // one LDS read of the next slice between every two MFMAs of this one, then the last 8 MFMAs
#define GB_INTERLEAVE()                                  \
  do {                                                   \
    _Pragma("unroll") for (int r_ = 0; r_ < 12; ++r_) {  \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0); \
    }                                                    \
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);   \
  } while (0)
    bf16x8 xa[8], wa[4], xb[8], wb[4];
    // slice 0 whole in LDS (slice 2 then goes into the ring's third slot), its fragments read
    if (nk > 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(GB_LOADS));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (GB_STAGES - 1 < nk) issue(GB_STAGES - 1, (GB_STAGES - 1) * GB_BK);
    read_frags(0, xa, wa);
    // Pairs of slices; the second step of the last pair may have no next slice: it then re-reads slice nk - 1
    // (its LDS slot is no longer written), so no branch separates a step's reads from its MFMAs and the
    // scheduler can interleave them. An odd count leaves slice nk - 1 in xa for the step after the loop.
    // next_slice(j) with j + 1 == nk waits for every load and passes a barrier; it issues nothing.
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
      next_slice(kt);
      read_frags(kt + 1, xb, wb);
      mfmas(xa, wa);
      GB_INTERLEAVE();
      next_slice(kt + 1);  // (past the last slice: only the waits and the barrier)
      read_frags(min(kt + 2, nk - 1), xa, wa);
      mfmas(xb, wb);
      GB_INTERLEAVE();
    }
    if (kt < nk) {
      __builtin_amdgcn_s_waitcnt(0xC07F);
      mfmas(xa, wa);
    }
#undef GB_INTERLEAVE
  } else {
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
      bf16x8 xf[8], wf[4];
      read_frags(kt, xf, wf);
      mfmas(xf, wf);
      // keep that order: the scheduler would otherwise sink each W read next to its 8 MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // 12 LDS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);  // then the 32 MFMAs
    }
  }

  // Epilogue through LDS: a lane holds 4 consecutive columns of one row per (i, j), so direct stores would
  // write 16 rows x 16-32 B per instruction. Each wavefront instead stages its 128-row quadrant in its own
  // quarter of the (now idle) ring, a pass of rows at a time (row pitch + 16 B against bank conflicts), and
  // stores 16-byte chunks whose lanes cover whole rows.
  // The epilogue's global operands are loaded here, before the barrier, so their round trips overlap the other
  // wavefronts' last MFMAs instead of being taken one 16-row group at a time: the residual rows and the bias
  // (GB_RESID), the QK-norm weights and every row's rotary position (GB_QKV; the table rows, which depend on the
  // positions, go one group ahead inside the loop).
  const int fr_e = lane & 15, fg_e = lane >> 4;
  u32x2 res_old[RESID ? 8 : 1][4];
  f32x4 res_b4[(RESID || RESID32) ? 4 : 1];
  // GB_RESID_F32: the old fp32 residual of two 16-row groups (the current one and the next, loaded one group ahead;
  // all 8 would take 128 registers beside the accumulators)
  f32x4 r32_old[RESID32 ? 2 : 1][4];
  auto r32_load = [&](int j, f32x4 (&dst)[4]) {
    int64_t rrow = m0 + wm * 128 + 16 * j + fr_e;
    rrow = rrow < M ? rrow : M - 1;
    const float *yrow = static_cast<const float *>(qa.resid_in ? qa.resid_in : y) + rrow * N + n0 + wn * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = *reinterpret_cast<const f32x4 *>(yrow + 16 * i + 4 * fg_e);
  };
  using NwT = typename std::conditional<W32, f32x4, u32x2>::type;
  NwT qk_nw[QKV ? 4 : 1];
  int qk_rp[QKV ? 8 : 1];
  const int qk_hd = (n0 + wn * 64) >> 6;  // GB_QKV: this wavefront's head (64 columns, wave-uniform)
  const bool qk_rot = QKV && qk_hd < qa.H + qa.HKV;
  const void *qk_w = QKV ? (qk_hd < qa.H ? qa.qw : qa.kw) : nullptr;
  if (RESID32) {
    r32_load(0, r32_old[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      res_b4[i] = qa.bias != nullptr ? *reinterpret_cast<const f32x4 *>(qa.bias + n0 + wn * 64 + 16 * i + 4 * fg_e)
                                     : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (RESID) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int64_t rrow = m0 + wm * 128 + 16 * j + fr_e;
      rrow = rrow < M ? rrow : M - 1;
      const bf16_t *yrow = static_cast<const bf16_t *>(qa.resid_in ? qa.resid_in : y) + rrow * N + n0 + wn * 64;
#pragma unroll
      for (int i = 0; i < 4; ++i) res_old[j][i] = *reinterpret_cast<const u32x2 *>(yrow + 16 * i + 4 * fg_e);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      res_b4[i] = qa.bias != nullptr ? *reinterpret_cast<const f32x4 *>(qa.bias + n0 + wn * 64 + 16 * i + 4 * fg_e)
                                     : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (qk_rot) {
    if (qk_w != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (W32)
          qk_nw[i] = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(qk_w) + 16 * i + 4 * fg_e);
        else
          qk_nw[i] = *reinterpret_cast<const u32x2 *>(static_cast<const bf16_t *>(qk_w) + 16 * i + 4 * fg_e);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int64_t rrow = m0 + wm * 128 + 16 * j + fr_e;
      rrow = rrow < M ? rrow : M - 1;
      int64_t rp = qa.rope_pos != nullptr ? qa.rope_pos[rrow] : qa.pos[rrow];
      qk_rp[j] = static_cast<int>(rp < 0 ? 0 : (rp >= qa.table_rows ? qa.table_rows - 1 : rp));
    }
  }
  // GB_QKV: the rotary table entries of 16-row group j (lane: its row's 4 consecutive entries at 16 i + 4 fg,
  // i = 0, 1): four fp32 values (GB_QKV) or four bf16 values in two words (GB_QKV_BF16) per table and i
  using TabT = typename std::conditional<TAB_F32, f32x4, u32x2>::type;
  auto qk_tables = [&](int j, TabT (&c)[2], TabT (&sn)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t ti = static_cast<int64_t>(qk_rp[j]) * 32 + 16 * i + 4 * fg_e;
      if constexpr (TAB_F32) {
        c[i] = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(qa.cos_t) + ti);
        sn[i] = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(qa.sin_t) + ti);
      } else {
        c[i] = *reinterpret_cast<const u32x2 *>(static_cast<const bf16_t *>(qa.cos_t) + ti);
        sn[i] = *reinterpret_cast<const u32x2 *>(static_cast<const bf16_t *>(qa.sin_t) + ti);
      }
    }
  };
  TabT qk_c[2][2], qk_s[2][2];  // two row groups' table entries: the current one and the next
  if (qk_rot) qk_tables(0, qk_c[0], qk_s[0]);
  __syncthreads();  // every wavefront has finished reading the ring
  constexpr int ESZ = (OUT_F32 || RESID32) ? 4 : 2;   // output element bytes
  constexpr int QCOLS = SWIGLU ? 32 : 64;             // output columns of a wavefront
  constexpr int RB = QCOLS * ESZ;                     // bytes of one quadrant row
  constexpr int PITCH = RB + 16;
  // rows staged per pass: what fits this wavefront's share of the ring (a power of two, 32..128)
  constexpr int STG_BYTES = static_cast<int>(GB_SMEM / NWAVES);
  constexpr int PASS_ROWS = 128 * PITCH <= STG_BYTES ? 128 : (64 * PITCH <= STG_BYTES ? 64 : 32);
  constexpr int CPR = RB / 16;                        // 16-byte chunks per row
  static_assert(PASS_ROWS * PITCH <= STG_BYTES, "epilogue staging exceeds the wavefront's share of LDS");
  char *stg = smem + wid * STG_BYTES;
  const int64_t qrow0 = m0 + wm * 128;
  const int qcol0 = n0 + wn * QCOLS;
#pragma unroll
  for (int pass = 0; pass < 128 / PASS_ROWS; ++pass) {
#pragma unroll
    for (int jj = 0; jj < PASS_ROWS / 16; ++jj) {
      const int j = pass * (PASS_ROWS / 16) + jj;
      char *rowp = stg + (16 * jj + fr) * PITCH;
      if (RESID) {
        // lane: row 16 j + fr, columns qcol0 + 16 i + 4 fg + e; the old residual is read right here (each element
        // by the lane that overwrites it)
        int64_t rrow = qrow0 + 16 * j + fr;
        const bool live = rrow < M;
        rrow = live ? rrow : M - 1;
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x2 old = res_old[j][i];
          const f32x4 b4 = res_b4[i];
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float xo = (e & 1) ? hi_bf(old[e >> 1]) : lo_bf(old[e >> 1]);
            o[e] = round_bf(round_bf(acc[i][j][e] + b4[e]) + round_bf(qa.alpha * xo));
            ss += o[e] * o[e];
          }
          *reinterpret_cast<u32x2 *>(rowp + (16 * i + 4 * fg) * 2) = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
        }
        ss += __shfl_xor(ss, 16, 64);  // the row's other 48 columns of this block: lanes fr + 16, + 32, + 48
        ss += __shfl_xor(ss, 32, 64);
        if (live && fg == 0) qa.ss_out[rrow * (N >> 6) + (qcol0 >> 6)] = ss;
      } else if (RESID32) {
        // lane: row 16 j + fr, columns qcol0 + 16 i + 4 fg + e (the same elements r32_load read for it)
        if (j + 1 < 8) r32_load(j + 1, r32_old[(j + 1) & 1]);
        const int64_t rrow = qrow0 + 16 * j + fr;
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 old = r32_old[j & 1][i];
          const f32x4 b4 = res_b4[i];
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[e] = qa.alpha * old[e] + round_bf(acc[i][j][e] + b4[e]);
            ss += o[e] * o[e];
          }
          *reinterpret_cast<f32x4 *>(rowp + (16 * i + 4 * fg) * 4) = o;
        }
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (rrow < M && fg == 0) qa.ss_out[rrow * (N >> 6) + (qcol0 >> 6)] = ss;
      } else if (QKV) {
        // this wavefront's 64 columns are one head (wave-uniform); lane: row 16 j + fr, columns 16 i + 4 fg + e
        const int hd = qcol0 >> 6;
        float v[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[i][e] = round_bf(acc[i][j][e]);
        if (qa.raw != nullptr && qcol0 < N) {  // the unrotated projection, as the plain product stores it
          const int64_t rrow = qrow0 + 16 * j + fr;
          if (rrow < M)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              *reinterpret_cast<u32x2 *>(qa.raw + rrow * N + qcol0 + 16 * i + 4 * fg) =
                  u32x2{pack_bf(v[i][0], v[i][1]), pack_bf(v[i][2], v[i][3])};
        }
        if (hd < qa.H + qa.HKV) {  // q or k head: QK-norm, then the rotation
          // the next group's table entries go out before this group's arithmetic
          if (j + 1 < 8) qk_tables(j + 1, qk_c[(j + 1) & 1], qk_s[(j + 1) & 1]);
          if (qk_w != nullptr) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int e = 0; e < 4; ++e) ss += v[i][e] * v[i][e];
            ss += __shfl_xor(ss, 16, 64);  // the row's other 48 columns: lanes fr + 16, + 32, + 48
            ss += __shfl_xor(ss, 32, 64);
            const float r = rsqrtf(ss * (1.0f / 64.0f) + qa.eps);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                float wv;
                if constexpr (W32)
                  wv = qk_nw[i][e];
                else
                  wv = (e & 1) ? hi_bf(qk_nw[i][e >> 1]) : lo_bf(qk_nw[i][e >> 1]);
                v[i][e] = round_bf(v[i][e] * r * wv);
              }
          }
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            // the lane's 4 consecutive table entries (loaded one group ahead)
            const TabT c4 = qk_c[j & 1][i], s4 = qk_s[j & 1][i];
            float cs[4], sn[4];
            if constexpr (TAB_F32) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                cs[e] = c4[e];
                sn[e] = s4[e];
              }
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                cs[e] = (e & 1) ? hi_bf(c4[e >> 1]) : lo_bf(c4[e >> 1]);
                sn[e] = (e & 1) ? hi_bf(s4[e >> 1]) : lo_bf(s4[e >> 1]);
              }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float y1 = v[i][e], y2 = v[i + 2][e];
              v[i][e] = y1 * cs[e] - y2 * sn[e];
              v[i + 2][e] = y1 * sn[e] + y2 * cs[e];
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<u32x2 *>(rowp + (16 * i + 4 * fg) * 2) =
              u32x2{pack_bf(v[i][0], v[i][1]), pack_bf(v[i][2], v[i][3])};
      } else if (SWIGLU) {
        // silu(g) = g / (1 + e^-g) as g times the hardware reciprocal (1 ulp) instead of the IEEE division: the
        // epilogue's VALU work is on this product's critical path (the product ~5% faster at the prefill shape);
        // 0.007% of the outputs then differ from the division's by one bf16 ulp
        // qa.raw: the gate | up product rows [M, 2 N] as the plain product stores them (the backward's operand)
        const int64_t grow = qrow0 + 16 * j + fr;
        const bool keep = qa.raw != nullptr && grow < M && qcol0 < N;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float o[4], gt4[4], up4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gt = round_bf(acc[i][j][e]);
            const float up = round_bf(acc[i + 2][j][e]);
            gt4[e] = gt;
            up4[e] = up;
            o[e] = round_bf(gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt))) * up;
          }
          *reinterpret_cast<u32x2 *>(rowp + (16 * i + 4 * fg) * 2) = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
          if (keep) {
            bf16_t *gr = qa.raw + grow * (2 * static_cast<int64_t>(N)) + qcol0 + 16 * i + 4 * fg;
            *reinterpret_cast<u32x2 *>(gr) = u32x2{pack_bf(gt4[0], gt4[1]), pack_bf(gt4[2], gt4[3])};
            *reinterpret_cast<u32x2 *>(gr + N) = u32x2{pack_bf(up4[0], up4[1]), pack_bf(up4[2], up4[3])};
          }
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
    // GB_QKV with a cache: the cache row and position of the quadrant's 128 rows, one pair of rows per lane (rows
    // lane and 64 + lane), handed to the lane that stores a row's chunk by a lane shuffle below
    int cs_lo = 0, cs_hi = 0, cp_lo = 0, cp_hi = 0;
    if (QKV && (qcol0 >> 6) >= qa.H && qa.kc != nullptr) {
      const int64_t r0 = min(qrow0 + pass * PASS_ROWS + lane, M - 1), r1 = min(qrow0 + pass * PASS_ROWS + 64 + lane, M - 1);
      cs_lo = qa.seq[r0];
      cp_lo = qa.pos[r0];
      cs_hi = qa.seq[r1];
      cp_hi = qa.pos[r1];
    }
    // same wavefront reads back (LDS keeps a wavefront's accesses in order): chunk id -> (row, chunk)
#pragma unroll
    for (int it = 0; it < PASS_ROWS * CPR / 64; ++it) {
      const int id = it * 64 + lane;
      const int r = id / CPR, c = id % CPR;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + r * PITCH + c * 16);
      const int64_t row = qrow0 + pass * PASS_ROWS + r;
      const int col = qcol0 + c * (16 / ESZ);
      if (QKV) {
        const int hd = qcol0 >> 6;  // c: the 16-byte chunk (8 columns) of the head
        // (every lane takes part in the shuffles, before any lane leaves the iteration; r < 64 is fixed per it)
        const bool lo_half = it * 64 / CPR < 64;
        const int64_t sq = __shfl(lo_half ? cs_lo : cs_hi, r & 63, 64);
        const int64_t ps = __shfl(lo_half ? cp_lo : cp_hi, r & 63, 64);
        if (row >= M || hd >= qa.H + 2 * qa.HKV) continue;
        if (hd < qa.H) {
          *reinterpret_cast<u32x4 *>(qa.q + row * qa.q_ld + hd * 64 + 8 * c) = v;
          continue;
        }
        const bool is_k = hd < qa.H + qa.HKV;
        const int hk = is_k ? hd - qa.H : hd - qa.H - qa.HKV;
        bf16_t *cdst = is_k ? qa.kc : qa.vc;
        if (cdst != nullptr) {
          if (sq >= 0 && sq < qa.cache_rows && ps >= 0 && ps < qa.cache_len)
            *reinterpret_cast<u32x4 *>(cdst + sq * qa.stride_cb + ps * qa.stride_cs + hk * 64 + 8 * c) = v;
        }
        bf16_t *odst = is_k ? qa.ko : qa.vo;
        if (odst != nullptr) *reinterpret_cast<u32x4 *>(odst + row * qa.kv_ld + hk * 64 + 8 * c) = v;
        continue;
      }
      // non-temporal: the product's rows are read back by a later kernel, not by this one, and stores that
      // allocate in L2 would push out the A blocks the XCD's next column tiles read
      if (row < M && col < N)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(static_cast<char *>(y) + (row * N + col) * ESZ));
    }
  }
}

template <int EPI, int GW>
static int launch_big_gw(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, const GbQkv &qa,
                         hipStream_t s) {
  using SH = GbShape<GW>;
  VK_RAISE_LDS_ONCE((gemm_big_kernel<EPI, GW>), SH::SMEM, "linear");
  constexpr int OUT_COLS = EPI == GB_SWIGLU ? 32 * GW : 64 * GW;
  const int tiles_n = (N + OUT_COLS - 1) / OUT_COLS;
  const int64_t tiles_m = (M + GB_BM - 1) / GB_BM;
  const int64_t total = tiles_m * tiles_n;
  if (total >= (int64_t(1) << 31)) return fail(VK_ERR_ARG, "linear: too many tiles");
  gemm_big_kernel<EPI, GW><<<static_cast<unsigned>(total), 128 * GW, SH::SMEM, s>>>(x, w, y, M, N, K, tiles_n,
                                                                                    static_cast<int>(total), qa);
  return VK_OK;
}

// 256 x 256 tiles where they measured faster (same bits either way, M = 131136 and 4096): bf16 outputs at every K
// (K 512 / 1536 / 2048: 8 / 4 / 10% faster) and fp32 outputs from K = 1024 (3 / 10% at 1536 / 2048, 1.5% slower at
// 512). The SwiGLU, residual and Wqkv epilogues run 2-8% slower on them: with one workgroup per CU their epilogue
// no longer overlaps another workgroup's K loop.
template <int EPI>
static int launch_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, const GbQkv &qa,
                      hipStream_t s) {
  const bool wide = EPI == GB_BF16 || (EPI == GB_F32 && K >= 1024);
  if (wide) return launch_big_gw<EPI, 4>(x, w, y, M, N, K, qa, s);
  return launch_big_gw<EPI, 2>(x, w, y, M, N, K, qa, s);
}

// Entry used by vk_linear for large M and by vk_gemm_rows (K % 64 == 0: an even number of K slices; N % 8 == 0:
// whole 16-byte output chunks).
int gemm_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, bool swiglu, bool out_f32,
             hipStream_t s) {
  const GbQkv none{};
  if (swiglu) return launch_big<GB_SWIGLU>(x, w, y, M, N, K, none, s);
  if (out_f32) return launch_big<GB_F32>(x, w, y, M, N, K, none, s);
  return launch_big<GB_BF16>(x, w, y, M, N, K, none, s);
}

// The SwiGLU product that also stores its gate | up rows [M, 2 N] to gu (for vk_linear's gu_out).
int gemm_big_swiglu_keep(const bf16_t *x, const bf16_t *w, void *y, bf16_t *gu, int64_t M, int N, int K,
                         hipStream_t s) {
  GbQkv keep{};
  keep.raw = gu;
  return launch_big<GB_SWIGLU>(x, w, y, M, N, K, keep, s);
}

}  // namespace vk

using namespace vk;

extern "C" int vk_linear_qkv_rope(const void *x, const void *w, int64_t M, int32_t K, const void *q_norm_w,
                                  const void *k_norm_w, int32_t norm_w_dtype, float eps, const void *cos_t, const void *sin_t,
                                  int32_t table_dtype, int64_t table_rows, const int32_t *pos, const int32_t *rope_pos,
                                  const int32_t *seq, void *q, int64_t q_ld, void *k_cache, void *v_cache,
                                  int64_t stride_cb, int64_t stride_cs, int64_t cache_rows, int64_t cache_len,
                                  void *k_out, void *v_out, int64_t kv_ld, void *qkv_out, int32_t n_heads,
                                  int32_t n_kv_heads, int32_t head_dim, void *stream) {
  VK_CHECK_ARG(x && w && cos_t && sin_t && q, "linear_qkv_rope: null pointer");
  VK_CHECK_ARG(head_dim == 64, "linear_qkv_rope: built for head_dim 64 (got %d)", head_dim);
  VK_CHECK_ARG(n_heads > 0 && n_kv_heads > 0, "linear_qkv_rope: bad head counts");
  const int N = 64 * (n_heads + 2 * n_kv_heads);
  VK_CHECK_ARG(M >= 0 && K > 0 && K % 64 == 0, "linear_qkv_rope: need K %% 64 == 0");
  VK_CHECK_ARG(M < (int64_t(1) << 31) / 256 * 256, "linear_qkv_rope: M too large");
  VK_CHECK_ARG((q_norm_w == nullptr) == (k_norm_w == nullptr), "linear_qkv_rope: q and k norm weights go together");
  VK_CHECK_ARG(table_dtype == VK_DTYPE_BF16 || table_dtype == VK_DTYPE_F32, "linear_qkv_rope: bad table dtype");
  VK_CHECK_ARG(norm_w_dtype == VK_DTYPE_BF16 || norm_w_dtype == VK_DTYPE_F32, "linear_qkv_rope: bad norm weight dtype");
  VK_CHECK_ARG(norm_w_dtype == VK_DTYPE_BF16 || table_dtype == VK_DTYPE_F32,
               "linear_qkv_rope: fp32 norm weights go with fp32 rotary tables");
  VK_CHECK_ARG(q_norm_w == nullptr || norm_w_dtype == VK_DTYPE_BF16 || (vk_aligned16(q_norm_w) && vk_aligned16(k_norm_w)),
               "linear_qkv_rope: fp32 norm weights must be 16-byte aligned");
  VK_CHECK_ARG(table_rows > 0 && (pos != nullptr || rope_pos != nullptr), "linear_qkv_rope: rotary positions");
  VK_CHECK_ARG((k_cache == nullptr) == (v_cache == nullptr), "linear_qkv_rope: k_cache and v_cache go together");
  VK_CHECK_ARG(k_cache == nullptr || (seq != nullptr && pos != nullptr), "linear_qkv_rope: cache writes need seq and pos");
  VK_CHECK_ARG((k_out == nullptr) == (v_out == nullptr), "linear_qkv_rope: k_out and v_out go together");
  VK_CHECK_ARG(q_ld % 8 == 0 && kv_ld % 8 == 0 && stride_cb % 8 == 0 && stride_cs % 8 == 0,
               "linear_qkv_rope: row strides must be multiples of 8 elements");
  VK_CHECK_ARG(vk_aligned16(cos_t) && vk_aligned16(sin_t), "linear_qkv_rope: rotary tables must be 16-byte aligned");
  VK_CHECK_ARG(qkv_out == nullptr || vk_aligned16(qkv_out), "linear_qkv_rope: qkv_out must be 16-byte aligned");
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(q) && (k_cache == nullptr || (vk_aligned16(k_cache) &&
               vk_aligned16(v_cache))) && (k_out == nullptr || (vk_aligned16(k_out) && vk_aligned16(v_out))),
               "linear_qkv_rope: pointers must be 16-byte aligned");
  if (M == 0) return VK_OK;
  GbQkv qa;
  qa.qw = q_norm_w;
  qa.kw = k_norm_w;
  qa.eps = eps;
  qa.cos_t = cos_t;
  qa.sin_t = sin_t;
  qa.table_f32 = table_dtype == VK_DTYPE_F32;
  qa.table_rows = table_rows;
  qa.pos = pos;
  qa.rope_pos = rope_pos;
  qa.seq = seq;
  qa.q = static_cast<bf16_t *>(q);
  qa.q_ld = q_ld;
  qa.kc = static_cast<bf16_t *>(k_cache);
  qa.vc = static_cast<bf16_t *>(v_cache);
  qa.stride_cb = stride_cb;
  qa.stride_cs = stride_cs;
  qa.cache_rows = cache_rows;
  qa.cache_len = cache_len;
  qa.ko = static_cast<bf16_t *>(k_out);
  qa.vo = static_cast<bf16_t *>(v_out);
  qa.kv_ld = kv_ld;
  qa.raw = static_cast<bf16_t *>(qkv_out);
  qa.H = n_heads;
  qa.HKV = n_kv_heads;
  qa.resid_in = nullptr;
  const auto xb = static_cast<const bf16_t *>(x), wb = static_cast<const bf16_t *>(w);
  const int rc = norm_w_dtype == VK_DTYPE_F32 ? launch_big<GB_QKV_W32>(xb, wb, nullptr, M, N, K, qa, VK_STREAM(stream))
                 : qa.table_f32               ? launch_big<GB_QKV>(xb, wb, nullptr, M, N, K, qa, VK_STREAM(stream))
                                              : launch_big<GB_QKV_BF16>(xb, wb, nullptr, M, N, K, qa, VK_STREAM(stream));
  if (rc != VK_OK) return rc;
  return launch_status("linear_qkv_rope");
}

extern "C" int vk_linear_residual_big(const void *a, const void *w, void *x, int32_t x_dtype, int64_t M, int32_t N,
                                      int32_t K, const float *bias, float alpha, float *ss_out, const void *x_in,
                                      void *stream) {
  VK_CHECK_ARG(a && w && x && ss_out, "linear_residual_big: null pointer");
  VK_CHECK_ARG(x_in == nullptr || vk_aligned16(x_in), "linear_residual_big: x_in must be 16-byte aligned");
  VK_CHECK_ARG(x_dtype == VK_DTYPE_BF16 || x_dtype == VK_DTYPE_F32, "linear_residual_big: bad residual dtype");
  VK_CHECK_ARG(M >= 0 && N > 0 && N % 128 == 0 && K > 0 && K % 64 == 0,
               "linear_residual_big: need N %% 128 == 0 and K %% 64 == 0 (N=%d K=%d)", N, K);
  VK_CHECK_ARG(M < (int64_t(1) << 31) / 256 * 256, "linear_residual_big: M too large");
  VK_CHECK_ARG(vk_aligned16(a) && vk_aligned16(w) && vk_aligned16(x) && (bias == nullptr || vk_aligned16(bias)),
               "linear_residual_big: pointers must be 16-byte aligned");
  if (M == 0) return VK_OK;
  GbQkv qa{};
  qa.bias = bias;
  qa.alpha = alpha;
  qa.ss_out = ss_out;
  qa.resid_in = x_in;
  const auto ab = static_cast<const bf16_t *>(a), wb = static_cast<const bf16_t *>(w);
  const int rc = x_dtype == VK_DTYPE_F32 ? launch_big<GB_RESID_F32>(ab, wb, x, M, N, K, qa, VK_STREAM(stream))
                                         : launch_big<GB_RESID>(ab, wb, x, M, N, K, qa, VK_STREAM(stream));
  if (rc != VK_OK) return rc;
  return launch_status("linear_residual_big");
}
