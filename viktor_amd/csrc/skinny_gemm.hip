// Small-M GEMMs of a decode step (one row per sequence, M = batch) with the surrounding elementwise
// work fused in, so a decoder layer is five launches:
//   norm_qkv_rope   rmsnorm(x) (or embedding gather + rmsnorm) -> x Wqkv^T -> QK-norm + RoPE -> q out,
//                   k / v written to the KV cache                     (add_rmsnorm + linear + qkv_rope_cache)
//   linear_residual x += bf16(a W^T)                                  (o / down projection + residual add)
//   norm_linear     act(rmsnorm(x) W^T), act = SwiGLU / none           (mlp norm + gate_up + SwiGLU)
// Rounding points are those of the unfused reference path (viktor/triton_ops.py, viktor/fast_decoder.py:
// 33-60): the normalised activations, the GEMM outputs, the residual sum, and each QK-norm / RoPE step
// are rounded to bf16 exactly where the unfused ops store bf16.
//
// MI355X design: a workgroup owns a 32 x BN output tile and its WAVES wavefronts split K (each a
// contiguous K slice), so a launch has (N / BN) x (M / 32) workgroups of short dependency chains:
// every wave issues all its A and B fragment loads (16-byte, straight from global / L2 into MFMA
// registers) before its first v_mfma_f32_16x16x32_bf16; partial tiles are summed through LDS in a
// fixed wave order (deterministic), and the epilogue runs on the summed tile with 8 lanes per row.
#include <math.h>

#include "common.h"

namespace vk {

// PRO_NORM_SS: RMSNorm with the row sums of squares handed over by the residual GEMM that produced x.
// PRO_EMBED_RES: the embedding gather + RMSNorm with the rows resident in LDS (the panel kernel's form of
// PRO_EMBED_NORM).
enum Prologue { PRO_NONE = 0, PRO_NORM = 1, PRO_EMBED_NORM = 2, PRO_NORM_SS = 3, PRO_EMBED_RES = 4 };
enum Epilogue { EPI_BF16 = 0, EPI_F32 = 1, EPI_SWIGLU = 2, EPI_RESID = 3, EPI_ROPE = 4 };

struct SkinnyArgs {
  const bf16_t *a;       // A [M, K]; PRO_EMBED_NORM: the embedding table [vocab, K]
  const int64_t *tok;    // PRO_EMBED_NORM: token ids [M]
  int64_t vocab;
  const bf16_t *norm_w;  // PRO_NORM / PRO_EMBED_NORM: RMSNorm weight [K]
  float eps;
  bf16_t *x_store;       // PRO_EMBED_NORM / _RES: gathered rows are stored here (the residual stream) [M, K]
  const bf16_t *w;       // weights [N, K] ([2N, K] gate | up for EPI_SWIGLU)
  void *y;               // output [M, N] (EPI_RESID: the residual, updated in place)
  int64_t M;
  int N, K;
  // EPI_ROPE: heads of 64 columns: q heads 0..H-1, k heads, v heads
  const bf16_t *qw, *kw;
  const void *cos_t, *sin_t;
  int table_f32;
  int64_t table_rows;
  const int32_t *pos, *rope_pos, *seq;
  bf16_t *kc, *vc;
  int64_t stride_cb, stride_cs, cache_rows, cache_len;
  int H, HKV;
  // EPI_RESID: per-row partial sums of squares of the updated residual, one per 32-column block
  // ([M, N / 32] fp32, N = 512; NULL: none). PRO_NORM_SS: those sums for the A rows ([M, K / 32], K = 512).
  float *ss_out;
  const float *ss_in;
#ifdef VK_PHASE_STAMPS
  uint64_t *stamps;  // the profiling build's per-workgroup phase timestamps (8 slots each; null: none)
#endif
};

constexpr int SK_BM = 32;

// Phase timestamps of the profiling build (compiled with VK_PHASE_STAMPS; the product library has none): lane 0
// of wave 0 of every workgroup writes the 100 MHz real-time counter to slot k of its 8: 0 entry, 1 first operands
// landed, 2 K loop start, 3 K loop end, 4 epilogue start (the tile summed in LDS), 5 end (its own stores done).
#ifdef VK_PHASE_STAMPS
#define VK_PHASE(p, k)                                                                      \
  do {                                                                                      \
    if ((p).stamps && threadIdx.x == 0) (p).stamps[8 * blockIdx.x + (k)] = wall_clock64(); \
  } while (0)
#define VK_PHASE_END(p)            \
  do {                             \
    __builtin_amdgcn_s_waitcnt(0); \
    VK_PHASE(p, 5);                \
  } while (0)
#else
#define VK_PHASE(p, k) \
  do {                 \
  } while (0)
#define VK_PHASE_END(p) \
  do {                  \
  } while (0)
#endif

// LDS writes of this wave done, then a plain s_barrier: __syncthreads() would also drain every
// outstanding global load (its release fence), the prefetched operands and epilogue data included.
// Builtins, not inline asm: the compiler's wait analysis treats an asm statement as unknown memory
// traffic and would then drain all loads before later LDS reads.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt / expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int BN, int WAVES, int KSTEPS, int PRO, int EPI>
__global__ __launch_bounds__(WAVES * 64) void skinny_gemm_kernel(const SkinnyArgs p) {
  static_assert(WAVES >= 4, "the epilogue maps 256 threads to 32 rows x 8 column groups");
  static_assert(BN == 32 || BN == 64, "BN is 32 or 64 columns");
  constexpr bool SWI = EPI == EPI_SWIGLU;
  constexpr bool ROPE = EPI == EPI_ROPE;
  constexpr int NT = BN / 16;            // n tiles of one operand group
  constexpr int NB = SWI ? 2 * BN : BN;  // output columns accumulated (gate + up for SwiGLU)
  constexpr int NTT = NB / 16;
  constexpr int HALVES = BN / 32;        // 32-column halves of the epilogue
  static_assert(!ROPE || BN == 64, "the rope epilogue works on whole 64-column heads");
  __shared__ float part[WAVES][SK_BM][NB + 1];
  __shared__ float ssq[WAVES][SK_BM];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * SK_BM;
  const int n0 = blockIdx.x * BN;
  const int K = p.K;
  const int kb = wid * KSTEPS * 32;  // this wave's K slice
  const int fr = lane & 15, fk = (lane >> 4) * 8;

  // epilogue mapping: thread tid < 256 -> row m0 + tid / 8 and columns 4 (tid % 8) .. + 3 of each half
  const int rr = (tid >> 3) & (SK_BM - 1), sub = tid & 7;
  const int64_t erow = m0 + rr;
  const bool row_ok = tid < SK_BM * 8 && erow < p.M;

  // ---- every load that does not depend on a result is issued first, in this order: RoPE positions,
  // A, norm weight, B, epilogue data; the compiler's counted waits then only hold for what is used.
  int64_t e_pos = 0, e_seq = 0, rp = 0;
  if constexpr (ROPE) {
    if (row_ok) {
      e_pos = p.pos[erow];
      e_seq = p.seq[erow];
      rp = p.rope_pos ? p.rope_pos[erow] : e_pos;
    }
  }
  u32x4 af[KSTEPS][2];
  const bf16_t *arow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int64_t row = m0 + 16 * i + fr;
    row = row < p.M ? row : p.M - 1;
    if (PRO == PRO_EMBED_NORM) {
      int64_t t = p.tok[row];
      t = (t < 0 || t >= p.vocab) ? 0 : t;
      arow[i] = p.a + t * K;
    } else {
      arow[i] = p.a + row * K;
    }
  }
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i) af[s][i] = *reinterpret_cast<const u32x4 *>(arow[i] + kb + 32 * s + fk);
  u32x4 nwf[PRO != PRO_NONE ? KSTEPS : 1];
  if constexpr (PRO != PRO_NONE) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) nwf[s] = *reinterpret_cast<const u32x4 *>(p.norm_w + kb + 32 * s + fk);
  }
  u32x4 bfr[KSTEPS][NTT];
#pragma unroll
  for (int j = 0; j < NTT; ++j) {
    int col = n0 + 16 * (j % NT) + fr;
    col = col < p.N ? col : p.N - 1;
    const int wrow = (SWI && j >= NT) ? col + p.N : col;
    const bf16_t *src = p.w + static_cast<int64_t>(wrow) * K + kb + fk;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) bfr[s][j] = *reinterpret_cast<const u32x4 *>(src + 32 * s);
  }
  asm volatile("" ::: "memory");
  // residual values this thread adds to (EPI_RESID) / the QK-norm weights and RoPE table entries of its
  // columns (EPI_ROPE, addressed by the positions loaded first)
  u32x2 old[HALVES];
  u32x2 wnf[2];
  f32x4 csf, snf;
  const int hd = n0 / 64;
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int hf = 0; hf < HALVES; ++hf) {
      old[hf] = u32x2{0u, 0u};
      const int col = n0 + 32 * hf + 4 * sub;
      if (row_ok && col < p.N) old[hf] = *reinterpret_cast<const u32x2 *>(static_cast<bf16_t *>(p.y) + erow * p.N + col);
    }
  }
  if constexpr (ROPE) {
    wnf[0] = wnf[1] = u32x2{0u, 0u};
    csf = snf = f32x4{0.f, 0.f, 0.f, 0.f};
    if (hd < p.H + p.HKV) {
      const bf16_t *wn = hd < p.H ? p.qw : p.kw;
      wnf[0] = *reinterpret_cast<const u32x2 *>(wn + 4 * sub);
      wnf[1] = *reinterpret_cast<const u32x2 *>(wn + 32 + 4 * sub);
      rp = rp < 0 ? 0 : (rp >= p.table_rows ? p.table_rows - 1 : rp);
      if (p.table_f32) {
        csf = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(p.cos_t) + rp * 32 + 4 * sub);
        snf = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(p.sin_t) + rp * 32 + 4 * sub);
      } else {
        const u32x2 c2 = *reinterpret_cast<const u32x2 *>(static_cast<const bf16_t *>(p.cos_t) + rp * 32 + 4 * sub);
        const u32x2 s2 = *reinterpret_cast<const u32x2 *>(static_cast<const bf16_t *>(p.sin_t) + rp * 32 + 4 * sub);
        csf = f32x4{lo_bf(c2[0]), hi_bf(c2[0]), lo_bf(c2[1]), hi_bf(c2[1])};
        snf = f32x4{lo_bf(s2[0]), hi_bf(s2[0]), lo_bf(s2[1]), hi_bf(s2[1])};
      }
    }
  }

  // ---- prologue: RMSNorm of the A rows over the full K (sum of squares across lanes and waves) ----
  if constexpr (PRO != PRO_NONE) {
    float ss[2] = {0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = lo_bf(af[s][i][e]), hi = hi_bf(af[s][i][e]);
          ss[i] += lo * lo + hi * hi;
        }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ss[i] += __shfl_xor(ss[i], 16, 64);
      ss[i] += __shfl_xor(ss[i], 32, 64);
    }
    if (lane < 16) {
      ssq[wid][fr] = ss[0];
      ssq[wid][16 + fr] = ss[1];
    }
    if (PRO == PRO_EMBED_NORM && blockIdx.x == 0) {
      // the gathered rows become the residual stream
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t row = m0 + 16 * i + fr;
        if (row < p.M) {
#pragma unroll
          for (int s = 0; s < KSTEPS; ++s)
            *reinterpret_cast<u32x4 *>(p.x_store + row * K + kb + 32 * s + fk) = af[s][i];
        }
      }
    }
    lds_barrier();
    float r[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) t += ssq[w][16 * i + fr];
      r[i] = rsqrtf(t / static_cast<float>(K) + p.eps);
    }
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          af[s][i][e] = pack_bf(lo_bf(af[s][i][e]) * r[i] * lo_bf(nwf[s][e]), hi_bf(af[s][i][e]) * r[i] * hi_bf(nwf[s][e]));
  }

  // ---- MFMA over this wave's K slice ----
  f32x4 acc[2][NTT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NTT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NTT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[s][i]),
                                                            __builtin_bit_cast(bf16x8, bfr[s][j]), acc[i][j], 0, 0, 0);

  // ---- split-K reduction through LDS ----
  {
    const int oc = lane & 15, orow = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NTT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[wid][16 * i + orow + e][16 * j + oc] = acc[i][j][e];
  }
  lds_barrier();
  if (tid >= SK_BM * 8) return;

  // ---- epilogue: thread -> (row rr, 8-lane group sub); columns {4 sub .. 4 sub + 3} of each half ----
  float v[HALVES][4];
  float vu[HALVES][4];
#pragma unroll
  for (int hf = 0; hf < HALVES; ++hf)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = 32 * hf + 4 * sub + c;
      float sacc = 0.f, uacc = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        sacc += part[w][rr][col];
        if (SWI) uacc += part[w][rr][BN + col];
      }
      v[hf][c] = sacc;
      vu[hf][c] = uacc;
    }
  if constexpr (ROPE) {
    const int H = p.H, HKV = p.HKV;
    float x1[4], x2[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      x1[c] = round_bf(v[0][c]);
      x2[c] = round_bf(v[1][c]);
    }
    if (hd < H + HKV) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) ss += x1[c] * x1[c] + x2[c] * x2[c];
      ss += __shfl_xor(ss, 1, 64);
      ss += __shfl_xor(ss, 2, 64);
      ss += __shfl_xor(ss, 4, 64);
      const float r = rsqrtf(ss / 64.f + p.eps);
      const float w1[4] = {lo_bf(wnf[0][0]), hi_bf(wnf[0][0]), lo_bf(wnf[0][1]), hi_bf(wnf[0][1])};
      const float w2[4] = {lo_bf(wnf[1][0]), hi_bf(wnf[1][0]), lo_bf(wnf[1][1]), hi_bf(wnf[1][1])};
      float a1[4], a2[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float y1 = round_bf(x1[c] * r * w1[c]);
        const float y2 = round_bf(x2[c] * r * w2[c]);
        a1[c] = y1 * csf[c] - y2 * snf[c];
        a2[c] = y1 * snf[c] + y2 * csf[c];
      }
      const u32x2 o1 = u32x2{pack_bf(a1[0], a1[1]), pack_bf(a1[2], a1[3])};
      const u32x2 o2 = u32x2{pack_bf(a2[0], a2[1]), pack_bf(a2[2], a2[3])};
      if (row_ok) {
        if (hd < H) {
          bf16_t *dst = static_cast<bf16_t *>(p.y) + (erow * H + hd) * 64 + 4 * sub;
          *reinterpret_cast<u32x2 *>(dst) = o1;
          *reinterpret_cast<u32x2 *>(dst + 32) = o2;
        } else if (e_seq >= 0 && e_seq < p.cache_rows && e_pos >= 0 && e_pos < p.cache_len) {
          bf16_t *dst = p.kc + e_seq * p.stride_cb + e_pos * p.stride_cs + (hd - H) * 64 + 4 * sub;
          *reinterpret_cast<u32x2 *>(dst) = o1;
          *reinterpret_cast<u32x2 *>(dst + 32) = o2;
        }
      }
    } else if (row_ok && e_seq >= 0 && e_seq < p.cache_rows && e_pos >= 0 && e_pos < p.cache_len) {
      // v head: the rounded projection goes to the cache unchanged
      bf16_t *dst = p.vc + e_seq * p.stride_cb + e_pos * p.stride_cs + (hd - H - HKV) * 64 + 4 * sub;
      *reinterpret_cast<u32x2 *>(dst) = u32x2{pack_bf(x1[0], x1[1]), pack_bf(x1[2], x1[3])};
      *reinterpret_cast<u32x2 *>(dst + 32) = u32x2{pack_bf(x2[0], x2[1]), pack_bf(x2[2], x2[3])};
    }
    return;
  }
  if (!row_ok) return;
#pragma unroll
  for (int hf = 0; hf < HALVES; ++hf) {
    const int col = n0 + 32 * hf + 4 * sub;
    if (col >= p.N) continue;  // N is a multiple of 4 (checked on the host)
    const int64_t off = erow * p.N + col;
    if (EPI == EPI_F32) {
      *reinterpret_cast<f32x4 *>(static_cast<float *>(p.y) + off) = f32x4{v[hf][0], v[hf][1], v[hf][2], v[hf][3]};
    } else {
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float val = v[hf][c];
        if (EPI == EPI_SWIGLU) {
          const float g = round_bf(val);
          const float u = round_bf(vu[hf][c]);
          val = round_bf(g / (1.0f + __expf(-g))) * u;
        }
        o[c] = val;
      }
      if (EPI == EPI_RESID) {
        o[0] = lo_bf(old[hf][0]) + round_bf(o[0]);
        o[1] = hi_bf(old[hf][0]) + round_bf(o[1]);
        o[2] = lo_bf(old[hf][1]) + round_bf(o[2]);
        o[3] = hi_bf(old[hf][1]) + round_bf(o[3]);
      }
      *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(p.y) + off) = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
    }
  }
}

// ---- panel kernel: the K dimension streamed through an LDS ring --------------------------------------
//
// A workgroup (4 waves) owns 32 rows x 64 output columns (64 gate + 64 up weight rows for SwiGLU) over the
// whole K. K advances in 64-wide stages through a 3- or 4-slot LDS ring filled by direct global->LDS loads
// (global_load_lds_dwordx4: lane l of an instruction lands at slot base + 16 l), so two or three stages
// are in flight while one feeds the MFMAs and the prefetch costs no registers. An LDS row is 128 bytes (64 K
// values); the 16-byte chunk c of row r sits in slot c ^ ((r >> 1) & 7), which spreads the 16 rows of every
// fragment read over all 16 bank groups. The product is formed transposed (the weight fragment is the MFMA
// A operand), the tile is handed to the epilogue through LDS, and the epilogue is the one above with the
// same rounding points. RMSNorm: the sums of squares come from a pre-pass over the workgroup's rows issued
// before the ring; each fragment is normalised (bf16(x / rms * w)) as it is read.
constexpr int PG_BM = 32;
constexpr int PG_BN = 64;
constexpr int PG_BK = 64;
constexpr int PG_ROWB = PG_BK * 2;
constexpr int PG_NORM_K = 512;  // the RMSNorm prologue is built for K = 512 (d_model)
constexpr int PG_SS_COLS = 32;  // columns per handed-over partial sum of squares
constexpr int PG_SS_N = PG_NORM_K / PG_SS_COLS;  // partials per row (16)

// s_waitcnt immediate: vmcnt <= n, expcnt / lgkmcnt unconstrained (gfx9 encoding: vmcnt[3:0] bits 3:0,
// vmcnt[5:4] bits 15:14, expcnt bits 6:4, lgkmcnt bits 11:8)
constexpr int pg_vmcnt(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

typedef __attribute__((address_space(3))) void lds_void_t;

// one stage of the ring: this wave's LOADS direct-load instructions (instruction q = wid + NWAVES j -> 1 KB at
// base + 1024 q). A device function rather than a lambda: with a lambda around the builtin, the host pass
// drops the kernel's launch stub.
template <int LOADS, int NWAVES = 4>
__device__ __forceinline__ void pg_issue(char *base, const bf16_t *const *src, int k0, int wid) {
#pragma unroll
  for (int j = 0; j < LOADS; ++j)
    __builtin_amdgcn_global_load_lds(src[j] + k0, (lds_void_t *)(base + (wid + NWAVES * j) * 1024), 16, 0, 0);
}

// One 16-byte direct global->LDS load per lane (a whole 1 KB row for a wave); a device function for the
// same reason as pg_issue: the builtin written in the kernel body also drops the launch stub.
__device__ __forceinline__ void pg_issue_row(char *dst, const bf16_t *src) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t *)dst, 16, 0, 0);
}
// The same with 4 bytes per lane (lane l lands at dst + 4 l).
__device__ __forceinline__ void pg_issue_dword(char *dst, const int32_t *src) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t *)dst, 4, 0, 0);
}

// Wait until at most `ahead` stages of this wave's direct loads (LOADS instructions each) are outstanding.
// s_waitcnt takes an immediate, so one branch per count (ahead is wave-uniform).
template <int LOADS, int MAXA>
__device__ __forceinline__ void pg_wait_ahead(int ahead) {
  if constexpr (MAXA >= 1) {
    if (ahead >= MAXA) {
      __builtin_amdgcn_s_waitcnt(pg_vmcnt(MAXA * LOADS));
      return;
    }
    pg_wait_ahead<LOADS, MAXA - 1>(ahead);
  } else {
    __builtin_amdgcn_s_waitcnt(pg_vmcnt(0));
  }
}

// RMSNorm of a resident A tile in place (rows of K = 512 bf16, chunk c of row r in slot c ^ (r & 15)) from
// the row sums of squares handed over by the producing residual product (ssx: [rows][16] fp32 in LDS, one per
// 32 columns) and the norm weight (nwx: 512 bf16 in LDS): x = bf16(x * (1 / rms) * w), 1 / rms =
// rsqrt(sum / 512 + eps) with the row's 16 partials summed pairwise in a fixed order. This wave takes rows r = wid + RSTEP i (i < NR), a whole 1 KB row
// per step (lane l takes slot l, conflict-free). Lane l first computes 1 / rms of row l, and a row's value is
// read from its lane; all rows' reads are issued before the first write, so the LDS round trips overlap
// (a read after a write to the same tile would wait for it).
template <int NR, int RSTEP>
__device__ __forceinline__ void pg_normalise_rows(char *tile, const char *nwx, const char *ssx, int rows, int wid,
                                                  int lane, float eps) {
  const int lr = lane < rows ? lane : 0;
  float s4[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(ssx + PG_SS_N * 4 * lr + 16 * q);
    s4[q] = (v[0] + v[1]) + (v[2] + v[3]);
  }
  const float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  const float rn_lane = rsqrtf(ss * (1.0f / PG_NORM_K) + eps);
  u32x4 xr[NR], wr[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = wid + RSTEP * i;
    xr[i] = *reinterpret_cast<const u32x4 *>(tile + r * (PG_NORM_K * 2) + 16 * lane);
    wr[i] = *reinterpret_cast<const u32x4 *>(nwx + 16 * (lane ^ (r & 15)));
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = wid + RSTEP * i;
    const float rn = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rn_lane), r));
    u32x4 xn;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      xn[e] = pack_bf(lo_bf(xr[i][e]) * rn * lo_bf(wr[i][e]), hi_bf(xr[i][e]) * rn * hi_bf(wr[i][e]));
    *reinterpret_cast<u32x4 *>(tile + r * (PG_NORM_K * 2) + 16 * lane) = xn;
  }
}

// The same normalisation with each row's sum of squares taken from the tile itself (the embedding rows of
// the first layer have none handed over): a row's 512 squares summed per lane, then across the wave in a
// fixed butterfly order. With store, the raw rows also go to x_store (the residual stream) first; chunk c of
// the row sits in slot c ^ (r & 15).
template <int NR, int RSTEP>
__device__ __forceinline__ void pg_normalise_rows_own(char *tile, const char *nwx, int wid, int lane, float eps,
                                                      bf16_t *x_store, int64_t m0, int64_t M, bool store) {
  u32x4 xr[NR], wr[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = wid + RSTEP * i;
    xr[i] = *reinterpret_cast<const u32x4 *>(tile + r * (PG_NORM_K * 2) + 16 * lane);
    wr[i] = *reinterpret_cast<const u32x4 *>(nwx + 16 * (lane ^ (r & 15)));
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = wid + RSTEP * i;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf(xr[i][e]), hi = hi_bf(xr[i][e]);
      ss += lo * lo + hi * hi;
    }
    ss = wave_sum(ss);
    const float rn = rsqrtf(ss * (1.0f / PG_NORM_K) + eps);
    const int64_t grow = m0 + r;
    if (store && grow < M)
      *reinterpret_cast<u32x4 *>(x_store + grow * PG_NORM_K + 8 * (lane ^ (r & 15))) = xr[i];
    u32x4 xn;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      xn[e] = pack_bf(lo_bf(xr[i][e]) * rn * lo_bf(wr[i][e]), hi_bf(xr[i][e]) * rn * hi_bf(wr[i][e]));
    *reinterpret_cast<u32x4 *>(tile + r * (PG_NORM_K * 2) + 16 * lane) = xn;
  }
}

template <int PRO, int EPI, int KS>
struct PanelShape {
  static constexpr bool SWI = EPI == EPI_SWIGLU;
  static constexpr bool XRES = PRO == PRO_NORM_SS || PRO == PRO_EMBED_RES;  // A resident in LDS (K = 512)
  static constexpr int WR = SWI ? 2 * PG_BN : PG_BN;  // weight rows per tile
  static constexpr int ROWS = (XRES ? 0 : PG_BM) + WR;  // LDS rows per ring stage
  static constexpr int STAGEB = ROWS * PG_ROWB;
  static constexpr int LOADS = ROWS / 8 / 4;          // direct-load instructions per wave per stage
  // ring depth: 4 slots (3 stages in flight) for 12 KB stages, 3 for the 20 KB SwiGLU stages (and for the
  // 16 KB SwiGLU weight stages beside a resident A tile), so two workgroups share a CU where the grid has
  // more workgroups than CUs. The K loop moves stages at the per-CU L2 -> LDS rate (about 90 GB/s, from
  // per-phase timestamps): 5 or 6 slots for the one-workgroup-per-CU K-split shapes measured no faster.
  static constexpr int STAGES = SWI ? 3 : 4;
  static constexpr int XB = XRES ? PG_BM * PG_NORM_K * 2 : 0;  // resident A tile: 32 rows x 1 KB
  static constexpr int PARTB = PG_BM * (WR + 1) * 4;
  static constexpr int RING = STAGES * STAGEB;  // one ring per K slice (KS slices)
  static constexpr int BODY = XB + KS * RING > PARTB ? XB + KS * RING : PARTB;
  // + the RMSNorm weight and row sums of the pre-pass variants
  static constexpr int SMEM = BODY + ((PRO == PRO_NORM || PRO == PRO_EMBED_NORM) ? PG_NORM_K * 2 + PG_BM * 4 : 0);
};

// KS = 2: 8 wavefronts, waves 0-3 take the first half of K and waves 4-7 the second, each half through
// its own ring; the two partial tiles are summed in LDS (fixed order) before the epilogue. This halves the
// latency chain of the K loop for the shapes with few workgroups (o / down / qkv projections).
//
// PRO_NORM_SS: the A tile (32 rows x K = 512) is loaded once into LDS (one direct load per row, chunk c of
// row r in slot c ^ (r & 15)), normalised in place in one pass -- 1 / rms from the row sums of squares the
// producing residual GEMM left, bf16(x / rms * w) -- and read from there; the ring carries only W.
template <int PRO, int EPI, int KS>
__global__ __launch_bounds__(256 * KS) void panel_gemm_kernel(const SkinnyArgs p, int m_blocks, int tiles) {
  static_assert(KS == 1 || (KS == 2 && (PRO == PRO_NONE || PRO == PRO_NORM_SS || PRO == PRO_EMBED_RES)),
                "K halves only without the pre-pass norm prologue");
  using S = PanelShape<PRO, EPI, KS>;
  static_assert(!S::XRES || S::STAGES - 1 <= PG_NORM_K / PG_BK / KS,
                "resident-A variants issue STAGES - 1 whole stages before the normalisation");
  static_assert(S::LOADS * (S::STAGES - 1) <= 63, "a wave's stages in flight must fit the vmcnt counter");
  constexpr bool XRES = S::XRES;
  constexpr bool SWI = S::SWI;
  constexpr bool ROPE = EPI == EPI_ROPE;
  constexpr int HALVES = 2;  // 64 output columns = two 32-column halves in the epilogue
  static_assert(S::ROWS % 32 == 0, "a stage is whole 8-row instructions for 4 waves");
  __shared__ __attribute__((aligned(16))) char smem[S::SMEM];

  VK_PHASE(p, 0);
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wq = wid & 3, kh = wid >> 2;  // wave within its K slice, K slice
  // XCD-aware tile order: workgroup p runs on XCD p % 8, which owns a contiguous range of tiles; tiles are
  // numbered n-block-major, so the workgroups of one XCD share weight tiles (a bijection for any count)
  const int pid = blockIdx.x, xcd = pid & 7, idx = pid >> 3;
  const int q8 = tiles >> 3, r8 = tiles & 7;
  const int tile = xcd * q8 + min(xcd, r8) + idx;
  const int nb = tile / m_blocks, mb = tile % m_blocks;
  const int64_t m0 = static_cast<int64_t>(mb) * PG_BM;
  const int n0 = nb * PG_BN;
  // K stays a run-time value (with the norm it is 512, checked on the host): with a constant trip count
  // the compiler unrolls the K loop, sees the ring offsets and drains every load before each LDS read
  const int K = p.K, nk = K / (PG_BK * KS), kbase = kh * (K / KS);
  const int fr = lane & 15, fg = lane >> 4;

  // epilogue mapping: thread -> row m0 + tid / 8, columns 4 (tid % 8) .. + 3 of each 32-column half
  const int rr = (tid >> 3) & (PG_BM - 1), sub = tid & 7;
  const int64_t erow = m0 + rr;
  const bool row_ok = tid < 256 && erow < p.M;

  // 1. RoPE positions (the table loads depend on them; XRES: staged in LDS below)
  int64_t e_pos = 0, e_seq = 0, rp = 0;
  if constexpr (ROPE && !XRES) {
    if (row_ok) {
      e_pos = p.pos[erow];
      e_seq = p.seq[erow];
      rp = p.rope_pos ? p.rope_pos[erow] : e_pos;
    }
  }
  // 2. A row pointers (embedding rows through the token ids)
  auto a_row = [&](int r) {
    int64_t row = m0 + r;
    row = row < p.M ? row : p.M - 1;
    if (PRO == PRO_EMBED_NORM || PRO == PRO_EMBED_RES) {
      int64_t t = p.tok[row];
      t = (t < 0 || t >= p.vocab) ? 0 : t;
      return p.a + t * K;
    }
    return p.a + row * K;
  };
  // 3. the ring: stage 0 and 1 in flight first. Instruction q (= wid + 4 j) of a stage covers LDS rows
  //    8 q .. 8 q + 7 (A rows first, then weight rows); lane l -> row 8 q + l / 8, slot l % 8, K chunk
  //    slot ^ ((row >> 1) & 7)
  const bf16_t *src[S::LOADS];
#pragma unroll
  for (int j = 0; j < S::LOADS; ++j) {
    const int q = wq + 4 * j;
    const int r = 8 * q + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    if (!XRES && r < PG_BM) {
      src[j] = a_row(r) + 8 * c + kbase;
    } else {
      const int wr = XRES ? r : r - PG_BM;
      int col = n0 + (SWI ? (wr & (PG_BN - 1)) : wr);
      col = col < p.N ? col : p.N - 1;
      const int wrow = (SWI && wr >= PG_BN) ? col + p.N : col;
      src[j] = p.w + static_cast<int64_t>(wrow) * K + 8 * c + kbase;
    }
  }
#define PG_ISSUE(stage) \
  pg_issue<S::LOADS>(smem + S::XB + kh * S::RING + ((stage) % S::STAGES) * S::STAGEB, src, (stage) * PG_BK, wq)
  // PRO_NORM_SS: the norm weight (1 KB) goes to the last slot of the first ring, which the K loop fills only
  // after the normalisation; every wave loads it (the same bytes) ahead of its tile rows, so the one counted
  // wait before the normalisation covers it. Register loads are kept out of this stretch: one consumed while
  // direct loads are in flight makes the compiler wait for all of them.
  // The tile's row sums of squares (32 rows x 16 fp32 = 2 KB) follow it there the same way: lane l of load h
  // brings quarter l % 4 of row 16 h + l / 4; and for RoPE the rows' int32 positions: [pos x 32 | seq x 32] and
  // [rope pos x 32 | again], 4 bytes per lane (rows past M read row M - 1; their results are not stored).
  char *const nwx = smem + S::XB + (S::STAGES - 1) * S::STAGEB;
  char *const ssx = nwx + PG_NORM_K * 2;
  char *const psx = ssx + PG_BM * PG_SS_N * 4;
  static_assert(!XRES || PG_NORM_K * 2 + PG_BM * PG_SS_N * 4 + 2 * 64 * 4 <= S::STAGEB, "staging fits one ring slot");
  if constexpr (XRES) {
    pg_issue_row(nwx, p.norm_w + 8 * lane);
#pragma unroll
    for (int h = 0; h < (PRO == PRO_NORM_SS ? PG_BM * PG_SS_N * 4 / 1024 : 0); ++h) {
      int64_t srow = m0 + 16 * h + (lane >> 2);
      srow = srow < p.M ? srow : p.M - 1;
      pg_issue_row(ssx + 1024 * h, reinterpret_cast<const bf16_t *>(p.ss_in + srow * PG_SS_N + 4 * (lane & 3)));
    }
    if constexpr (ROPE) {
      int64_t prow = m0 + (lane & 31);
      prow = prow < p.M ? prow : p.M - 1;
      pg_issue_dword(psx, (lane < 32 ? p.pos : p.seq) + prow);
      pg_issue_dword(psx + 256, (p.rope_pos ? p.rope_pos : p.pos) + prow);
    }
  }
  if constexpr (XRES) {
    // the resident A tile next: row i of the tile is instruction i, issued by wave i % (4 KS)
#pragma unroll
    for (int i = 0; i < PG_BM / (4 * KS); ++i) {
      const int r = wid + 4 * KS * i;
      const int c = lane ^ (r & 15);
      pg_issue_row(smem + r * (PG_NORM_K * 2), a_row(r) + 8 * c);
    }
  }
  asm volatile("" ::: "memory");
  // (XRES: K = 512, so every one of these stages exists; issued without a branch, the compiler can count
  // the loads still in flight at the wait before the normalisation)
#pragma unroll
  for (int s = 0; s < S::STAGES - 1; ++s)
    if (XRES || s < nk) PG_ISSUE(s);
  asm volatile("" ::: "memory");

  // 4. RMSNorm (K = 512): wave w reads rows 8 w .. 8 w + 7; lane l owns row 8 w + l / 8 and the 64 K values
  //    at 64 (l % 8), so a row's sum of squares is a reduction over 8 lanes. These loads, and the norm
  //    weight staged to LDS, are consumed before the loop: inside it only LDS is read, so the counted waits
  //    on the ring are the only ones.
  // the norm weight and the row sums of squares sit in the ring's LDS block, past the ring: LDS accesses
  // to another object after a direct load make the compiler drain every load before them
  bf16_t *nws = reinterpret_cast<bf16_t *>(smem + S::BODY);
  float *rs = reinterpret_cast<float *>(smem + S::BODY + PG_NORM_K * 2);
  float rinv[1] = {1.f};
  if constexpr (PRO == PRO_NORM || PRO == PRO_EMBED_NORM) {
    const int pre_row = 8 * wid + (lane >> 3);
    const int pre_k = 64 * (lane & 7);
    u32x4 xv[8];
    const bf16_t *xr = a_row(pre_row) + pre_k;
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = *reinterpret_cast<const u32x4 *>(xr + 8 * j);
    const u32x4 nwv = *reinterpret_cast<const u32x4 *>(p.norm_w + 8 * lane);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lo_bf(xv[j][e]), hi = hi_bf(xv[j][e]);
        ss += lo * lo + hi * hi;
      }
    const int64_t grow = m0 + pre_row;
    if (PRO == PRO_EMBED_NORM && nb == 0 && grow < p.M) {  // the gathered rows become the residual stream
#pragma unroll
      for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4 *>(p.x_store + grow * K + pre_k + 8 * j) = xv[j];
    }
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 4, 64);
    if ((lane & 7) == 0) rs[pre_row] = ss;
    // every wave stores the (identical) weight: a load left unconsumed on some waves would make the
    // compiler drain all loads wherever its registers are reused
    *reinterpret_cast<u32x4 *>(nws + 8 * lane) = nwv;
    lds_barrier();
    rinv[0] = rsqrtf(rs[tid >> 3] / static_cast<float>(K) + p.eps);  // the row of this thread's chunk
  }

  // 4'. PRO_NORM_SS: normalise the resident A tile in place, a whole 1 KB row per wave and step (lane l takes
  //     slot l, conflict-free). 1 / rms comes from the row's 16 partial sums (one per 32 columns), summed in
  //     a fixed order. K = 512 (checked on the host), so the first STAGES - 1 ring stages were all issued:
  //     waiting until only their loads are outstanding retires this wave's weight, row sums and tile rows.
  if constexpr (XRES) {
    __builtin_amdgcn_s_waitcnt(pg_vmcnt(S::LOADS * (S::STAGES - 1)));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    VK_PHASE(p, 1);
    if constexpr (PRO == PRO_EMBED_RES)  // the gathered rows' own sums; the nb == 0 tiles keep the raw rows
      pg_normalise_rows_own<PG_BM / (4 * KS), 4 * KS>(smem, nwx, wid, lane, p.eps, p.x_store, m0, p.M, nb == 0);
    else
      pg_normalise_rows<PG_BM / (4 * KS), 4 * KS>(smem, nwx, ssx, PG_BM, wid, lane, p.eps);
    if constexpr (ROPE) {  // read before the barrier below, which retires them: the loop reuses the slot
      const int32_t *ps = reinterpret_cast<const int32_t *>(psx);
      e_pos = ps[rr];
      e_seq = ps[32 + rr];
      rp = ps[64 + rr];
    }
    lds_barrier();
  }

  // 5. epilogue data (consumed after the loop)
  u32x2 old[HALVES];
  u32x2 wnf[2];
  f32x4 csf, snf;
  u32x2 ctw[2], stw[2];  // the raw table words, widened in the epilogue (here it would wait for the loads)
  const int hd = n0 / 64;
  if constexpr (EPI == EPI_RESID) {
    // unconditional (row and column clamped; unused where out of range): a load under a branch makes the
    // compiler wait for every outstanding load, the ring's included, where its register is merged
    const int64_t orow = erow < p.M ? erow : p.M - 1;
#pragma unroll
    for (int hf = 0; hf < HALVES; ++hf) {
      int col = n0 + 32 * hf + 4 * sub;
      col = col < p.N ? col : p.N - 4;
      old[hf] = *reinterpret_cast<const u32x2 *>(static_cast<bf16_t *>(p.y) + orow * p.N + col);
    }
  }
  if constexpr (ROPE) {
    // without branches (loads in branches make the compiler wait for them at the join): v heads load the
    // q-norm weight and the tables too, unused; an fp32 table row is two 8-byte words, a bf16 row one (read
    // twice)
    const bf16_t *wn = hd < p.H ? p.qw : p.kw;
    wnf[0] = *reinterpret_cast<const u32x2 *>(wn + 4 * sub);
    wnf[1] = *reinterpret_cast<const u32x2 *>(wn + 32 + 4 * sub);
    rp = rp < 0 ? 0 : (rp >= p.table_rows ? p.table_rows - 1 : rp);
    const int64_t esz = p.table_f32 ? 4 : 2;
    const int64_t toff = (rp * 32 + 4 * sub) * esz, thi = p.table_f32 ? 8 : 0;
    const char *ct = static_cast<const char *>(p.cos_t) + toff, *st = static_cast<const char *>(p.sin_t) + toff;
    ctw[0] = *reinterpret_cast<const u32x2 *>(ct);
    ctw[1] = *reinterpret_cast<const u32x2 *>(ct + thi);
    stw[0] = *reinterpret_cast<const u32x2 *>(st);
    stw[1] = *reinterpret_cast<const u32x2 *>(st + thi);
  }
  // fragment byte offsets inside a stage: LDS row R, K chunk c -> R * 128 + 16 * (c ^ ((R >> 1) & 7))
  auto frag_off = [](int R, int c) { return R * PG_ROWB + 16 * (c ^ ((R >> 1) & 7)); };
  constexpr int NW = SWI ? 2 : 1;
  int woff[NW][2], xoff[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int wt = 0; wt < NW; ++wt)
      woff[wt][ks] = frag_off((XRES ? 0 : PG_BM) + wt * PG_BN + 16 * wq + fr, 4 * ks + fg);
#pragma unroll
    for (int t = 0; t < 2; ++t) xoff[t][ks] = frag_off(16 * t + fr, 4 * ks + fg);
  }
  f32x4 acc[NW][2];
#pragma unroll
  for (int wt = 0; wt < NW; ++wt)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[wt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (XRES) VK_PHASE(p, 2);
  for (int kt = 0; kt < nk; ++kt) {
    // this wave's loads of stage kt are done once at most (stages issued after it) x LOADS remain
    pg_wait_ahead<S::LOADS, S::STAGES - 2>(min(nk - 1 - kt, S::STAGES - 2));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (!XRES && kt == 0) {
      VK_PHASE(p, 1);
      VK_PHASE(p, 2);
    }
    if (kt + S::STAGES - 1 < nk) PG_ISSUE(kt + S::STAGES - 1);
    char *base = smem + S::XB + kh * S::RING + (kt % S::STAGES) * S::STAGEB;
    if constexpr (PRO == PRO_NORM || PRO == PRO_EMBED_NORM) {
      // RMSNorm of the stage's A tile in place, once per workgroup: thread t takes the 16-byte chunk in
      // slot t % 8 of row t / 8 (K chunk c = slot ^ ((row >> 1) & 7)) -> bf16(x / rms * w)
      const int row = tid >> 3, c = (tid & 7) ^ ((row >> 1) & 7);
      u32x4 *xc = reinterpret_cast<u32x4 *>(base + row * PG_ROWB + 16 * (tid & 7));
      const u32x4 xr = *xc;
      const u32x4 wv = *reinterpret_cast<const u32x4 *>(nws + kt * PG_BK + 8 * c);
      u32x4 xn;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xn[e] = pack_bf(lo_bf(xr[e]) * rinv[0] * lo_bf(wv[e]), hi_bf(xr[e]) * rinv[0] * hi_bf(wv[e]));
      *xc = xn;
      lds_barrier();
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 xf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if constexpr (XRES) {  // resident tile: row 16 t + fr, K chunk 8 (global stage) + 4 ks + fg
          const int c = 8 * (kh * nk + kt) + 4 * ks + fg;
          xf[t] = *reinterpret_cast<const u32x4 *>(smem + (16 * t + fr) * (PG_NORM_K * 2) + 16 * (c ^ fr));
        } else {
          xf[t] = *reinterpret_cast<const u32x4 *>(base + xoff[t][ks]);
        }
      }
#pragma unroll
      for (int wt = 0; wt < NW; ++wt) {
        const u32x4 wf = *reinterpret_cast<const u32x4 *>(base + woff[wt][ks]);
#pragma unroll
        for (int t = 0; t < 2; ++t)
          acc[wt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf),
                                                               __builtin_bit_cast(bf16x8, xf[t]), acc[wt][t], 0, 0, 0);
      }
    }
  }

#undef PG_ISSUE
  VK_PHASE(p, 3);
  // tile -> LDS: acc[wt][t] lane holds C^T[weight row 16 wq + 4 g + e (+ 64 for up)][A row 16 t + lane % 16];
  // with two K slices the second adds its partial tile to the first
  lds_barrier();
  float *part = reinterpret_cast<float *>(smem);  // [PG_BM][WR + 1]
#pragma unroll
  for (int h = 0; h < KS; ++h) {
    if (kh == h) {
#pragma unroll
      for (int wt = 0; wt < NW; ++wt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float &dst = part[(16 * t + fr) * (S::WR + 1) + wt * PG_BN + 16 * wq + 4 * fg + e];
            dst = h == 0 ? acc[wt][t][e] : dst + acc[wt][t][e];
          }
    }
    lds_barrier();
  }
  if (tid >= 256) return;
  VK_PHASE(p, 4);

  // ---- epilogue: thread -> (row rr, 4-column group sub) of each 32-column half ----
  float v[HALVES][4], vu[HALVES][4];
#pragma unroll
  for (int hf = 0; hf < HALVES; ++hf)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = 32 * hf + 4 * sub + c;
      v[hf][c] = part[rr * (S::WR + 1) + col];
      vu[hf][c] = SWI ? part[rr * (S::WR + 1) + PG_BN + col] : 0.f;
    }
  if constexpr (ROPE) {
    const int H = p.H, HKV = p.HKV;
    if (p.table_f32) {
      csf = f32x4{__uint_as_float(ctw[0][0]), __uint_as_float(ctw[0][1]), __uint_as_float(ctw[1][0]),
                  __uint_as_float(ctw[1][1])};
      snf = f32x4{__uint_as_float(stw[0][0]), __uint_as_float(stw[0][1]), __uint_as_float(stw[1][0]),
                  __uint_as_float(stw[1][1])};
    } else {
      csf = f32x4{lo_bf(ctw[0][0]), hi_bf(ctw[0][0]), lo_bf(ctw[0][1]), hi_bf(ctw[0][1])};
      snf = f32x4{lo_bf(stw[0][0]), hi_bf(stw[0][0]), lo_bf(stw[0][1]), hi_bf(stw[0][1])};
    }
    float x1[4], x2[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      x1[c] = round_bf(v[0][c]);
      x2[c] = round_bf(v[1][c]);
    }
    if (hd < H + HKV) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) ss += x1[c] * x1[c] + x2[c] * x2[c];
      ss += __shfl_xor(ss, 1, 64);
      ss += __shfl_xor(ss, 2, 64);
      ss += __shfl_xor(ss, 4, 64);
      const float r = rsqrtf(ss / 64.f + p.eps);
      const float w1[4] = {lo_bf(wnf[0][0]), hi_bf(wnf[0][0]), lo_bf(wnf[0][1]), hi_bf(wnf[0][1])};
      const float w2[4] = {lo_bf(wnf[1][0]), hi_bf(wnf[1][0]), lo_bf(wnf[1][1]), hi_bf(wnf[1][1])};
      float a1[4], a2[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float y1 = round_bf(x1[c] * r * w1[c]);
        const float y2 = round_bf(x2[c] * r * w2[c]);
        a1[c] = y1 * csf[c] - y2 * snf[c];
        a2[c] = y1 * snf[c] + y2 * csf[c];
      }
      const u32x2 o1 = u32x2{pack_bf(a1[0], a1[1]), pack_bf(a1[2], a1[3])};
      const u32x2 o2 = u32x2{pack_bf(a2[0], a2[1]), pack_bf(a2[2], a2[3])};
      if (row_ok) {
        if (hd < H) {
          bf16_t *dst = static_cast<bf16_t *>(p.y) + (erow * H + hd) * 64 + 4 * sub;
          *reinterpret_cast<u32x2 *>(dst) = o1;
          *reinterpret_cast<u32x2 *>(dst + 32) = o2;
        } else if (e_seq >= 0 && e_seq < p.cache_rows && e_pos >= 0 && e_pos < p.cache_len) {
          bf16_t *dst = p.kc + e_seq * p.stride_cb + e_pos * p.stride_cs + (hd - H) * 64 + 4 * sub;
          *reinterpret_cast<u32x2 *>(dst) = o1;
          *reinterpret_cast<u32x2 *>(dst + 32) = o2;
        }
      }
    } else if (row_ok && e_seq >= 0 && e_seq < p.cache_rows && e_pos >= 0 && e_pos < p.cache_len) {
      // v head: the rounded projection goes to the cache unchanged
      bf16_t *dst = p.vc + e_seq * p.stride_cb + e_pos * p.stride_cs + (hd - H - HKV) * 64 + 4 * sub;
      *reinterpret_cast<u32x2 *>(dst) = u32x2{pack_bf(x1[0], x1[1]), pack_bf(x1[2], x1[3])};
      *reinterpret_cast<u32x2 *>(dst + 32) = u32x2{pack_bf(x2[0], x2[1]), pack_bf(x2[2], x2[3])};
    }
    VK_PHASE_END(p);
    return;
  }
  float ssq[HALVES] = {};  // EPI_RESID: this thread's share of the row's sum of squares over each 32-column half
#pragma unroll
  for (int hf = 0; hf < HALVES; ++hf) {
    const int col = n0 + 32 * hf + 4 * sub;
    if (!row_ok || col >= p.N) continue;  // N is a multiple of 4 (checked on the host)
    const int64_t off = erow * p.N + col;
    if (EPI == EPI_F32) {
      *reinterpret_cast<f32x4 *>(static_cast<float *>(p.y) + off) = f32x4{v[hf][0], v[hf][1], v[hf][2], v[hf][3]};
    } else {
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float val = v[hf][c];
        if (EPI == EPI_SWIGLU) {
          const float g = round_bf(val);
          const float u = round_bf(vu[hf][c]);
          val = round_bf(g / (1.0f + __expf(-g))) * u;
        }
        o[c] = val;
      }
      if (EPI == EPI_RESID) {
        o[0] = lo_bf(old[hf][0]) + round_bf(o[0]);
        o[1] = hi_bf(old[hf][0]) + round_bf(o[1]);
        o[2] = lo_bf(old[hf][1]) + round_bf(o[2]);
        o[3] = hi_bf(old[hf][1]) + round_bf(o[3]);
      }
      const u32x2 packed = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
      *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(p.y) + off) = packed;
      if (EPI == EPI_RESID) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float lo = lo_bf(packed[e]), hi = hi_bf(packed[e]);
          ssq[hf] += lo * lo + hi * hi;
        }
      }
    }
  }
  if constexpr (EPI == EPI_RESID) {
    if (p.ss_out) {  // the 8 lanes of a row (consecutive) reduce their shares in a fixed order
#pragma unroll
      for (int hf = 0; hf < HALVES; ++hf) {
        float v = ssq[hf];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        if (row_ok && sub == 0) p.ss_out[erow * (p.N / PG_SS_COLS) + 2 * nb + hf] = v;
      }
    }
  }
  VK_PHASE_END(p);
}

// ---- norm + gate_up + SwiGLU on 32 rows x 96 output columns (the decode step's MLP input product) ---------
//
// The panel kernel's 32 x 64 SwiGLU tiles put the decode step's 512 x 1536 output on 384 workgroups, two per CU
// on half the chip: those CUs move 2 x (32 + 128) KB from L2 into LDS, at about 100 GB/s per CU. Here a
// workgroup owns 32 rows x 96 output columns (96 gate + 96 up weight rows): 256 workgroups, one per CU, each
// moving 32 + 192 KB. The product's time follows the bytes per CU and how many wavefronts issue the loads.
//   * A (32 rows x K = 512) is resident in LDS, normalised in place from the handed-over row sums of squares
//     (pg_normalise_rows, as the panel kernel: the same bits);
//   * the 192 weight rows stream through a 4-slot ring of 64-wide K stages (24 KB) by direct global->LDS loads;
//   * NWV wavefronts (the decode step runs 8): with 8, wave w multiplies A block w & 1 by weight blocks
//     3 (w >> 1) .. + 2 (16 x 16 x 32 MFMA, C^T formulation); with 4, both A blocks by blocks 3 w .. + 2;
//   * the tile goes through LDS to the SwiGLU epilogue, with the panel kernel's rounding points.
constexpr int GW_BM = 32, GW_BN = 96, GW_WR = 2 * GW_BN, GW_STAGES = 4;
constexpr int GW_XB = GW_BM * PG_NORM_K * 2;           // resident A: 32 KB
constexpr int GW_STAGEB = GW_WR * PG_ROWB;              // 24 KB
constexpr int GW_PITCH = GW_WR + 1;                     // fp32 row pitch of the tile handed to the epilogue
constexpr int GW_SMEM = GW_XB + GW_STAGES * GW_STAGEB;  // 128 KB: one workgroup per CU
static_assert(GW_BM * GW_PITCH * 4 <= GW_STAGES * GW_STAGEB, "the fp32 tile reuses the ring");
static_assert(PG_NORM_K * 2 + GW_BM * PG_SS_N * 4 <= GW_STAGEB, "norm weight and row sums fit one ring slot");
static_assert(GW_WR == 4 * 3 * 16, "four column groups of three 16-row weight blocks");

template <int NWV>
__global__ __launch_bounds__(64 * NWV) void gate_up_wide_kernel(const SkinnyArgs p, int m_blocks, int tiles) {
  static_assert(NWV == 4 || NWV == 8, "4 waves (both A blocks each) or 8 (one A block each)");
  constexpr int GW_LOADS = GW_WR / 8 / NWV;  // direct loads per wave per stage
  constexpr int TA = 8 / NWV;                // A blocks per wave
  static_assert(GW_LOADS * (GW_STAGES - 1) + GW_BM / NWV + 3 <= 63, "a wave's loads in flight fit the vmcnt counter");
  __shared__ __attribute__((aligned(16))) char smem[GW_SMEM];
  VK_PHASE(p, 0);
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware order (as the panel kernel): workgroup p runs on XCD p % 8, which owns a contiguous range of the
  // n-block-major tiles, so the workgroups of one XCD share weight tiles
  const int pid = blockIdx.x, xcd = pid & 7, idx = pid >> 3;
  const int q8 = tiles >> 3, r8 = tiles & 7;
  const int tile = xcd * q8 + min(xcd, r8) + idx;
  const int nb = tile / m_blocks, mb = tile % m_blocks;
  const int64_t m0 = static_cast<int64_t>(mb) * GW_BM;
  const int n0 = nb * GW_BN;
  // run-time K (512, checked on the host): a constant trip count lets the compiler unroll the K loop, see the
  // ring offsets and drain every load before each LDS read
  const int K = p.K, nk = K / PG_BK;
  // weight sources: instruction q = wid + NWV j of a stage covers ring rows 8 q .. 8 q + 7 (gate rows, then up
  // rows); lane l -> row 8 q + l / 8, slot l % 8, K chunk slot ^ ((row >> 1) & 7)
  const bf16_t *src[GW_LOADS];
#pragma unroll
  for (int j = 0; j < GW_LOADS; ++j) {
    const int r = 8 * (wid + NWV * j) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int wrow = r < GW_BN ? n0 + r : p.N + n0 + (r - GW_BN);  // n0 + 95 < N (N % 96 == 0)
    src[j] = p.w + static_cast<int64_t>(wrow) * K + 8 * c;
  }
  // the norm weight (1 KB) and the 32 rows' 16 partial sums of squares (2 KB) go to the last ring slot, which the
  // K loop fills only after the normalisation; every wave loads them (the same bytes), so its own counted wait
  // covers them. Lane l of load h brings quarter l % 4 of row 16 h + l / 4.
  char *const nwx = smem + GW_XB + (GW_STAGES - 1) * GW_STAGEB;
  char *const ssx = nwx + PG_NORM_K * 2;
  pg_issue_row(nwx, p.norm_w + 8 * lane);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int64_t srow = m0 + 16 * h + (lane >> 2);
    srow = srow < p.M ? srow : p.M - 1;
    pg_issue_row(ssx + 1024 * h, reinterpret_cast<const bf16_t *>(p.ss_in + srow * PG_SS_N + 4 * (lane & 3)));
  }
  // the resident A tile: row i is one instruction, issued by wave i % NWV; chunk c of row r in slot c ^ (r & 15)
#pragma unroll
  for (int i = 0; i < GW_BM / NWV; ++i) {
    const int r = wid + NWV * i;
    int64_t row = m0 + r;
    row = row < p.M ? row : p.M - 1;
    pg_issue_row(smem + r * (PG_NORM_K * 2), p.a + row * K + 8 * (lane ^ (r & 15)));
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int s = 0; s < GW_STAGES - 1; ++s)
    pg_issue<GW_LOADS, NWV>(smem + GW_XB + s * GW_STAGEB, src, s * PG_BK, wid);
  asm volatile("" ::: "memory");
  // waiting until only the ring's loads are outstanding retires this wave's staging and tile rows; the barrier,
  // every wave's
  __builtin_amdgcn_s_waitcnt(pg_vmcnt(GW_LOADS * (GW_STAGES - 1)));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  VK_PHASE(p, 1);
  pg_normalise_rows<GW_BM / NWV, NWV>(smem, nwx, ssx, GW_BM, wid, lane, p.eps);
  lds_barrier();
  VK_PHASE(p, 2);

  // wave w: A blocks t0 .. t0 + TA - 1, weight blocks 3 wg .. 3 wg + 2
  const int t0 = NWV == 8 ? (wid & 1) : 0, wg = NWV == 8 ? (wid >> 1) : wid;
  const int fr = lane & 15, fg = lane >> 4;
  int woff[3][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int R = 16 * (3 * wg + j) + fr, c = 4 * ks + fg;
      woff[j][ks] = R * PG_ROWB + 16 * (c ^ ((R >> 1) & 7));
    }
  f32x4 acc[TA][3];
#pragma unroll
  for (int t = 0; t < TA; ++t)
#pragma unroll
    for (int j = 0; j < 3; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < nk; ++kt) {
    pg_wait_ahead<GW_LOADS, GW_STAGES - 2>(min(nk - 1 - kt, GW_STAGES - 2));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's stage kt has landed; every wave is done with stage kt - 1
    asm volatile("" ::: "memory");
    if (kt + GW_STAGES - 1 < nk)
      pg_issue<GW_LOADS, NWV>(smem + GW_XB + ((kt + GW_STAGES - 1) % GW_STAGES) * GW_STAGEB, src,
                              (kt + GW_STAGES - 1) * PG_BK, wid);
    const char *base = smem + GW_XB + (kt % GW_STAGES) * GW_STAGEB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 xf[TA];
#pragma unroll
      for (int t = 0; t < TA; ++t) {  // resident row 16 (t0 + t) + fr, K chunk 8 kt + 4 ks + fg
        const int c = 8 * kt + 4 * ks + fg;
        xf[t] = *reinterpret_cast<const u32x4 *>(smem + (16 * (t0 + t) + fr) * (PG_NORM_K * 2) + 16 * (c ^ fr));
      }
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const u32x4 wf = *reinterpret_cast<const u32x4 *>(base + woff[j][ks]);
#pragma unroll
        for (int t = 0; t < TA; ++t)
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf),
                                                              __builtin_bit_cast(bf16x8, xf[t]), acc[t][j], 0, 0, 0);
      }
    }
  }

  VK_PHASE(p, 3);
  // tile -> LDS: acc[t][j] lane holds C^T[weight row 16 (3 wg + j) + 4 fg + e][A row 16 (t0 + t) + fr]
  lds_barrier();
  float *part = reinterpret_cast<float *>(smem + GW_XB);  // [GW_BM][GW_PITCH]
#pragma unroll
  for (int t = 0; t < TA; ++t)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        part[(16 * (t0 + t) + fr) * GW_PITCH + 16 * (3 * wg + j) + 4 * fg + e] = acc[t][j][e];
  lds_barrier();
  VK_PHASE(p, 4);

  // SwiGLU epilogue: 32 rows x 24 groups of 4 columns; out = bf16(bf16(silu(bf16(g))) bf16(u))
  constexpr int ITEMS = GW_BM * GW_BN / 4;
#pragma unroll
  for (int it = 0; it < (ITEMS + 64 * NWV - 1) / (64 * NWV); ++it) {
    const int i = tid + 64 * NWV * it, rr = i / 24, grp = i - 24 * rr;
    const int64_t erow = m0 + rr;
    if (i >= ITEMS || erow >= p.M) continue;
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float g = round_bf(part[rr * GW_PITCH + 4 * grp + c]);
      const float u = round_bf(part[rr * GW_PITCH + GW_BN + 4 * grp + c]);
      o[c] = round_bf(g / (1.0f + __expf(-g))) * u;
    }
    *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(p.y) + erow * p.N + n0 + 4 * grp) =
        u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
  }
  VK_PHASE_END(p);
}

#ifdef VK_PHASE_STAMPS
// The profiling build's stamp buffer: each launch takes the next 8 x workgroups slots while they last.
static uint64_t *g_stamps = nullptr;
static int64_t g_stamp_cap = 0, g_stamp_used = 0;
static SkinnyArgs with_stamps(const SkinnyArgs &a, int64_t wgs) {
  SkinnyArgs p = a;
  p.stamps = nullptr;
  if (g_stamps && g_stamp_used + 8 * wgs <= g_stamp_cap) {
    p.stamps = g_stamps + g_stamp_used;
    g_stamp_used += 8 * wgs;
  }
  return p;
}
#else
static const SkinnyArgs &with_stamps(const SkinnyArgs &a, int64_t) { return a; }
#endif

static int launch_gate_up_wide(const SkinnyArgs &a, hipStream_t s) {
  const int64_t m_blocks = (a.M + GW_BM - 1) / GW_BM;
  const int64_t tiles = m_blocks * (a.N / GW_BN);
  // 8 wavefronts: more of them issuing the direct loads (4 measured 7% slower)
  gate_up_wide_kernel<8><<<static_cast<unsigned>(tiles), 512, 0, s>>>(with_stamps(a, tiles), static_cast<int>(m_blocks),
                                                                      static_cast<int>(tiles));
  return VK_OK;
}

// ---- residual product on 32 x 32 tiles (the decode step's o / down projections) ------------------------
//
// x[M, N] += bf16(A[M, K] W[N, K]^T) with the rounding points of add_rmsnorm, and (optionally) the row's sum of
// squares of the updated x over each 32-column block. A workgroup's time hardly depends on how many run beside
// it (measured at K = 512: 4.2 us for 32 workgroups, 4.6 us for 256): it is set by the bytes one CU moves from
// L2 into LDS (about 100 GB/s per CU) plus a fixed cost. 32 x 32 tiles put the decode step's 512 x 512 output on
// 256 workgroups moving 64 x K x 2 bytes each, against 128 panel workgroups of 32 x 64 moving 96 x K x 2.
//   * KSP K slices of 4 wavefronts (the decode step runs KSP = 2); each slice streams its 32 A and 32 W rows
//     through its own ring of 64-wide K stages (8 KB; 12 / KSP slots) by direct global->LDS loads (lane l of an
//     instruction lands at slot base + 16 l);
//   * wave (slice h, q) multiplies A block q >> 1 by weight block q & 1 (one 16 x 16 x 32 MFMA tile, C^T
//     formulation: the weight fragment is the A operand);
//   * the slices' tiles meet in LDS and the epilogue adds them in slice order (with two slices the panel
//     kernel's K-split sum, bit for bit).
constexpr int RS_BM = 32, RS_BN = 32;
constexpr int RS_ROWS = RS_BM + RS_BN;          // LDS rows per ring stage (A rows, then W rows)
constexpr int RS_STAGEB = RS_ROWS * PG_ROWB;    // 8 KB
constexpr int RS_LOADS = RS_ROWS / 8 / 4;       // direct loads per wave per stage
constexpr int RS_PITCH = RS_BN + 1;             // fp32 row pitch of a half's tile
constexpr int RS_SMEM = 12 * RS_STAGEB;         // 96 KB: 12 ring slots in all
static_assert(4 * RS_BM * RS_PITCH * 4 <= RS_SMEM, "every K slice's fp32 tile fits the rings");
static_assert(RS_BN == PG_SS_COLS, "one partial sum of squares per tile row");

template <int KSP>
__global__ __launch_bounds__(256 * KSP) void resid_gemm_kernel(const SkinnyArgs p, int m_blocks, int tiles) {
  constexpr int RS_STAGES = 12 / KSP;               // slots per ring (one ring per K slice)
  constexpr int RS_RING = RS_STAGES * RS_STAGEB;
  __shared__ __attribute__((aligned(16))) char smem[RS_SMEM];
  VK_PHASE(p, 0);
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wq = wid & 3, kh = wid >> 2;  // wave within its K slice, K slice
  // XCD-aware order (as the panel kernel): workgroup p runs on XCD p % 8, which owns a contiguous range of the
  // n-block-major tiles
  const int pid = blockIdx.x, xcd = pid & 7, idx = pid >> 3;
  const int q8 = tiles >> 3, r8 = tiles & 7;
  const int tile = xcd * q8 + min(xcd, r8) + idx;
  const int nb = tile / m_blocks, mb = tile % m_blocks;
  const int64_t m0 = static_cast<int64_t>(mb) * RS_BM;
  const int n0 = nb * RS_BN;
  // run-time K (a constant trip count lets the compiler unroll the loop, see the ring offsets and drain every
  // load before each LDS read)
  const int K = p.K, nk = K / (PG_BK * KSP), kbase = kh * (K / KSP);
  const int fr = lane & 15, fg = lane >> 4;

  // sources: instruction q = wq + 4 j of a stage covers ring rows 8 q .. 8 q + 7; lane l -> row 8 q + l / 8,
  // slot l % 8, K chunk slot ^ ((row >> 1) & 7); rows past M or N read the last row (not stored)
  const bf16_t *src[RS_LOADS];
#pragma unroll
  for (int j = 0; j < RS_LOADS; ++j) {
    const int r = 8 * (wq + 4 * j) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    if (r < RS_BM) {
      int64_t row = m0 + r;
      row = row < p.M ? row : p.M - 1;
      src[j] = p.a + row * K + 8 * c + kbase;
    } else {
      int col = n0 + r - RS_BM;
      col = col < p.N ? col : p.N - 1;
      src[j] = p.w + static_cast<int64_t>(col) * K + 8 * c + kbase;
    }
  }
  char *const ring = smem + kh * RS_RING;
#pragma unroll
  for (int s = 0; s < RS_STAGES - 1; ++s)
    if (s < nk) pg_issue<RS_LOADS>(ring + s * RS_STAGEB, src, s * PG_BK, wq);

  // epilogue mapping: thread t < 256 -> row m0 + t / 8, columns 4 (t % 8) .. + 3; the old residual is loaded
  // now, unconditionally (row and column clamped): a load under a branch makes the compiler wait for every
  // outstanding load, the ring's included, where its register is merged
  const int rr = (tid >> 3) & (RS_BM - 1), sub = tid & 7;
  const int64_t erow = m0 + rr;
  const int ecol = n0 + 4 * sub;
  u32x2 old;
  {
    const int64_t orow = erow < p.M ? erow : p.M - 1;
    const int ocol = ecol < p.N ? ecol : p.N - 4;
    old = *reinterpret_cast<const u32x2 *>(static_cast<const bf16_t *>(p.y) + orow * p.N + ocol);
  }

  const int ta = wq >> 1, wb = wq & 1;
  int xoff[2], woff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int c = 4 * ks + fg;
    const int RA = 16 * ta + fr, RW = RS_BM + 16 * wb + fr;
    xoff[ks] = RA * PG_ROWB + 16 * (c ^ ((RA >> 1) & 7));
    woff[ks] = RW * PG_ROWB + 16 * (c ^ ((RW >> 1) & 7));
  }
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kt = 0; kt < nk; ++kt) {
    pg_wait_ahead<RS_LOADS, RS_STAGES - 2>(min(nk - 1 - kt, RS_STAGES - 2));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's stage kt has landed; every wave is done with stage kt - 1
    asm volatile("" ::: "memory");
    if (kt == 0) {
      VK_PHASE(p, 1);
      VK_PHASE(p, 2);
    }
    if (kt + RS_STAGES - 1 < nk)
      pg_issue<RS_LOADS>(ring + ((kt + RS_STAGES - 1) % RS_STAGES) * RS_STAGEB, src, (kt + RS_STAGES - 1) * PG_BK, wq);
    const char *base = ring + (kt % RS_STAGES) * RS_STAGEB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 xf = *reinterpret_cast<const u32x4 *>(base + xoff[ks]);
      const u32x4 wf = *reinterpret_cast<const u32x4 *>(base + woff[ks]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf), __builtin_bit_cast(bf16x8, xf), acc,
                                                    0, 0, 0);
    }
  }

  VK_PHASE(p, 3);
  // tiles -> LDS: acc lane holds C^T[weight row 16 wb + 4 fg + e][A row 16 ta + fr] of its K half
  lds_barrier();
  float *part = reinterpret_cast<float *>(smem);  // [2][RS_BM][RS_PITCH]
#pragma unroll
  for (int e = 0; e < 4; ++e) part[(kh * RS_BM + 16 * ta + fr) * RS_PITCH + 16 * wb + 4 * fg + e] = acc[e];
  lds_barrier();
  if (tid >= 256) return;
  VK_PHASE(p, 4);

  // x = bf16(x + bf16(sum of the slices' tiles in slice order)); the row's sum of squares over the 32 columns from the 8 lanes
  // of the row (consecutive) in a fixed order
  float o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float v = part[rr * RS_PITCH + 4 * sub + c];
#pragma unroll
    for (int h = 1; h < KSP; ++h) v += part[(h * RS_BM + rr) * RS_PITCH + 4 * sub + c];
    o[c] = round_bf(v);
  }
  o[0] += lo_bf(old[0]);
  o[1] += hi_bf(old[0]);
  o[2] += lo_bf(old[1]);
  o[3] += hi_bf(old[1]);
  const u32x2 packed = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
  const bool ok = erow < p.M && ecol < p.N;  // N is a multiple of 4 (checked on the host)
  if (ok) *reinterpret_cast<u32x2 *>(static_cast<bf16_t *>(p.y) + erow * p.N + ecol) = packed;
  if (p.ss_out) {
    float ssq = 0.f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float lo = lo_bf(packed[e]), hi = hi_bf(packed[e]);
      ssq += lo * lo + hi * hi;
    }
    ssq += __shfl_xor(ssq, 1, 64);
    ssq += __shfl_xor(ssq, 2, 64);
    ssq += __shfl_xor(ssq, 4, 64);
    if (erow < p.M && sub == 0) p.ss_out[erow * (p.N / PG_SS_COLS) + nb] = ssq;
  }
  VK_PHASE_END(p);
}

static int launch_resid(const SkinnyArgs &a, hipStream_t s) {
  const int64_t m_blocks = (a.M + RS_BM - 1) / RS_BM;
  const int64_t tiles = m_blocks * ((a.N + RS_BN - 1) / RS_BN);
  // two K slices: one slice of 4 wavefronts measured 18% slower at K = 1536 (fewer loads in flight per CU),
  // four slices no faster in the decode step
  resid_gemm_kernel<2><<<static_cast<unsigned>(tiles), 512, 0, s>>>(with_stamps(a, tiles), static_cast<int>(m_blocks),
                                                                    static_cast<int>(tiles));
  return VK_OK;
}

template <int PRO, int EPI>
static int launch_panel(const SkinnyArgs &a, hipStream_t s) {
  const int64_t m_blocks = (a.M + PG_BM - 1) / PG_BM;
  const int64_t n_blocks = (a.N + PG_BN - 1) / PG_BN;
  const int64_t tiles = m_blocks * n_blocks;
  if (tiles >= (int64_t(1) << 31)) return fail(VK_ERR_ARG, "linear: too many tiles");
  // two K slices when the 8-wave workgroups (one per CU: two rings of LDS) still fit in one round
  constexpr bool can_split = (PRO == PRO_NONE || PRO == PRO_NORM_SS || PRO == PRO_EMBED_RES) && EPI != EPI_SWIGLU;
  if (can_split && a.K % (2 * PG_BK) == 0 && tiles <= device_cus_cached()) {
    panel_gemm_kernel<PRO, EPI, can_split ? 2 : 1><<<static_cast<unsigned>(tiles), 512, 0, s>>>(
        with_stamps(a, tiles), static_cast<int>(m_blocks), static_cast<int>(tiles));
  } else {
    panel_gemm_kernel<PRO, EPI, 1><<<static_cast<unsigned>(tiles), 256, 0, s>>>(with_stamps(a, tiles),
                                                                             static_cast<int>(m_blocks),
                                                                             static_cast<int>(tiles));
  }
  return VK_OK;
}

// The panel kernel takes K % 64 == 0 (with a norm: K = 512); the split-K kernel the rest.
static bool panel_ok(const SkinnyArgs &a, int pro) {
  return a.K % PG_BK == 0 && (pro == PRO_NONE || a.K == PG_NORM_K);
}

template <int BN, int WAVES, int KSTEPS, int PRO, int EPI>
static void launch_skinny(const SkinnyArgs &a, hipStream_t s) {
  const dim3 grid((a.N + BN - 1) / BN, static_cast<unsigned>((a.M + SK_BM - 1) / SK_BM));
  skinny_gemm_kernel<BN, WAVES, KSTEPS, PRO, EPI><<<grid, WAVES * 64, 0, s>>>(a);
}

#ifndef VK_SK512_WAVES
#define VK_SK512_WAVES 8  // waves splitting K = 512 (each 512 / 32 / waves k-steps)
#endif

// K = 512 (d_model) with VK_SK512_WAVES waves, K = 1536 (ffn) with 8 waves of 6 k-steps
template <int BN, int PRO, int EPI>
static int dispatch_k(const SkinnyArgs &a, hipStream_t s) {
  if (a.K == 512) {
    launch_skinny<BN, VK_SK512_WAVES, 16 / VK_SK512_WAVES, PRO, EPI>(a, s);
  } else if (a.K == 1536) {
    launch_skinny<BN, 8, 6, PRO, EPI>(a, s);
  } else if (a.K == 256) {
    launch_skinny<BN, 4, 2, PRO, EPI>(a, s);
  } else if (a.K == 1024) {
    launch_skinny<BN, 8, 4, PRO, EPI>(a, s);
  } else {
    return fail(VK_ERR_UNSUPPORTED, "skinny linear: K must be 256, 512, 1024 or 1536 (got %d)", a.K);
  }
  return VK_OK;
}

static SkinnyArgs base_args(const void *a, const void *w, void *y, int64_t M, int N, int K) {
  SkinnyArgs p{};
  p.a = static_cast<const bf16_t *>(a);
  p.w = static_cast<const bf16_t *>(w);
  p.y = y;
  p.M = M;
  p.N = N;
  p.K = K;
  return p;
}

}  // namespace vk

using namespace vk;

extern "C" int vk_norm_linear(const void *x, const void *norm_w, float eps, const void *w, void *y, int64_t M, int32_t N,
                              int32_t K, int32_t swiglu, int32_t out_dtype, const float *ss_in, void *stream) {
  VK_CHECK_ARG(x && w && y, "norm_linear: null pointer");
  VK_CHECK_ARG(M >= 0 && N > 0 && N % 4 == 0 && K > 0, "norm_linear: bad sizes");
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(y) && (!norm_w || vk_aligned16(norm_w)),
               "norm_linear: alignment");
  VK_CHECK_ARG(!(swiglu && out_dtype == VK_DTYPE_F32), "norm_linear: the SwiGLU epilogue stores bf16");
  if (M == 0) return VK_OK;
  SkinnyArgs p = base_args(x, w, y, M, N, K);
  p.norm_w = static_cast<const bf16_t *>(norm_w);
  p.eps = eps;
  p.ss_in = ss_in;
  hipStream_t s = VK_STREAM(stream);
  int rc;
  if (ss_in) {  // the norm from the producing GEMM's row sums of squares
    VK_CHECK_ARG(norm_w && K == PG_NORM_K && vk_aligned16(ss_in), "norm_linear: ss_in needs norm_w and K = %d",
                 PG_NORM_K);
    // 32 x 96 SwiGLU tiles while they fit one resident round of the chip (the decode step's 512 rows)
    const bool wide = swiglu && N % GW_BN == 0 && ((M + GW_BM - 1) / GW_BM) * (N / GW_BN) <= device_cus_cached();
    rc = wide     ? launch_gate_up_wide(p, s)
         : swiglu ? launch_panel<PRO_NORM_SS, EPI_SWIGLU>(p, s)
                  : (out_dtype == VK_DTYPE_F32 ? launch_panel<PRO_NORM_SS, EPI_F32>(p, s)
                                             : launch_panel<PRO_NORM_SS, EPI_BF16>(p, s));
  } else if (panel_ok(p, norm_w ? PRO_NORM : PRO_NONE)) {
    if (norm_w)
      rc = swiglu ? launch_panel<PRO_NORM, EPI_SWIGLU>(p, s)
                  : (out_dtype == VK_DTYPE_F32 ? launch_panel<PRO_NORM, EPI_F32>(p, s)
                                               : launch_panel<PRO_NORM, EPI_BF16>(p, s));
    else
      rc = swiglu ? launch_panel<PRO_NONE, EPI_SWIGLU>(p, s)
                  : (out_dtype == VK_DTYPE_F32 ? launch_panel<PRO_NONE, EPI_F32>(p, s)
                                               : launch_panel<PRO_NONE, EPI_BF16>(p, s));
  } else if (norm_w) {
    if (swiglu)
      rc = dispatch_k<32, PRO_NORM, EPI_SWIGLU>(p, s);
    else if (out_dtype == VK_DTYPE_F32)
      rc = dispatch_k<32, PRO_NORM, EPI_F32>(p, s);
    else
      rc = dispatch_k<32, PRO_NORM, EPI_BF16>(p, s);
  } else {
    if (swiglu)
      rc = dispatch_k<32, PRO_NONE, EPI_SWIGLU>(p, s);
    else if (out_dtype == VK_DTYPE_F32)
      rc = dispatch_k<32, PRO_NONE, EPI_F32>(p, s);
    else
      rc = dispatch_k<32, PRO_NONE, EPI_BF16>(p, s);
  }
  if (rc != VK_OK) return rc;
  return launch_status("norm_linear");
}

extern "C" int vk_linear_residual(const void *a, const void *w, void *x, int64_t M, int32_t N, int32_t K,
                                  float *ss_out, void *stream) {
  VK_CHECK_ARG(a && w && x, "linear_residual: null pointer");
  VK_CHECK_ARG(M >= 0 && N > 0 && N % 4 == 0 && K > 0, "linear_residual: bad sizes");
  VK_CHECK_ARG(vk_aligned16(a) && vk_aligned16(w) && vk_aligned16(x), "linear_residual: alignment");
  if (M == 0) return VK_OK;
  SkinnyArgs p = base_args(a, w, x, M, N, K);
  p.ss_out = ss_out;
  VK_CHECK_ARG(!ss_out || (panel_ok(p, PRO_NONE) && N == PG_NORM_K),
               "linear_residual: row sums of squares need K %% 64 == 0 and N = %d", PG_NORM_K);
  // 32 x 32 tiles while they fit one resident round of the chip (the decode step's 512 rows), else the panel
  const int64_t rs_tiles = ((M + RS_BM - 1) / RS_BM) * ((N + RS_BN - 1) / RS_BN);
  const int rc = (K % (2 * PG_BK) == 0 && rs_tiles <= device_cus_cached())
                     ? launch_resid(p, VK_STREAM(stream))
                     : (panel_ok(p, PRO_NONE) ? launch_panel<PRO_NONE, EPI_RESID>(p, VK_STREAM(stream))
                                              : dispatch_k<32, PRO_NONE, EPI_RESID>(p, VK_STREAM(stream)));
  if (rc != VK_OK) return rc;
  return launch_status("linear_residual");
}

extern "C" int vk_norm_qkv_rope_cache(const void *x, const int64_t *tok, int64_t vocab, void *x_store,
                                      const void *norm_w, float eps, const void *w_qkv, const void *q_norm_w,
                                      const void *k_norm_w, const void *cos_t, const void *sin_t, int32_t table_dtype,
                                      int64_t table_rows, const int32_t *pos, const int32_t *rope_pos,
                                      const int32_t *seq, void *q, void *k_cache, void *v_cache, int64_t stride_cb,
                                      int64_t stride_cs, int64_t cache_rows, int64_t cache_len, int64_t M, int32_t K,
                                      int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const float *ss_in,
                                      void *stream) {
  VK_CHECK_ARG(x && w_qkv && q_norm_w && k_norm_w && cos_t && sin_t && pos && seq && q && k_cache && v_cache,
               "norm_qkv_rope_cache: null pointer");
  VK_CHECK_ARG(norm_w || !tok, "norm_qkv_rope_cache: the embedding gather needs norm_w");
  VK_CHECK_ARG(head_dim == 64, "norm_qkv_rope_cache: built for head_dim 64");
  VK_CHECK_ARG(tok == nullptr || (x_store != nullptr && vocab > 0), "norm_qkv_rope_cache: embedding needs x_store");
  VK_CHECK_ARG(table_dtype == VK_DTYPE_BF16 || table_dtype == VK_DTYPE_F32, "norm_qkv_rope_cache: table dtype");
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w_qkv) && (!norm_w || vk_aligned16(norm_w)) && vk_aligned16(q) &&
                   vk_aligned16(q_norm_w) && vk_aligned16(k_norm_w) && vk_aligned16(cos_t) && vk_aligned16(sin_t),
               "norm_qkv_rope_cache: alignment");
  if (M == 0) return VK_OK;
  SkinnyArgs p = base_args(x, w_qkv, q, M, (n_heads + 2 * n_kv_heads) * 64, K);
  p.tok = tok;
  p.vocab = vocab;
  p.x_store = static_cast<bf16_t *>(x_store);
  p.norm_w = static_cast<const bf16_t *>(norm_w);
  p.eps = eps;
  p.qw = static_cast<const bf16_t *>(q_norm_w);
  p.kw = static_cast<const bf16_t *>(k_norm_w);
  p.cos_t = cos_t;
  p.sin_t = sin_t;
  p.table_f32 = table_dtype == VK_DTYPE_F32;
  p.table_rows = table_rows;
  p.pos = pos;
  p.rope_pos = rope_pos;
  p.seq = seq;
  p.kc = static_cast<bf16_t *>(k_cache);
  p.vc = static_cast<bf16_t *>(v_cache);
  p.stride_cb = stride_cb;
  p.stride_cs = stride_cs;
  p.cache_rows = cache_rows;
  p.cache_len = cache_len;
  p.H = n_heads;
  p.HKV = n_kv_heads;
  hipStream_t s = VK_STREAM(stream);
  p.ss_in = ss_in;
  int rc;
  if (ss_in) {  // the norm from the producing GEMM's row sums of squares
    VK_CHECK_ARG(norm_w && !tok && K == PG_NORM_K && vk_aligned16(ss_in),
                 "norm_qkv_rope_cache: ss_in needs norm_w, no tok and K = %d", PG_NORM_K);
    rc = launch_panel<PRO_NORM_SS, EPI_ROPE>(p, s);
  } else if (!norm_w)  // x is the normalised activation already
    rc = panel_ok(p, PRO_NONE) ? launch_panel<PRO_NONE, EPI_ROPE>(p, s) : dispatch_k<64, PRO_NONE, EPI_ROPE>(p, s);
  else if (panel_ok(p, PRO_NORM))
    rc = tok ? launch_panel<PRO_EMBED_RES, EPI_ROPE>(p, s) : launch_panel<PRO_NORM, EPI_ROPE>(p, s);
  else
    rc = tok ? dispatch_k<64, PRO_EMBED_NORM, EPI_ROPE>(p, s) : dispatch_k<64, PRO_NORM, EPI_ROPE>(p, s);
  if (rc != VK_OK) return rc;
  return launch_status("norm_qkv_rope_cache");
}

#ifdef VK_PHASE_STAMPS
// Profiling build only (not part of the product library or its header): the stamp buffer ([cap] uint64 device
// memory, 8 slots per workgroup of each later launch of the panel, gate_up and residual kernels; null: off), and
// the slots taken so far.
extern "C" int vk_phase_stamps_set(uint64_t *buf, int64_t cap) {
  VK_CHECK_ARG(cap >= 0 && (buf || cap == 0), "phase_stamps_set: bad buffer");
  g_stamps = buf;
  g_stamp_cap = cap;
  g_stamp_used = 0;
  return VK_OK;
}
extern "C" int vk_phase_stamps_used(int64_t *used) {
  VK_CHECK_ARG(used, "phase_stamps_used: null pointer");
  *used = g_stamp_used;
  return VK_OK;
}
#endif
