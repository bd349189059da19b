// Single-query GQA decode attention over one layer of the static KV cache [B, S, HKV=2, D=64] (bf16).
//
// Semantics: viktor/decode_attention.py:11-53 -- per sequence b and query head h,
//   out = softmax(q . K[:len]^T * D^-0.5) V[:len], fp32 online softmax in the exp2 domain, the
//   probabilities rounded to bf16 before the PV product, output rounded to bf16.
//
// MI355X design:
//   * A cache row (one position, both KV heads) is 2 x 64 bf16 = 256 contiguous bytes. Each lane reads
//     16-byte pieces of it directly into MFMA fragments, so every K/V byte is fetched exactly once for
//     all 8 query heads (4 per KV head).
//   * Both KV heads go through one MFMA chain with a block-diagonal query operand: column r (query
//     head r) of Q^T is non-zero only on the 64 K-values of its own KV head, so
//     S^T[pos, r] = K_row(pos)[128] . Qbd[r][128] is the score of head r against its own KV head.
//   * S^T = K Q^T (v_mfma_f32_16x16x32_bf16: A = 16 cache rows, B = Q^T) leaves each lane holding the
//     scores of one query row (lane % 16) at 4 positions of each 16-position half-tile. The PV product
//     is computed transposed, O^T = V^T P^T, whose B operand needs exactly those (row, 8 positions)
//     values: the probabilities never leave the lane that computed them, and the online-softmax
//     rescale of O^T is lane-local too. The K-order of a 32-position tile is permuted consistently in
//     both operands ({4g..4g+3, 16+4g..16+4g+3} for lane group g).
//   * V^T needs position-contiguous fragments, the cache is column-contiguous: each wavefront stages
//     its 32 x 128 V tile in its own LDS slice (16-byte writes) and reads the transposed fragments with
//     gfx950's transpose reads (two ds_read_b64_tr_b16 per fragment, in place of eight 2-byte reads).
//   * Work split: a workgroup of WAVES wavefronts per (sequence, key split); its wavefronts take
//     interleaved 32-position tiles; per-wave (max, sum, O) partials are merged through LDS. When the
//     batch alone cannot fill the chip (B < 2 x CUs) the key range is split across workgroups and a
//     small combine kernel merges the split partials from the workspace.
#include <math.h>

#include <mutex>

#include "common.h"

namespace vk {

constexpr int DA_H = 8;        // query heads
constexpr int DA_HKV = 2;      // KV heads
constexpr int DA_D = 64;       // head dim
constexpr int DA_ROW = 128;    // HKV * D elements per cache row
constexpr int DA_TILE = 32;    // positions per wavefront iteration
constexpr int DA_PITCH = 136;  // LDS row pitch of the V tile (bf16 elements)
constexpr int DA_WAVES = 8;

struct DecodeSplit {
  int nsplit;  // key splits per sequence
  int tps;     // 32-position tiles per split
};

static DecodeSplit decode_split(int64_t B, int64_t max_len, int cus) {
  const int ntiles = static_cast<int>((max_len + DA_TILE - 1) / DA_TILE);
  const int64_t want = 2 * static_cast<int64_t>(cus > 0 ? cus : 256);
  int nsplit = 1;
  if (B < want) nsplit = static_cast<int>((want + B - 1) / B);
  const int max_split = (ntiles + DA_WAVES - 1) / DA_WAVES;  // at least one tile per wave
  if (nsplit > max_split) nsplit = max_split;
  if (nsplit < 1) nsplit = 1;
  const int tps = (ntiles + nsplit - 1) / nsplit;
  nsplit = (ntiles + tps - 1) / tps;
  return {nsplit, tps};
}

template <bool SPLIT>
__global__ __launch_bounds__(DA_WAVES * 64) void decode_attn_kernel(
    const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc, const bf16_t *__restrict__ vc,
    const int32_t *__restrict__ lengths, const int32_t *__restrict__ rows, int64_t cache_rows,
    bf16_t *__restrict__ out, int64_t stride_b, int64_t stride_s, int64_t max_len, int tps, int nsplit,
    float *__restrict__ ws_o, float *__restrict__ ws_ml, float scale_log2) {
  __shared__ __attribute__((aligned(16))) bf16_t Vs[DA_WAVES][DA_TILE * DA_PITCH];

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform for the compiler
  const int64_t b = blockIdx.y;
  const int split = blockIdx.x;
  // cache row of sequence b (rows == NULL: row b); a row outside the cache gives a zero output (the
  // combine kernel writes it when the key range is split)
  const int64_t crow = rows ? static_cast<int64_t>(rows[b]) : b;
  if (crow < 0 || crow >= cache_rows) {
    if (!SPLIT && split == 0)
      for (int o = threadIdx.x; o < DA_H * DA_D; o += DA_WAVES * 64) out[b * DA_H * DA_D + o] = 0;
    return;  // uniform over the workgroup
  }
  int64_t len = lengths[b];
  len = len < 1 ? 1 : (len > max_len ? max_len : len);
  const int ntiles = static_cast<int>((len + DA_TILE - 1) / DA_TILE);
  const int t_begin = split * tps;
  const int t_end = min(t_begin + tps, ntiles);
  if (t_begin >= t_end) return;  // whole workgroup: this split lies past the sequence

  const int qrow = lane & 15;  // query head of this lane's S^T / O^T column; also the A-fragment row
  const int g = lane >> 4;     // lane group: K-values 8g..8g+7 of each 32-wide fragment

  // block-diagonal Q^T fragments: chunk c (32 of the 128 row values) belongs to KV head c / 2
  bf16x8 bq[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool own = qrow < DA_H && (qrow >> 2) == (c >> 1);
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (own) v = *reinterpret_cast<const u32x4 *>(q + (b * DA_H + qrow) * DA_D + (c & 1) * 32 + g * 8);
    bq[c] = __builtin_bit_cast(bf16x8, v);
  }

  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const bf16_t *kb = kc + crow * stride_b;
  const bf16_t *vb = vc + crow * stride_b;
  bf16_t *vs = Vs[wid];

  // Software pipeline: the next tile's K loads are issued as soon as the score MFMAs have consumed the
  // current K fragments, and its V loads as soon as the current V tile sits in LDS, so every wave keeps
  // 16 KB of loads in flight through the softmax and PV phases without extra registers.
  u32x4 kf[2][4], vf[2][4];
  auto row_ptr = [&](const bf16_t *base, int tt, int pb) {
    int64_t p = static_cast<int64_t>(tt) * DA_TILE + 16 * pb + qrow;
    p = p < len ? p : len - 1;  // rows past the length: any valid row, masked below
    return base + p * stride_s + g * 8;
  };
  auto load_k = [&](int tt) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const bf16_t *r = row_ptr(kb, tt, pb);
#pragma unroll
      for (int c = 0; c < 4; ++c) kf[pb][c] = *reinterpret_cast<const u32x4 *>(r + 32 * c);
    }
  };
  auto load_v = [&](int tt) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const bf16_t *r = row_ptr(vb, tt, pb);
#pragma unroll
      for (int c = 0; c < 4; ++c) vf[pb][c] = *reinterpret_cast<const u32x4 *>(r + 32 * c);
    }
  };
  // prefetches are unconditional (a wave past its last tile re-reads the current one, an L2 hit) so the
  // compiler can count the outstanding loads across the loop back edge instead of draining them all
  const int t_first = min(t_begin + wid, t_end - 1);
  load_k(t_first);
  asm volatile("" ::: "memory");  // keep K before V: the loop waits for K with the V loads still in flight
  load_v(t_first);
  for (int t = t_begin + wid; t < t_end; t += DA_WAVES) {
    const int64_t p0 = static_cast<int64_t>(t) * DA_TILE;
    const int tn = t + DA_WAVES < t_end ? t + DA_WAVES : t;
    // scores S^T[pos][qrow]
    f32x4 st[2];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      st[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        st[pb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[pb][c]), bq[c], st[pb], 0, 0, 0);
    }
    load_k(tn);
    // online softmax over this tile (lane holds positions p0 + 16 pb + 4 g + i)
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t p = p0 + 16 * pb + 4 * g + i;
        const float v = p < len ? st[pb][i] * scale_log2 : -INFINITY;
        sv[pb * 4 + i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.f;
    bf16x8 pf;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const float p = exp2f(sv[jj] - m_new);
      psum += p;
      pf[jj] = __builtin_bit_cast(__bf16, f2bf(p));
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] *= alpha;

    // stage V (row-major) in this wave's LDS slice, read transposed fragments
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<u32x4 *>(&vs[(16 * pb + qrow) * DA_PITCH + 32 * c + g * 8]) = vf[pb][c];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    load_v(tn);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // V^T fragment: column 16 j + qrow at positions 4 g .. + 3 and 16 + 4 g .. + 3, by transpose reads
      const bf16x8 va = lds_tr_frag<DA_PITCH>(vs, 0, 16 * j, lane);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf, acc[j], 0, 0, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // row sums: add the 4 lane groups of each query row
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  __syncthreads();  // every wave is done with its V slice: reuse the LDS for the merge
  float *Os = reinterpret_cast<float *>(&Vs[0][0]);  // [WAVES][8][128]
  float *Ms = Os + DA_WAVES * DA_H * DA_ROW;          // [WAVES][8]
  float *Ls = Ms + DA_WAVES * DA_H;                   // [WAVES][8]
  if (qrow < DA_H) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) Os[(wid * DA_H + qrow) * DA_ROW + 16 * j + 4 * g + i] = acc[j][i];
    if (g == 0) {
      Ms[wid * DA_H + qrow] = m_run;
      Ls[wid * DA_H + qrow] = l_run;
    }
  }
  __syncthreads();
  for (int o = threadIdx.x; o < DA_H * DA_D; o += DA_WAVES * 64) {
    const int h = o / DA_D, d = o % DA_D;
    const int col = (h / (DA_H / DA_HKV)) * DA_D + d;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DA_WAVES; ++w) M = fmaxf(M, Ms[w * DA_H + h]);
    float L = 0.f, N = 0.f;
#pragma unroll
    for (int w = 0; w < DA_WAVES; ++w) {
      const float e = exp2f(Ms[w * DA_H + h] - M);
      L += e * Ls[w * DA_H + h];
      N += e * Os[(w * DA_H + h) * DA_ROW + col];
    }
    if (!SPLIT) {
      out[(b * DA_H + h) * DA_D + d] = f2bf(N / L);
    } else {
      const int64_t base = (b * nsplit + split) * DA_H + h;
      ws_o[base * DA_D + d] = N;
      if (d == 0) {
        ws_ml[base * 2] = M;
        ws_ml[base * 2 + 1] = L;
      }
    }
  }
}

// Merge the key-split partials of each sequence (only the splits its length reaches).
__global__ __launch_bounds__(DA_H * DA_D) void decode_attn_combine(const float *__restrict__ ws_o,
                                                                    const float *__restrict__ ws_ml,
                                                                    const int32_t *__restrict__ lengths,
                                                                    const int32_t *__restrict__ rows,
                                                                    int64_t cache_rows, bf16_t *__restrict__ out,
                                                                    int64_t max_len, int tps, int nsplit) {
  const int64_t b = blockIdx.x;
  const int h = threadIdx.x / DA_D, d = threadIdx.x % DA_D;
  const int64_t crow = rows ? static_cast<int64_t>(rows[b]) : b;
  if (crow < 0 || crow >= cache_rows) {  // no partials were written for a row outside the cache
    out[(b * DA_H + h) * DA_D + d] = 0;
    return;
  }
  int64_t len = lengths[b];
  len = len < 1 ? 1 : (len > max_len ? max_len : len);
  const int ntiles = static_cast<int>((len + DA_TILE - 1) / DA_TILE);
  const int nvalid = min(nsplit, (ntiles + tps - 1) / tps);
  float M = -INFINITY;
  for (int s = 0; s < nvalid; ++s) M = fmaxf(M, ws_ml[((b * nsplit + s) * DA_H + h) * 2]);
  float L = 0.f, N = 0.f;
  for (int s = 0; s < nvalid; ++s) {
    const int64_t base = (b * nsplit + s) * DA_H + h;
    const float e = exp2f(ws_ml[base * 2] - M);
    L += e * ws_ml[base * 2 + 1];
    N += e * ws_o[base * DA_D + d];
  }
  out[(b * DA_H + h) * DA_D + d] = f2bf(N / L);
}

static int64_t workspace_bytes_for(int64_t B, const DecodeSplit &sp) {
  if (sp.nsplit <= 1) return 0;
  return B * sp.nsplit * DA_H * (DA_D + 2) * static_cast<int64_t>(sizeof(float));
}


// ---- groups of sequences that share one prefix (GSPO: G samples of one window) ----------------------
//
// A sequence of group p attends to the group's prefix rows (frames + BOS, one copy in the prefix cache
// [P, S_pre, 2, 64]) followed by its own rows (sampled tokens, own-row cache [B, S_own, 2, 64]).
// One launch: a workgroup per (part, subgroup, KV head), where a subgroup is G consecutive members of a
// prefix group (the whole group, or 1 / msplit of it). Its query columns are the 4 heads of that KV head
// for its G members (4 G columns), and it walks one tile space: the prefix tiles (every column attends),
// then the own-row tiles of members 0..G-1 (only that member's 4 columns attend; the others are masked).
// The tile space is cut into `nparts` equal parts, so every wave runs a long software-pipelined loop.
// With nparts > 1 each part leaves a partial (max, sum, unnormalised output) per column and a small
// combine kernel merges the parts of each (sequence, head); with one part the workgroup writes the bf16
// output itself. With msplit > 1 the subgroups of one prefix group read the same prefix rows, launched
// next to each other on one XCD, so the second read comes from its L2.

// resident workgroups per CU the part count aims for, per wave count (each wave's K / V ring takes 16 KB of
// LDS)
constexpr int gu_wg_per_cu(int waves) { return waves >= 8 ? 1 : 2; }
constexpr int GU_TILE = 32;
// Each wave streams its K / V tiles through a ring of two LDS stages (K tile 4 KB, V tile 4 KB) by direct
// global->LDS loads. A tile row (one KV head: 64 bf16 = 128 B) keeps its 16-byte chunk c in slot c ^ swz(row),
// which spreads the 16 rows of an MFMA fragment read over all bank groups.
constexpr int GU_TILEB = GU_TILE * 128;   // 4 KB
constexpr int GU_STAGEB = 2 * GU_TILEB;   // K + V
constexpr int GU_WAVEB = 2 * GU_STAGEB;   // two stages per wave
__device__ __forceinline__ int gu_swz(int row) { return (row >> 1) & 7; }
// s_waitcnt immediate: vmcnt <= n, expcnt / lgkmcnt unconstrained
constexpr int gu_vmcnt(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }
typedef __attribute__((address_space(3))) void gu_lds_void_t;
// Loads whose wait the kernel places itself: the compiler's wait placement does not count the direct
// global->LDS loads, so after them it would wait for every outstanding load before the first use of an
// ordinary load's result, the ring's prefetch included. These loads are invisible to it; each use follows
// an explicit s_waitcnt and a register touch (gu_touch) that orders the use after it.
__device__ __forceinline__ u32x4 gu_load16(const void *ptr) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(ptr));
  return v;
}
__device__ __forceinline__ int gu_load4(const void *ptr) {
  int v;
  asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(ptr));
  return v;
}
template <typename T>
__device__ __forceinline__ void gu_touch(T &v) { asm volatile("" : "+v"(v)); }
// one 32-row tile of K or V (rows row0 .. row0 + 31 of base, clamped to clamp - 1) into dst: 4 direct loads,
// instruction j -> rows 8 j .. 8 j + 7, lane l -> row 8 j + l / 8, LDS slot l % 8 holding chunk (l % 8) ^ swz(row)
__device__ __forceinline__ void gu_issue_tile(char *dst, const bf16_t *base, int64_t stride, int row0, int clamp,
                                              int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 8 * j + (lane >> 3);
    int rr = row0 + r;
    rr = rr < clamp ? rr : clamp - 1;
    const int gc = (lane & 7) ^ gu_swz(r);
    __builtin_amdgcn_global_load_lds(base + static_cast<int64_t>(rr) * stride + 8 * gc,
                                     (gu_lds_void_t *)(dst + 1024 * j), 16, 0, 0);
  }
}
// The four transposed V fragments of lds_tr_frag (dt = 0..3: column 16 dt + lane % 16 at rows 4 g .. + 3 and
// 16 + 4 g .. + 3) from a swizzled tile: eight ds_read_b64_tr_b16 in one asm statement that also waits for them.
// (Written as the builtin, each transpose read makes the compiler first wait for every outstanding direct
// global->LDS load, which would drain the ring's prefetch.)
__device__ __forceinline__ void gu_tr_frags(const char *tile, int lane, bf16x8 (&va)[4]) {
  const int g = lane >> 4, s = lane & 15;
  const int r = 4 * g + (s >> 2), h = (s & 3) >> 1, half = 8 * (s & 1);
  unsigned a[8];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    a[2 * dt] = static_cast<unsigned>(reinterpret_cast<uintptr_t>(tile + r * 128 + 16 * ((2 * dt + h) ^ gu_swz(r)) + half));
    a[2 * dt + 1] = static_cast<unsigned>(
        reinterpret_cast<uintptr_t>(tile + (r + 16) * 128 + 16 * ((2 * dt + h) ^ gu_swz(r + 16)) + half));
  }
  s16x4_t v[8];
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n\t"
      "ds_read_b64_tr_b16 %1, %9\n\t"
      "ds_read_b64_tr_b16 %2, %10\n\t"
      "ds_read_b64_tr_b16 %3, %11\n\t"
      "ds_read_b64_tr_b16 %4, %12\n\t"
      "ds_read_b64_tr_b16 %5, %13\n\t"
      "ds_read_b64_tr_b16 %6, %14\n\t"
      "ds_read_b64_tr_b16 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
  typedef short s16x8_t __attribute__((ext_vector_type(8)));
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    va[dt] = __builtin_bit_cast(bf16x8, s16x8_t{v[2 * dt][0], v[2 * dt][1], v[2 * dt][2], v[2 * dt][3],
                                                v[2 * dt + 1][0], v[2 * dt + 1][1], v[2 * dt + 1][2], v[2 * dt + 1][3]});
}

template <int G, int GU_WAVES>
__global__ __launch_bounds__(GU_WAVES * 64) void grouped_attn_kernel(
    const bf16_t *__restrict__ q, const bf16_t *__restrict__ kp, const bf16_t *__restrict__ vp,
    const int32_t *__restrict__ pre_len, int64_t stride_pb, int64_t stride_ps, int64_t pre_max,
    const bf16_t *__restrict__ ks, const bf16_t *__restrict__ vs, const int32_t *__restrict__ own_len,
    int64_t stride_sb, int64_t stride_ss, int64_t own_max, int nparts, int msplit, float *__restrict__ ws_o,
    float *__restrict__ ws_ml, bf16_t *__restrict__ out, float scale_log2) {
  constexpr int NC = 4 * G;            // query columns of one KV head (G members x 4 heads)
  constexpr int NCB = (NC + 15) / 16;  // 16-column MFMA blocks
  constexpr int LDS_V = GU_WAVES * GU_WAVEB;
  constexpr int LDS_M = (GU_WAVES * NC * 64 + 2 * GU_WAVES * NC) * 4;
  constexpr int LDS_BOS = LDS_V > LDS_M ? LDS_V : LDS_M;  // the prefix's last K / V row (256 B), past the rest
  __shared__ __attribute__((aligned(16))) char smem[LDS_BOS + 256];

  // wave-uniform values go through readfirstlane / readlane so the tile loop and segment search stay scalar
  const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, g = lane >> 4;
  // 1-D grid, XCD-aware: workgroup i runs on XCD i % 8, which takes a contiguous range of the logical order
  // (subgroup, part, KV head) with the KV head fastest, so the two workgroups that read the two halves of
  // the same 256-byte cache rows run back to back on one XCD, and so do the subgroups of one prefix group
  // (a bijection for any count)
  const int tiles = gridDim.x, pid = blockIdx.x, xcd = pid & 7, idx = pid >> 3;
  const int lt_id = xcd * (tiles >> 3) + min(xcd, tiles & 7) + idx;
  const int kvh = lt_id & 1, part = (lt_id >> 1) % nparts, p = (lt_id >> 1) / nparts;  // p: subgroup
  const int pp = p / msplit;                                                            // its prefix group

  // The part's tiles: its static share of the prefix tiles (sized by pre_max, so they are known before any
  // length is read; tiles past the group's actual prefix length are fully masked), then its share of the
  // own-row tiles of all G members taken as one sequence (member 0's tiles, then member 1's, ...). Both
  // shares are equal cuts, so parts are balanced for any part count. The tiles cover the prefix rows but its
  // last (a window's BOS row, 2049 = 64 x 32 + 1 at the rollout's shape), which the last wavefront of the last
  // part adds by VALU after its tiles: a 32-row tile for that one row would make the workgroup's tile count
  // 1 or 5 (mod 8) at every step, so one to five wavefronts would run one more tile than the rest.
  const int tp_all = static_cast<int>((pre_max - 1 + GU_TILE - 1) / GU_TILE);
  const int pt0 = tp_all * part / nparts, npre = tp_all * (part + 1) / nparts - pt0;
  const bf16_t *kpre = kp + pp * stride_pb + kvh * DA_D, *vpre = vp + pp * stride_pb + kvh * DA_D;

  struct TileRef {
    const bf16_t *k, *v;
    int64_t stride;
    int row0, len, clamp, seg, mc;  // seg: 0 = prefix, 1 + m = member m's own rows; mc: member cursor
  };
  char *const wring = smem + wid * GU_WAVEB;  // this wave's two stages
  // the first tile is a prefix tile whenever wid < npre: its loads need no length (rows clamped to pre_max - 1,
  // always valid; its mask waits for the length)
  TileRef cur;
  cur.k = kpre;
  cur.v = vpre;
  cur.stride = stride_ps;
  cur.row0 = (pt0 + wid) * GU_TILE;
  cur.len = 0;
  cur.clamp = static_cast<int>(pre_max);
  cur.seg = 0;
  cur.mc = 0;
  // the wave's first two tiles t0 = wid and t0 + W are prefix tiles whenever they are inside the static prefix
  // share: their loads go out with the query and length loads, before any length is known
  const bool spec = wid < npre, spec2 = wid + GU_WAVES < npre;

  // Q^T fragments (loaded before the lengths, so both round trips overlap, and before the first tile's K / V, see
  // below): column j = 16 cb + col -> member
  // j / 4, head kvh * 4 + j % 4, the two 32-wide halves of D
  // (a column past NC loads column NC - 1 and is zeroed once the loads have landed)
  u32x4 qraw[NCB][2];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int j = min(16 * cb + col, NC - 1);
    const int64_t row = static_cast<int64_t>(p) * G + j / 4;
#pragma unroll
    for (int c = 0; c < 2; ++c)
      qraw[cb][c] = gu_load16(q + (row * DA_H + kvh * 4 + (j & 3)) * DA_D + 32 * c + 8 * g);
  }
  // lengths, per wave in registers: lane m < G = member m's own rows, lane G = the prefix; incl = inclusive
  // prefix sum of the members' own-tile counts
  // (loaded without a branch, so no wait lands between these loads and the first tiles' loads: a lane past the
  // members reads member G - 1's entry, and the prefix length is one scalar load)
  int own_raw = gu_load4(own_len + static_cast<int64_t>(p) * G + (lane < G ? lane : G - 1));
  const int pre_raw = pre_len[pp];
  // The first two tiles' K / V go out right after the query and length loads, before the lengths are known.
  TileRef nxt = cur;
  nxt.row0 = (pt0 + wid + GU_WAVES) * GU_TILE;
  // Then the query and length loads are waited for by a count that leaves those tiles in flight, in the same
  // branch that issued them (after a join of paths with different load counts the compiler would drain all).
  if (spec2) {
    gu_issue_tile(wring, cur.k, cur.stride, cur.row0, cur.clamp, lane);
    gu_issue_tile(wring + GU_TILEB, cur.v, cur.stride, cur.row0, cur.clamp, lane);
    gu_issue_tile(wring + GU_STAGEB, nxt.k, nxt.stride, nxt.row0, nxt.clamp, lane);
    gu_issue_tile(wring + GU_STAGEB + GU_TILEB, nxt.v, nxt.stride, nxt.row0, nxt.clamp, lane);
    asm volatile("s_waitcnt vmcnt(16)");
  } else if (spec) {
    gu_issue_tile(wring, cur.k, cur.stride, cur.row0, cur.clamp, lane);
    gu_issue_tile(wring + GU_TILEB, cur.v, cur.stride, cur.row0, cur.clamp, lane);
    asm volatile("s_waitcnt vmcnt(8)");
  } else {
    asm volatile("s_waitcnt vmcnt(0)");
  }
  gu_touch(own_raw);
  bf16x8 bq[NCB][2];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      gu_touch(qraw[cb][c]);
      bq[cb][c] = __builtin_bit_cast(bf16x8, 16 * cb + col < NC ? qraw[cb][c] : u32x4{0u, 0u, 0u, 0u});
    }
  int len = 0, cnt = 0;
  if (lane < G) {
    const int64_t l = own_raw;
    len = static_cast<int>(l < 0 ? 0 : (l > own_max ? own_max : l));
    cnt = (len + GU_TILE - 1) / GU_TILE;
  } else if (lane == G) {
    const int64_t l = pre_raw;
    len = static_cast<int>(l < 1 ? 1 : (l > pre_max ? pre_max : l));
  }
  int incl = cnt;
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  const int own_all = __builtin_amdgcn_readlane(incl, G - 1);
  const int ou0 = static_cast<int>(static_cast<int64_t>(own_all) * part / nparts);
  const int T = npre + static_cast<int>(static_cast<int64_t>(own_all) * (part + 1) / nparts) - ou0;  // tiles
  // The wavefront that adds the prefix's last row after its tiles fetches that row now, by one direct load into
  // LDS (lanes 0-31: its K half of the row, lanes 32-63: its V half, 4 bytes each), so the row is there when the
  // tiles are done. A load issued after the first tiles' loads only makes the tile loop's counted waits
  // stricter (they count the loads issued after the tile they need).
  const bool bos_wave = wid == GU_WAVES - 1 && part == nparts - 1;
  if (bos_wave) {
    const int brow = __builtin_amdgcn_readlane(len, G) - 1;  // 0 .. pre_max - 1
    const bf16_t *src = (lane < 32 ? kpre : vpre) + static_cast<int64_t>(brow) * stride_ps + 2 * (lane & 31);
    __builtin_amdgcn_global_load_lds(src, (gu_lds_void_t *)(smem + LDS_BOS), 4, 0, 0);
  }

  f32x4 acc[NCB][4];
  float m_run[NCB], l_run[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[cb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[cb] = -INFINITY;
    l_run[cb] = 0.f;
  }

  // local tile t -> prefix tile pt0 + t (t < npre) or own-row tile ou0 + t - npre (member found by a
  // monotone search from the cursor), first row, lengths, row pointers
  auto locate = [&](int t, int m) {
    TileRef r;
    if (t < npre) {
      r.seg = 0;
      r.mc = m;
      r.len = __builtin_amdgcn_readlane(len, G) - 1;  // (the last prefix row is added apart)
      r.k = kpre;
      r.v = vpre;
      r.stride = stride_ps;
      r.row0 = (pt0 + t) * GU_TILE;
      r.clamp = static_cast<int>(pre_max);
    } else {
      const int u = ou0 + t - npre;
      while (u >= __builtin_amdgcn_readlane(incl, m)) ++m;
      r.seg = 1 + m;
      r.mc = m;
      r.len = __builtin_amdgcn_readlane(len, m);
      const int64_t b = static_cast<int64_t>(p) * G + m;
      r.k = ks + b * stride_sb + kvh * DA_D;
      r.v = vs + b * stride_sb + kvh * DA_D;
      r.stride = stride_ss;
      r.row0 = (u - (m ? __builtin_amdgcn_readlane(incl, m - 1) : 0)) * GU_TILE;
      r.clamp = r.len;
    }
    return r;
  };

  // This wave's tiles are t0 = wid, wid + W, ... (< T), two ahead in its LDS ring: tile t + 2W's K goes into
  // the stage of tile t once t's scores are formed, its V once t's V has been read. Each wait counts this
  // wave's loads issued after the ones it needs (4 per K or V tile): before the scores, t's V and tile t + W's
  // K / V; before P V, tile t + W's K / V and t + 2W's K, each while that tile exists.
  const int t0 = wid, t_end = T;
  if (t0 < t_end) {
    if (spec) {
      cur.len = __builtin_amdgcn_readlane(len, G) - 1;
    } else {
      cur = locate(t0, 0);
      gu_issue_tile(wring, cur.k, cur.stride, cur.row0, cur.clamp, lane);
      gu_issue_tile(wring + GU_TILEB, cur.v, cur.stride, cur.row0, cur.clamp, lane);
    }
    if (spec2) {
      nxt.len = cur.len;
    } else if (t0 + GU_WAVES < t_end) {
      nxt = locate(t0 + GU_WAVES, cur.mc);
      gu_issue_tile(wring + GU_STAGEB, nxt.k, nxt.stride, nxt.row0, nxt.clamp, lane);
      gu_issue_tile(wring + GU_STAGEB + GU_TILEB, nxt.v, nxt.stride, nxt.row0, nxt.clamp, lane);
    } else {
      nxt = cur;
    }
    int stage = 0;
    for (int t = t0; t < t_end; t += GU_WAVES) {
      const bool has1 = t + GU_WAVES < t_end, has2 = t + 2 * GU_WAVES < t_end;
      const TileRef nn = has2 ? locate(t + 2 * GU_WAVES, nxt.mc) : cur;
      char *const kst = wring + stage * GU_STAGEB, *const vst = kst + GU_TILEB;
      const int member = cur.seg - 1;  // -1: prefix tile, every column attends
      // an own-row tile feeds only its member's 4 columns: the other column blocks are skipped (wave-uniform)
      const int cb_only = member < 0 ? -1 : (4 * member) >> 4;
      if (has1)  // this tile's K has landed
        __builtin_amdgcn_s_waitcnt(gu_vmcnt(12));
      else
        __builtin_amdgcn_s_waitcnt(gu_vmcnt(4));
      u32x4 kf[2][2];
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int R = 16 * pb + col;
          kf[pb][c] = *reinterpret_cast<const u32x4 *>(kst + R * 128 + 16 * ((4 * c + g) ^ gu_swz(R)));
        }
      f32x4 st[2][NCB];
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          st[pb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (NCB > 1 && cb_only >= 0 && cb != cb_only) continue;
#pragma unroll
          for (int c = 0; c < 2; ++c)
            st[pb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[pb][c]), bq[cb][c],
                                                                 st[pb][cb], 0, 0, 0);
        }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // the K reads are done: the stage's K tile may be overwritten
      if (has2) gu_issue_tile(kst, nn.k, nn.stride, nn.row0, nn.clamp, lane);
      // a prefix tile inside the prefix needs no mask (the common case: a uniform branch)
      const bool full = member < 0 && cur.row0 + GU_TILE <= cur.len;
      bf16x8 pf[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        if (NCB > 1 && cb_only >= 0 && cb != cb_only) continue;
        float sv[8];
        if (full) {
#pragma unroll
          for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[pb * 4 + i] = st[pb][cb][i] * scale_log2;
        } else {
          // rows of this lane's group g that exist: 16 pb + i < nv (0 for a column of another member)
          const bool col_ok = member < 0 || ((16 * cb + col) >> 2) == member;
          const int nv = col_ok ? cur.len - cur.row0 - 4 * g : 0;
#pragma unroll
          for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              sv[pb * 4 + i] = 16 * pb + i < nv ? st[pb][cb][i] * scale_log2 : -INFINITY;
        }
        float mx = sv[0];
#pragma unroll
        for (int jj = 1; jj < 8; ++jj) mx = fmaxf(mx, sv[jj]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[cb], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;  // a column with no row yet stays empty
        // exponents are <= 0: the bare v_exp_f32 (no range reduction needed)
        float e[8], ps = 0.f;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          e[jj] = __builtin_amdgcn_exp2f(sv[jj] - m_use);
          ps += e[jj];
        }
        pf[cb] = __builtin_bit_cast(bf16x8, u32x4{pack_bf(e[0], e[1]), pack_bf(e[2], e[3]), pack_bf(e[4], e[5]),
                                                   pack_bf(e[6], e[7])});
        // rescale only when some column's running max moved (alpha is exactly 1 otherwise)
        if (__builtin_amdgcn_ballot_w64(m_new != m_run[cb])) {
          const float alpha = __builtin_amdgcn_exp2f(m_run[cb] - m_use);
          l_run[cb] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) acc[cb][dt] *= alpha;
        }
        l_run[cb] += ps;
        m_run[cb] = m_new;
      }
      if (has2)  // this tile's V has landed
        __builtin_amdgcn_s_waitcnt(gu_vmcnt(12));
      else if (has1)
        __builtin_amdgcn_s_waitcnt(gu_vmcnt(8));
      else
        __builtin_amdgcn_s_waitcnt(gu_vmcnt(0));
      bf16x8 va[4];
      gu_tr_frags(vst, lane, va);  // (waits for its reads: the stage's V tile may then be overwritten)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
          if (NCB == 1 || cb_only < 0 || cb == cb_only)
            acc[cb][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pf[cb], acc[cb][dt], 0, 0, 0);
      }
      if (has2) gu_issue_tile(vst, nn.v, nn.stride, nn.row0, nn.clamp, lane);
      cur = nxt;
      nxt = nn;
      stage ^= 1;
    }
    __builtin_amdgcn_s_waitcnt(gu_vmcnt(0));  // the ring's last loads, before its LDS is reused below
  }
  // The prefix's last row (row pre_len - 1) in the last wavefront of the last part, with the tile loop's rounding
  // points: the score over the 64 d (this lane's 16 q values, the q fragments' layout, then the column's 4 lanes),
  // the running-max rescale, the fp32 exponential into the row sum and its bf16 rounding into the output.
  if (bos_wave) {
    __builtin_amdgcn_s_waitcnt(gu_vmcnt(0));  // the row's load (a wavefront without tiles has not waited yet)
    const char *kb = smem + LDS_BOS, *vb = kb + 128;
    const u32x4 kr[2] = {*reinterpret_cast<const u32x4 *>(kb + 16 * g),
                         *reinterpret_cast<const u32x4 *>(kb + 64 + 16 * g)};
    u32x2 vr[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) vr[dt] = *reinterpret_cast<const u32x2 *>(vb + 32 * dt + 8 * g);
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      float sc = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x4 qq = __builtin_bit_cast(u32x4, bq[cb][c]);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc += lo_bf(qq[e]) * lo_bf(kr[c][e]) + hi_bf(qq[e]) * hi_bf(kr[c][e]);
      }
      sc += __shfl_xor(sc, 16, 64);
      sc += __shfl_xor(sc, 32, 64);
      const float sv = sc * scale_log2;
      const float m_new = fmaxf(m_run[cb], sv);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float e = __builtin_amdgcn_exp2f(sv - m_use);
      if (__builtin_amdgcn_ballot_w64(m_new != m_run[cb])) {
        const float alpha = __builtin_amdgcn_exp2f(m_run[cb] - m_use);
        l_run[cb] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) acc[cb][dt] *= alpha;
      }
      m_run[cb] = m_new;
      l_run[cb] += g == 0 ? e : 0.f;  // (the row sum is reduced over the column's 4 lanes below)
      const float pb = round_bf(e);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        acc[cb][dt][0] = fmaf(pb, lo_bf(vr[dt][0]), acc[cb][dt][0]);
        acc[cb][dt][1] = fmaf(pb, hi_bf(vr[dt][0]), acc[cb][dt][1]);
        acc[cb][dt][2] = fmaf(pb, lo_bf(vr[dt][1]), acc[cb][dt][2]);
        acc[cb][dt][3] = fmaf(pb, hi_bf(vr[dt][1]), acc[cb][dt][3]);
      }
    }
  }
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    l_run[cb] += __shfl_xor(l_run[cb], 16, 64);
    l_run[cb] += __shfl_xor(l_run[cb], 32, 64);
  }
  __syncthreads();
  float *Os = reinterpret_cast<float *>(smem);  // [WAVES][NC][64]
  float *Ms = Os + GU_WAVES * NC * 64;           // [WAVES][NC]
  float *Ls = Ms + GU_WAVES * NC;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int j = 16 * cb + col;
    if (j < NC) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) *reinterpret_cast<f32x4 *>(&Os[(wid * NC + j) * 64 + 16 * dt + 4 * g]) = acc[cb][dt];
      if (g == 0) {
        Ms[wid * NC + j] = m_run[cb];
        Ls[wid * NC + j] = l_run[cb];
      }
    }
  }
  __syncthreads();
  // partial of (subgroup p, KV head, part, column j); a column no row of this part reaches: (-inf, 0, 0).
  // One part: the output itself, bf16(N / L) -- what the combine computes from a single partial, bit for
  // bit (its weight is exp2(0) = 1); every column then has at least the first prefix row. A thread merges
  // 4 consecutive d of one column (16-byte LDS reads, one 8-byte store).
  for (int o = threadIdx.x; o < NC * 16; o += GU_WAVES * 64) {
    const int j = o >> 4, d0 = (o & 15) * 4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < GU_WAVES; ++w) M = fmaxf(M, Ms[w * NC + j]);
    float L = 0.f;
    f32x4 N = {0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < GU_WAVES; ++w) {
        const float e = exp2f(Ms[w * NC + j] - M);
        L += e * Ls[w * NC + j];
        const f32x4 ow = *reinterpret_cast<const f32x4 *>(&Os[(w * NC + j) * 64 + d0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) N[i] += e * ow[i];
      }
    }
    if (nparts == 1) {
      const int64_t b = static_cast<int64_t>(p) * G + j / 4;
      *reinterpret_cast<u32x2 *>(out + (b * DA_H + kvh * 4 + (j & 3)) * DA_D + d0) =
          u32x2{pack_bf(N[0] / L, N[1] / L), pack_bf(N[2] / L, N[3] / L)};
      continue;
    }
    const int64_t base = ((static_cast<int64_t>(p) * DA_HKV + kvh) * nparts + part) * NC + j;
    *reinterpret_cast<f32x4 *>(ws_o + base * DA_D + d0) = N;
    if (d0 == 0) {
      ws_ml[base * 2] = M;
      ws_ml[base * 2 + 1] = L;
    }
  }
}

// out[b, h] = merge of the NP partials of b's column (member b % G, head h) in its group's KV head; all
// partial loads are issued before the first use (NP is a compile-time count)
template <int NP>
__global__ __launch_bounds__(DA_H * DA_D) void grouped_combine_kernel(const float *__restrict__ ws_o,
                                                                      const float *__restrict__ ws_ml,
                                                                      bf16_t *__restrict__ out, int G) {
  const int64_t b = blockIdx.x;
  const int h = threadIdx.x / DA_D, d = threadIdx.x % DA_D;
  const int64_t p = b / G;
  const int NC = 4 * G;
  const int j = 4 * static_cast<int>(b % G) + (h & 3);
  const int64_t base0 = (p * DA_HKV + (h >> 2)) * NP * NC + j;
  float2 ml[NP];
  float o[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int64_t base = base0 + static_cast<int64_t>(k) * NC;
    ml[k] = *reinterpret_cast<const float2 *>(ws_ml + base * 2);
    o[k] = ws_o[base * DA_D + d];
  }
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < NP; ++k) M = fmaxf(M, ml[k].x);
  float L = 0.f, N = 0.f;
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const float e = ml[k].x == -INFINITY ? 0.f : exp2f(ml[k].x - M);
    L += e * ml[k].y;
    N += e * o[k];
  }
  out[(b * DA_H + h) * DA_D + d] = f2bf(N / L);
}

struct GroupedLayout {
  int gq;      // query members per workgroup (the kernel's G)
  int msplit;  // subgroups per prefix group (G / gq)
  int waves;   // wavefronts per workgroup
  int nparts;  // parts of each subgroup's tile space (1: no combine launch)
  int64_t o, ml, total;  // offsets / size in floats
};

// Groups of G >= 8 whose halves alone fill a resident round of 8-wave workgroups are split by member: each
// half walks the whole tile space (one part, no combine) with half the query columns, which also halves the
// masked work of the own-row tiles. Otherwise the whole group is one subgroup and its tile space is cut into
// parts: one resident round of workgroups over the CUs, and at least one tile per wave at the longest lengths.
static GroupedLayout grouped_layout(int64_t B, int G, int64_t pre_max, int64_t own_max, int cus) {
  GroupedLayout L{};
  if (G >= 8 && (B / G) * 2 * DA_HKV >= cus) {
    L.gq = G / 2;
    L.msplit = 2;
    L.waves = 8;  // (16 waves measured slower)
    L.nparts = 1;
  } else {
    L.gq = G;
    L.msplit = 1;
    L.waves = G == 8 ? 8 : 4;
    const int64_t pairs = (B / G) * DA_HKV;
    const int64_t target = static_cast<int64_t>(cus) * gu_wg_per_cu(L.waves);
    int64_t np = (target + pairs - 1) / pairs;
    const int64_t tmax = (pre_max + GU_TILE - 1) / GU_TILE + G * ((own_max + GU_TILE - 1) / GU_TILE);
    const int64_t cap = tmax / L.waves;
    if (np > cap) np = cap;
    if (np > 16) np = 16;  // the combine kernel is instantiated for 1 .. 16 parts
    if (np < 1) np = 1;
    L.nparts = static_cast<int>(np);
  }
  const int64_t cols = (B / L.gq) * DA_HKV * L.nparts * 4 * L.gq;
  L.o = 0;
  L.ml = cols * DA_D;
  L.total = L.ml + cols * 2;
  return L;
}

// Psub = subgroups (B / gq)
template <int G, int W>
static void launch_grouped(const bf16_t *q, const bf16_t *kp, const bf16_t *vp, const int32_t *pre_len,
                           int64_t Psub, int64_t stride_pb, int64_t stride_ps, int64_t pre_max, const bf16_t *ks,
                           const bf16_t *vs, const int32_t *own_len, int64_t stride_sb, int64_t stride_ss,
                           int64_t own_max, int nparts, int msplit, float *ws_o, float *ws_ml, bf16_t *out,
                           float scale_log2, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(Psub * nparts * DA_HKV));
  grouped_attn_kernel<G, W><<<grid, W * 64, 0, s>>>(q, kp, vp, pre_len, stride_pb, stride_ps, pre_max, ks, vs,
                                                    own_len, stride_sb, stride_ss, own_max, nparts, msplit, ws_o,
                                                    ws_ml, out, scale_log2);
}
}  // namespace vk

using namespace vk;

extern "C" int vk_decode_attention_workspace(int64_t B, int32_t H, int64_t max_len, int64_t *bytes) {
  VK_CHECK_ARG(bytes && B >= 0 && max_len > 0 && H == DA_H, "decode_attention_workspace: bad arguments");
  *bytes = workspace_bytes_for(B, decode_split(B, max_len, device_cus_cached()));
  return VK_OK;
}

// Argument checks shared by both decode-attention entry points (status VK_OK when the launch may go ahead).
static int check_decode_args(const void *q, const void *k_cache, const void *v_cache, const int32_t *lengths,
                             const int32_t *rows, int64_t cache_rows, void *out, int64_t B, int32_t H, int32_t HKV,
                             int32_t D, int64_t stride_b, int64_t stride_s, int64_t max_len) {
  VK_CHECK_ARG(q && k_cache && v_cache && lengths && out, "decode_attention: null pointer");
  VK_CHECK_ARG(cache_rows > 0, "decode_attention: the cache must hold at least one sequence row");
  VK_CHECK_ARG(rows != nullptr || cache_rows >= B,
               "decode_attention: %lld sequences but the cache holds %lld rows (pass rows to map them)",
               static_cast<long long>(B), static_cast<long long>(cache_rows));
  if (H != DA_H || HKV != DA_HKV || D != DA_D)
    return fail(VK_ERR_UNSUPPORTED, "decode_attention: built for H=8 HKV=2 D=64 (got %d/%d/%d)", H, HKV, D);
  VK_CHECK_ARG(B >= 0 && max_len > 0 && stride_s >= DA_ROW && stride_s % 8 == 0 && stride_b % 8 == 0,
               "decode_attention: bad strides / sizes");
  VK_CHECK_ARG(vk_aligned16(q) && vk_aligned16(k_cache) && vk_aligned16(v_cache),
               "decode_attention: q and the caches must be 16-byte aligned");
  VK_CHECK_ARG(B < 65536, "decode_attention: B must be < 65536");
  return VK_OK;
}

// The split kernel (when the key range is split, partials go to `workspace`) and its combine launch.
static int launch_decode_attention(const void *q, const void *k_cache, const void *v_cache, const int32_t *lengths,
                                   const int32_t *rows, int64_t cache_rows, void *out, int64_t B, int64_t stride_b,
                                   int64_t stride_s, int64_t max_len, const DecodeSplit &sp, void *workspace,
                                   void *stream) {
  const float scale_log2 = static_cast<float>(1.0 / sqrt(static_cast<double>(DA_D)) * 1.4426950408889634);
  hipStream_t s = VK_STREAM(stream);
  const dim3 grid(sp.nsplit, static_cast<unsigned>(B));
  if (sp.nsplit == 1) {
    decode_attn_kernel<false><<<grid, DA_WAVES * 64, 0, s>>>(
        static_cast<const bf16_t *>(q), static_cast<const bf16_t *>(k_cache), static_cast<const bf16_t *>(v_cache),
        lengths, rows, cache_rows, static_cast<bf16_t *>(out), stride_b, stride_s, max_len, sp.tps, 1, nullptr,
        nullptr, scale_log2);
    return launch_status("decode_attention");
  }
  float *ws_o = static_cast<float *>(workspace);
  float *ws_ml = ws_o + B * sp.nsplit * DA_H * DA_D;
  decode_attn_kernel<true><<<grid, DA_WAVES * 64, 0, s>>>(
      static_cast<const bf16_t *>(q), static_cast<const bf16_t *>(k_cache), static_cast<const bf16_t *>(v_cache),
      lengths, rows, cache_rows, static_cast<bf16_t *>(out), stride_b, stride_s, max_len, sp.tps, sp.nsplit, ws_o,
      ws_ml, scale_log2);
  int st = launch_status("decode_attention");
  if (st != VK_OK) return st;
  decode_attn_combine<<<static_cast<unsigned>(B), DA_H * DA_D, 0, s>>>(
      ws_o, ws_ml, lengths, rows, cache_rows, static_cast<bf16_t *>(out), max_len, sp.tps, sp.nsplit);
  return launch_status("decode_attention_combine");
}

extern "C" int vk_decode_attention(const void *q, const void *k_cache, const void *v_cache, const int32_t *lengths,
                                   const int32_t *rows, int64_t cache_rows, void *out, int64_t B, int32_t H,
                                   int32_t HKV, int32_t D, int64_t stride_b, int64_t stride_s, int64_t max_len,
                                   void *workspace, int64_t workspace_bytes, void *stream) {
  const int st = check_decode_args(q, k_cache, v_cache, lengths, rows, cache_rows, out, B, H, HKV, D, stride_b,
                                   stride_s, max_len);
  if (st != VK_OK || B == 0) return st;
  const DecodeSplit sp = decode_split(B, max_len, device_cus_cached());
  const int64_t need = workspace_bytes_for(B, sp);
  VK_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace != nullptr),
               "decode_attention: workspace of %lld bytes needed", static_cast<long long>(need));
  return launch_decode_attention(q, k_cache, v_cache, lengths, rows, cache_rows, out, B, stride_b, stride_s, max_len,
                                 sp, workspace, stream);
}

// ---- decode attention without an allocation ------------------------------------------------------------
// The key-split partials live in a file-scope device array instead of a caller-supplied workspace. Each GPU
// holds its own copy (for the life of the process); the host reaches it through the address that
// hipGetSymbolAddress returns on that device, looked up once per device and kept here -- the array's name in
// host code is only a stand-in, never a device address. Nothing in it needs clearing between calls: the
// combine kernel reads only the partials of splits that the same call's split kernel wrote.
constexpr int64_t kNoallocScratchBytes = int64_t(4) << 20;
static __device__ __align__(256) float scratch[kNoallocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

static int scratch_of_current_device(void **ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return fail(VK_ERR_LAUNCH, "decode_attention_noalloc: no current HIP device");
  if (dev >= kMaxDevices) return fail(VK_ERR_UNSUPPORTED, "decode_attention_noalloc: device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(VK_ERR_LAUNCH, "decode_attention_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return VK_OK;
}

extern "C" int vk_decode_attention_noalloc(const void *q, const void *k_cache, const void *v_cache,
                                           const int32_t *lengths, const int32_t *rows, int64_t cache_rows,
                                           void *out, int64_t B, int32_t H, int32_t HKV, int32_t D, int64_t stride_b,
                                           int64_t stride_s, int64_t max_len, void *stream) {
  const int st = check_decode_args(q, k_cache, v_cache, lengths, rows, cache_rows, out, B, H, HKV, D, stride_b,
                                   stride_s, max_len);
  if (st != VK_OK || B == 0) return st;
  const DecodeSplit sp = decode_split(B, max_len, device_cus_cached());
  const int64_t need = workspace_bytes_for(B, sp);
  VK_CHECK_ARG(need <= kNoallocScratchBytes,
               "decode_attention_noalloc: %lld sequences x %d key splits need %lld bytes of partials, more than the "
               "%lld-byte static scratch (use vk_decode_attention with a workspace)",
               static_cast<long long>(B), sp.nsplit, static_cast<long long>(need),
               static_cast<long long>(kNoallocScratchBytes));
  void *ws = nullptr;
  if (need > 0) {
    const int rc = scratch_of_current_device(&ws);
    if (rc != VK_OK) return rc;
  }
  return launch_decode_attention(q, k_cache, v_cache, lengths, rows, cache_rows, out, B, stride_b, stride_s, max_len,
                                 sp, ws, stream);
}

extern "C" int vk_decode_attention_grouped_workspace(int64_t B, int32_t G, int64_t pre_max, int64_t suf_max,
                                                     int64_t *bytes) {
  VK_CHECK_ARG(bytes && B > 0 && G > 0 && B % G == 0 && pre_max > 0 && suf_max > 0,
               "decode_attention_grouped_workspace: bad arguments");
  *bytes = grouped_layout(B, G, pre_max, suf_max, device_cus_cached()).total * static_cast<int64_t>(sizeof(float));
  return VK_OK;
}

extern "C" int vk_decode_attention_grouped_layout(int64_t B, int32_t G, int64_t pre_max, int64_t suf_max,
                                                  int32_t *members, int32_t *parts) {
  VK_CHECK_ARG(members && parts && B > 0 && G > 0 && B % G == 0 && pre_max > 0 && suf_max > 0,
               "decode_attention_grouped_layout: bad arguments");
  const GroupedLayout L = grouped_layout(B, G, pre_max, suf_max, device_cus_cached());
  *members = L.gq;
  *parts = L.nparts;
  return VK_OK;
}

extern "C" int vk_decode_attention_grouped(const void *q, const void *k_prefix, const void *v_prefix,
                                           const int32_t *prefix_len, int64_t stride_pb, int64_t stride_ps,
                                           int64_t pre_max, const void *k_suffix, const void *v_suffix,
                                           const int32_t *suffix_len, int64_t stride_sb, int64_t stride_ss,
                                           int64_t suf_max, void *out, int64_t B, int32_t G, int32_t H, int32_t HKV,
                                           int32_t D, void *workspace, int64_t workspace_bytes, void *stream) {
  VK_CHECK_ARG(q && k_prefix && v_prefix && prefix_len && k_suffix && v_suffix && suffix_len && out && workspace,
               "decode_attention_grouped: null pointer");
  if (H != DA_H || HKV != DA_HKV || D != DA_D)
    return fail(VK_ERR_UNSUPPORTED, "decode_attention_grouped: built for H=8 HKV=2 D=64 (got %d/%d/%d)", H, HKV, D);
  if (G != 2 && G != 4 && G != 8 && G != 16)
    return fail(VK_ERR_UNSUPPORTED, "decode_attention_grouped: group size must be 2, 4, 8 or 16 (got %d)", G);
  VK_CHECK_ARG(B > 0 && B % G == 0 && B < 65536 && pre_max > 0 && suf_max > 0, "decode_attention_grouped: sizes");
  VK_CHECK_ARG(stride_ps >= DA_ROW && stride_ss >= DA_ROW && stride_ps % 8 == 0 && stride_ss % 8 == 0 &&
                   stride_pb % 8 == 0 && stride_sb % 8 == 0,
               "decode_attention_grouped: strides");
  VK_CHECK_ARG(vk_aligned16(q) && vk_aligned16(k_prefix) && vk_aligned16(v_prefix) && vk_aligned16(k_suffix) &&
                   vk_aligned16(v_suffix),
               "decode_attention_grouped: alignment");
  const GroupedLayout L = grouped_layout(B, G, pre_max, suf_max, device_cus_cached());
  VK_CHECK_ARG(workspace_bytes >= L.total * static_cast<int64_t>(sizeof(float)),
               "decode_attention_grouped: workspace of %lld bytes needed",
               static_cast<long long>(L.total * sizeof(float)));
  const float scale_log2 = static_cast<float>(1.0 / sqrt(static_cast<double>(DA_D)) * 1.4426950408889634);
  hipStream_t s = VK_STREAM(stream);
  float *ws = static_cast<float *>(workspace);
  const auto qb = static_cast<const bf16_t *>(q);
  const auto kp = static_cast<const bf16_t *>(k_prefix);
  const auto vp = static_cast<const bf16_t *>(v_prefix);
  const auto ks = static_cast<const bf16_t *>(k_suffix);
  const auto vs = static_cast<const bf16_t *>(v_suffix);
  bf16_t *ob = static_cast<bf16_t *>(out);
#define VK_GROUPED(GG, WW)                                                                                     \
  launch_grouped<GG, WW>(qb, kp, vp, prefix_len, B / L.gq, stride_pb, stride_ps, pre_max, ks, vs, suffix_len,    \
                         stride_sb, stride_ss, suf_max, L.nparts, L.msplit, ws + L.o, ws + L.ml, ob, scale_log2, s)
  if (L.gq == 2) VK_GROUPED(2, 4);
  else if (L.gq == 4 && L.waves == 8) VK_GROUPED(4, 8);
  else if (L.gq == 4) VK_GROUPED(4, 4);
  else if (L.gq == 8) VK_GROUPED(8, 8);
  else VK_GROUPED(16, 4);
#undef VK_GROUPED
  const int rc = launch_status("decode_attention_grouped");
  if (rc != VK_OK || L.nparts == 1) return rc;  // one part: the kernel wrote the output
  const dim3 cgrid(static_cast<unsigned>(B));
  switch (L.nparts) {
#define VK_COMBINE(NP) \
  case NP: grouped_combine_kernel<NP><<<cgrid, DA_H * DA_D, 0, s>>>(ws + L.o, ws + L.ml, ob, L.gq); break;
    VK_COMBINE(1) VK_COMBINE(2) VK_COMBINE(3) VK_COMBINE(4) VK_COMBINE(5) VK_COMBINE(6) VK_COMBINE(7)
    VK_COMBINE(8) VK_COMBINE(9) VK_COMBINE(10) VK_COMBINE(11) VK_COMBINE(12) VK_COMBINE(13) VK_COMBINE(14)
    VK_COMBINE(15) VK_COMBINE(16)
#undef VK_COMBINE
    default: return fail(VK_ERR_ARG, "decode_attention_grouped: part count %d", L.nparts);
  }
  return launch_status("decode_attention_grouped combine");
}
