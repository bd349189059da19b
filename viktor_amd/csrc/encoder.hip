// The Dorado SUP encoder, the frames producer of the decoder (viktor/encoder.py:43-192): a stack of
// Conv1d + SiLU layers, then DeepNorm transformer layers with rotary, sliding-window attention and a SwiGLU
// MLP. The reference runs it on ONT's closed koi kernels (viktor/csrc/koi_tx.cpp:120-423) or in PyTorch;
// this file holds the gfx950 kernels of the HIP encoder. The transformer's matrix products run on the
// row-deterministic gemm_big kernel (vk_gemm_rows), so a chunk's frames do not depend on the other chunks
// of its batch.
//
// Chunk layout of the convolution stack ("padded layout"): layer i's activations are channels-last
// [rows, C_i] bf16 with chunk c's rows at [start[c], start[c] + len[c]) and M_i zero rows before every
// chunk (and after the last). With M_i = stride_i * M_{i+1} the input row of output row g is
// stride * g - pad for every row of the buffer, chunk boundaries included, so a convolution is one GEMM
// with a strided A operand (row g = winlen * C_in contiguous values starting at input row
// stride * g - pad) and the margins supply the zero padding of each chunk (the per-chunk Conv1d padding of
// viktor/encoder.py:166-175). Margin rows of an output are written as zeros; the last layer writes only
// data rows, compacted to [frames, C].
#include <math.h>

#include "common.h"

namespace vk {

// Chunk c with start[c] <= g (start ascending; rows before start[0] map to chunk 0). hint[g >> 8] is the
// chunk of row 256 * (g >> 8), so the walk from it is short (a 256-row block spans few chunks).
constexpr int CHUNK_HINT_SHIFT = 8;
__device__ __forceinline__ int find_chunk(const int32_t *__restrict__ start, const int32_t *__restrict__ hint, int n,
                                          int64_t g) {
  int c = hint[g >> CHUNK_HINT_SHIFT];
  while (c + 1 < n && start[c + 1] <= g) ++c;
  return c;
}

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + __expf(-v)); }

// ---- first convolution (C_in = 1): fp32 signal and weights, out = bf16(silu(bf16(conv + b))) ----------
constexpr int CF_MAX_WIN = 32;

constexpr int CF_MAX_W = 4096;  // C * winlen (weights staged in LDS)

__global__ __launch_bounds__(256) void conv_first_kernel(const float *__restrict__ sig,
                                                         const int64_t *__restrict__ sig_off,
                                                         const int32_t *__restrict__ start,
                                                         const int32_t *__restrict__ hint,
                                                         const int32_t *__restrict__ len, int n_chunks, int64_t rows,
                                                         const float *__restrict__ w, const float *__restrict__ b,
                                                         int C, int winlen, int stride, int pad,
                                                         bf16_t *__restrict__ out) {
  __shared__ float ws[CF_MAX_W];
  __shared__ float bs[512];
  for (int i = threadIdx.x; i < C * winlen; i += 256) ws[i] = w[i];
  for (int i = threadIdx.x; i < C; i += 256) bs[i] = b[i];
  __syncthreads();
  const int groups = C >> 3;  // 8 output channels per thread
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t g = idx / groups;
  const int cg = static_cast<int>(idx - g * groups);
  if (g >= rows) return;
  const int c = find_chunk(start, hint, n_chunks, g);
  const int64_t t = g - start[c];
  u32x4 res = {0u, 0u, 0u, 0u};
  if (t >= 0 && t < len[c]) {
    const int64_t n_in = static_cast<int64_t>(len[c]) * stride;  // samples of the chunk
    const float *s = sig + sig_off[c];
    float x[CF_MAX_WIN];
#pragma unroll
    for (int k = 0; k < CF_MAX_WIN; ++k) {
      const int64_t pos = t * stride - pad + k;
      x[k] = (k < winlen && pos >= 0 && pos < n_in) ? s[pos] : 0.f;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int co = cg * 8 + e;
      float acc = bs[co];
      const float *wr = ws + co * winlen;
#pragma unroll
      for (int k = 0; k < CF_MAX_WIN; ++k)
        if (k < winlen) acc = fmaf(wr[k], x[k], acc);
      o[e] = silu_f(round_bf(acc));
    }
    res = u32x4{pack_bf(o[0], o[1]), pack_bf(o[2], o[3]), pack_bf(o[4], o[5]), pack_bf(o[6], o[7])};
  }
  *reinterpret_cast<u32x4 *>(out + g * C + cg * 8) = res;
}

// ---- convolution as a strided GEMM: out[g, n] = silu(bf16(sum_k A[g, k] W[n, k] + bias[n])) ----------
// A[g, k] = a[g * lda + k] (k = tap * C_in + channel), W [N, K] in the same k order.
// Workgroup: 128 rows x 64 output channels, 4 wavefronts of 32 rows; C^T = W A^T so that each lane ends
// with 4 consecutive channels of one row (8-byte stores). LDS rows of 64 B hold one 32-wide K slice; the
// 16-byte chunk c of row r sits in slot c ^ ((r >> 2) & 3) so a fragment read (16 rows, one chunk) touches
// 16 distinct bank groups. Register-staged double buffer.
constexpr int CG_BM = 128, CG_BN = 64, CG_BK = 32;

__global__ __launch_bounds__(256) void conv_gemm_kernel(const bf16_t *__restrict__ a, int64_t lda,
                                                        const bf16_t *__restrict__ w, int K, int N,
                                                        const float *__restrict__ bias,
                                                        const int32_t *__restrict__ start,
                                                        const int32_t *__restrict__ hint,
                                                        const int32_t *__restrict__ len,
                                                        const int32_t *__restrict__ dst0, int n_chunks, int64_t rows,
                                                        int compact, bf16_t *__restrict__ out, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) char As[2][CG_BM * 64];
  __shared__ __attribute__((aligned(16))) char Ws[2][CG_BN * 64];
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int fr = lane & 15, fg = lane >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * CG_BM;
  const int n0 = blockIdx.y * CG_BN;

  // loads: A chunks q = tid, tid + 256 (row q >> 2, chunk q & 3); W chunk tid (row tid >> 2, chunk tid & 3)
  const bf16_t *asrc[2];
  int adst[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 256 * i;
    const int r = q >> 2, ch = q & 3;
    int64_t gr = m0 + r;
    gr = gr < rows ? gr : rows - 1;
    asrc[i] = a + gr * lda + 8 * ch;
    adst[i] = r * 64 + 16 * (ch ^ ((r >> 2) & 3));
  }
  const int wr = tid >> 2, wch = tid & 3;
  const bf16_t *wsrc = w + static_cast<int64_t>(n0 + wr) * K + 8 * wch;
  const int wdst = wr * 64 + 16 * (wch ^ ((wr >> 2) & 3));

  int aoff[2], woff[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int R = wid * 32 + 16 * j + fr;
    aoff[j] = R * 64 + 16 * (fg ^ ((R >> 2) & 3));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int R = 16 * i + fr;
    woff[i] = R * 64 + 16 * (fg ^ ((R >> 2) & 3));
  }

  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 ra[2], rw;
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(asrc[i] + k0);
    rw = *reinterpret_cast<const u32x4 *>(wsrc + k0);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<u32x4 *>(&As[buf][adst[i]]) = ra[i];
    *reinterpret_cast<u32x4 *>(&Ws[buf][wdst]) = rw;
  };

  const int nk = K / CG_BK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * CG_BK);
    bf16x8 af[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) af[j] = *reinterpret_cast<const bf16x8 *>(&As[buf][aoff[j]]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x8 wf = *reinterpret_cast<const bf16x8 *>(&Ws[buf][woff[i]]);
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, af[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  // epilogue: acc[i][j] lane holds C^T[channel 16 i + 4 fg + e][row 16 j + fr]
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t g = m0 + wid * 32 + 16 * j + fr;
    if (g >= rows) continue;
    const int c = find_chunk(start, hint, n_chunks, g);
    const int64_t t = g - start[c];
    const bool data = t >= 0 && t < len[c];
    if (compact && !data) continue;
    const int64_t dst = compact ? static_cast<int64_t>(dst0[c]) + t : g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = n0 + 16 * i + 4 * fg;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = data ? silu_f(round_bf(acc[i][j][e] + bias[col + e])) : 0.f;
      *reinterpret_cast<u32x2 *>(out + dst * ldo + col) = u32x2{pack_bf(o[0], o[1]), pack_bf(o[2], o[3])};
    }
  }
}

// ---- sliding-window attention with the rotary embedding applied on the fly --------------------------
// qkv [rows, 3 H 64] bf16 as the Wqkv product leaves it (q heads, then k heads, then v heads); chunk c's
// frames are rows cu[c] .. cu[c + 1] - 1 and take rotary positions 0 .. T - 1. Query i of a chunk sees keys
// j with -left <= j - i <= right (viktor/encoder.py:64-69), scale 1 / sqrt(64).
//
// Workgroup = 128 queries of one chunk x one head, 4 wavefronts of 32 query rows; K / V tiles of 64 keys
// (chunk-relative alignment, so a chunk's result does not depend on where it sits in the batch) double
// buffered in LDS; each tile serves the 128 queries. Q and K are rotated in fp32 and rounded to bf16 as
// apply_rope's output (viktor/encoder.py:36-40, 74-75): Q in registers (both halves of a rotation pair sit
// in the same lane), K by the thread that stages the key row. Products transposed as in the decoder's
// varlen kernel: S^T = K Q^T leaves each lane the scores of one query row, O^T = V^T P^T consumes them; V is
// staged transposed so that operand is two 8-byte LDS reads per lane.
constexpr int WA_D = 64, WA_Q = 128, WA_KT = 64, WA_PITCH = 72;
constexpr int WA_VTP = 68;  // keys per row of the transposed V tile (136 B: 8-byte operand reads conflict-free)

template <bool ROT>
__global__ __launch_bounds__(256, 4) void window_attn_kernel(const bf16_t *__restrict__ qkv, int64_t ld,
                                                          const int32_t *__restrict__ cu,
                                                          const int32_t *__restrict__ plan, int n_blocks, int n_chunks,
                                                          int H, const float *__restrict__ cos_t,
                                                          const float *__restrict__ sin_t, int left, int right,
                                                          float scale_log2, bf16_t *__restrict__ out, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][WA_KT * WA_PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t Vt[2][WA_D * WA_VTP];  // V^T: [d][key]
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int col = lane & 15, g = lane >> 4;

  // XCD-aware order: workgroup p runs on XCD p % 8; XCD x takes a contiguous range of (head, block) pairs,
  // so the neighbouring query blocks that re-read a chunk's keys share that XCD's L2
  const int total = n_blocks * H;
  const int p = blockIdx.x;
  const int xcd = p & 7, idx = p >> 3;
  const int q8 = total >> 3, r8 = total & 7;
  const int logical = xcd * q8 + min(xcd, r8) + idx;
  const int h = logical / n_blocks, blk = logical - h * n_blocks;
  const int chunk = plan[2 * blk], qs = plan[2 * blk + 1];
  if (chunk < 0 || chunk >= n_chunks) return;
  const int64_t row0 = cu[chunk];
  const int T = cu[chunk + 1] - static_cast<int>(row0);
  if (T <= 0 || qs < 0 || qs >= T) return;
  const int nq = min(WA_Q, T - qs);
  const int klo = max(0, qs - left), khi = min(T, qs + nq + right);  // keys [klo, khi) of the block
  const int kt0 = klo & ~(WA_KT - 1);
  const int ntiles = (khi - kt0 + WA_KT - 1) / WA_KT;

  // this wave's rows and the keys they may see
  const int r_first = qs + 32 * wid;
  const bool active = r_first < qs + nq;
  const int r_last = min(r_first + 31, qs + nq - 1);
  const int wlo = max(0, r_first - left), whi = min(T - 1, r_last + right);

  const bf16_t *qbase = qkv + h * WA_D;
  const bf16_t *kbase_p = qkv + (H + h) * WA_D;
  const bf16_t *vbase_p = qkv + (2 * H + h) * WA_D;

  int qpos[2];
  bf16x8 bq[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int r = r_first + 16 * qb + col;
    r = r < T ? r : T - 1;
    qpos[qb] = r;
    const bf16_t *src = qbase + (row0 + r) * ld + g * 8;
    const u32x4 lo = *reinterpret_cast<const u32x4 *>(src);
    const u32x4 hi = *reinterpret_cast<const u32x4 *>(src + 32);
    if (!ROT) {  // q already rotated (by the Wqkv product's epilogue)
      bq[qb][0] = __builtin_bit_cast(bf16x8, lo);
      bq[qb][1] = __builtin_bit_cast(bf16x8, hi);
      continue;
    }
    const f32x4 c0 = *reinterpret_cast<const f32x4 *>(cos_t + r * 32 + g * 8);
    const f32x4 c1 = *reinterpret_cast<const f32x4 *>(cos_t + r * 32 + g * 8 + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4 *>(sin_t + r * 32 + g * 8);
    const f32x4 s1 = *reinterpret_cast<const f32x4 *>(sin_t + r * 32 + g * 8 + 4);
    uint32_t y1w[4], y2w[4];
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) {
      float y1[2], y2[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int e = 2 * wv + hf;
        const float x1 = hf ? hi_bf(lo[wv]) : lo_bf(lo[wv]);
        const float x2 = hf ? hi_bf(hi[wv]) : lo_bf(hi[wv]);
        const float cs = e < 4 ? c0[e] : c1[e - 4];
        const float sn = e < 4 ? s0[e] : s1[e - 4];
        y1[hf] = x1 * cs - x2 * sn;
        y2[hf] = x1 * sn + x2 * cs;
      }
      y1w[wv] = pack_bf(y1[0], y1[1]);
      y2w[wv] = pack_bf(y2[0], y2[1]);
    }
    bq[qb][0] = __builtin_bit_cast(bf16x8, u32x4{y1w[0], y1w[1], y1w[2], y1w[3]});
    bq[qb][1] = __builtin_bit_cast(bf16x8, u32x4{y2w[0], y2w[1], y2w[2], y2w[3]});
  }

  f32x4 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f}, alpha_q[2];

  // tile staging: thread -> key row lrow, d chunks lc and lc + 4 (a rotation pair) of K and of V
  const int lrow = tid >> 2, lc = tid & 3;
  u32x4 rk0, rk1, rv0, rv1;
  f32x4 tc0, tc1, ts0, ts1;
  auto load_tile = [&](int t) {
    int key = kt0 + t * WA_KT + lrow;
    key = key < T ? key : T - 1;
    const int64_t off = (row0 + key) * ld + lc * 8;
    rk0 = *reinterpret_cast<const u32x4 *>(kbase_p + off);
    rk1 = *reinterpret_cast<const u32x4 *>(kbase_p + off + 32);
    rv0 = *reinterpret_cast<const u32x4 *>(vbase_p + off);
    rv1 = *reinterpret_cast<const u32x4 *>(vbase_p + off + 32);
    if (!ROT) return;
    tc0 = *reinterpret_cast<const f32x4 *>(cos_t + key * 32 + lc * 8);
    tc1 = *reinterpret_cast<const f32x4 *>(cos_t + key * 32 + lc * 8 + 4);
    ts0 = *reinterpret_cast<const f32x4 *>(sin_t + key * 32 + lc * 8);
    ts1 = *reinterpret_cast<const f32x4 *>(sin_t + key * 32 + lc * 8 + 4);
  };
  auto store_tile = [&](int buf) {
    u32x4 k1 = rk0, k2 = rk1;
#pragma unroll
    for (int wv = 0; wv < 4 && ROT; ++wv) {
      float y1[2], y2[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int e = 2 * wv + hf;
        const float x1 = hf ? hi_bf(rk0[wv]) : lo_bf(rk0[wv]);
        const float x2 = hf ? hi_bf(rk1[wv]) : lo_bf(rk1[wv]);
        const float cs = e < 4 ? tc0[e] : tc1[e - 4];
        const float sn = e < 4 ? ts0[e] : ts1[e - 4];
        y1[hf] = x1 * cs - x2 * sn;
        y2[hf] = x1 * sn + x2 * cs;
      }
      k1[wv] = pack_bf(y1[0], y1[1]);
      k2[wv] = pack_bf(y2[0], y2[1]);
    }
    *reinterpret_cast<u32x4 *>(&Ks[buf][lrow * WA_PITCH + lc * 8]) = k1;
    *reinterpret_cast<u32x4 *>(&Ks[buf][lrow * WA_PITCH + lc * 8 + 32]) = k2;
    // V transposed, so the O^T = V^T P^T operand is two 8-byte reads per lane
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) {
      Vt[buf][(lc * 8 + 2 * wv) * WA_VTP + lrow] = static_cast<bf16_t>(rv0[wv] & 0xffffu);
      Vt[buf][(lc * 8 + 2 * wv + 1) * WA_VTP + lrow] = static_cast<bf16_t>(rv0[wv] >> 16);
      Vt[buf][(32 + lc * 8 + 2 * wv) * WA_VTP + lrow] = static_cast<bf16_t>(rv1[wv] & 0xffffu);
      Vt[buf][(32 + lc * 8 + 2 * wv + 1) * WA_VTP + lrow] = static_cast<bf16_t>(rv1[wv] >> 16);
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kb0 = kt0 + t * WA_KT + 32 * ks;
      if (!active || kb0 > whi || kb0 + 31 < wlo) continue;  // wave-uniform: no row of this wave sees these keys
      const bf16_t *kt = &Ks[buf][32 * ks * WA_PITCH];
      const bf16_t *vt = &Vt[buf][32 * ks];
      f32x4 st[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        bf16x8 ka[2];
#pragma unroll
        for (int dc = 0; dc < 2; ++dc)
          ka[dc] = *reinterpret_cast<const bf16x8 *>(&kt[(16 * kb + col) * WA_PITCH + 32 * dc + g * 8]);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          st[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int dc = 0; dc < 2; ++dc)
            st[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[dc], bq[qb][dc], st[kb][qb], 0, 0, 0);
        }
      }
      // no mask needed when every key of the half is inside every row's window and inside the chunk
      const bool need_mask = kb0 < r_last - left || kb0 + 31 > r_first + right || kb0 + 31 >= T;
      bf16x8 pf[2];
      bool grew = false;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        // branch-free softmax step: the window test uses bitwise ands under one wave-uniform branch (a
        // short-circuit test per score compiled to a divergent branch per score)
        float sv[8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[kb * 4 + i] = st[kb][qb][i] * scale_log2;
        if (need_mask) {
          const int lo_k = qpos[qb] - left, hi_k = min(qpos[qb] + right, T - 1);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = kb0 + 16 * kb + 4 * g + i;
              sv[kb * 4 + i] = ((key >= lo_k) & (key <= hi_k)) ? sv[kb * 4 + i] : -INFINITY;
            }
        }
        float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[qb], mx);
        // a row may see no key of its first halves (window start): keep exp2 arguments finite
        const float m_sub = m_new == -INFINITY ? 0.f : m_new;
        // exponents are <= 0: the bare v_exp_f32 (no range reduction needed)
        float e[8], ps = 0.f;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          e[jj] = __builtin_amdgcn_exp2f(sv[jj] - m_sub);
          ps += e[jj];
        }
        pf[qb] = __builtin_bit_cast(bf16x8, u32x4{pack_bf(e[0], e[1]), pack_bf(e[2], e[3]), pack_bf(e[4], e[5]),
                                                   pack_bf(e[6], e[7])});
        // the running max moved: rescale this row's sum (and, below, its output); else alpha is exactly 1
        const bool moved = m_new != m_run[qb];
        const float alpha = moved ? __builtin_amdgcn_exp2f(m_run[qb] - m_sub) : 1.0f;
        alpha_q[qb] = alpha;
        grew |= moved;
        l_run[qb] = l_run[qb] * alpha + ps;
        m_run[qb] = m_new;
      }
      // rescale the outputs only when some row of the wave saw a new maximum (a multiply by 1 otherwise)
      if (__builtin_amdgcn_ballot_w64(grew) != 0) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) acc[dt][qb] *= alpha_q[qb];
      }
      // O^T += V^T P^T (key order {4g..4g+3, 16+4g..16+4g+3} in both operands)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const bf16_t *vr = vt + (16 * dt + col) * WA_VTP;
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(vr + 4 * g);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(vr + 16 + 4 * g);
        const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) acc[dt][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[qb], acc[dt][qb], 0, 0, 0);
      }
    }
    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = l_run[qb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int r = r_first + 16 * qb + col;
    if (r > r_last) continue;
    const float inv = 1.0f / l;
    bf16_t *dst = out + (row0 + r) * ldo + h * WA_D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      u32x2 pk;
      pk[0] = pack_bf(acc[dt][qb][0] * inv, acc[dt][qb][1] * inv);
      pk[1] = pack_bf(acc[dt][qb][2] * inv, acc[dt][qb][3] * inv);
      *reinterpret_cast<u32x2 *>(dst + 16 * dt) = pk;
    }
  }
}

// ---- DeepNorm residual + RMSNorm: x = bf16(rmsnorm(bf16(bf16(y + bias) + bf16(alpha x))) * w) -----------
// y fp32 [n, 512] (a product before rounding), x bf16 [n, 512] updated in place; one wavefront per row.
constexpr int DN_D = 512;

__global__ __launch_bounds__(256) void deepnorm_kernel(const float *__restrict__ y, const float *__restrict__ bias,
                                                       bf16_t *__restrict__ x, float alpha,
                                                       const float *__restrict__ w, float eps, int64_t n) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const int c0 = lane * 8;
  const f32x4 y0 = *reinterpret_cast<const f32x4 *>(y + row * DN_D + c0);
  const f32x4 y1 = *reinterpret_cast<const f32x4 *>(y + row * DN_D + c0 + 4);
  const u32x4 xw = *reinterpret_cast<const u32x4 *>(x + row * DN_D + c0);
  f32x4 b0 = {0.f, 0.f, 0.f, 0.f}, b1 = {0.f, 0.f, 0.f, 0.f};
  if (bias != nullptr) {
    b0 = *reinterpret_cast<const f32x4 *>(bias + c0);
    b1 = *reinterpret_cast<const f32x4 *>(bias + c0 + 4);
  }
  float r[8];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float yv = e < 4 ? y0[e] : y1[e - 4];
    const float bv = e < 4 ? b0[e] : b1[e - 4];
    const float xv = (e & 1) ? hi_bf(xw[e >> 1]) : lo_bf(xw[e >> 1]);
    r[e] = round_bf(round_bf(yv + bv) + round_bf(alpha * xv));
    ss += r[e] * r[e];
  }
  ss = wave_sum(ss);
  const float rn = rsqrtf(ss * (1.0f / DN_D) + eps);
  const f32x4 w0 = *reinterpret_cast<const f32x4 *>(w + c0);
  const f32x4 w1 = *reinterpret_cast<const f32x4 *>(w + c0 + 4);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = r[e] * rn * (e < 4 ? w0[e] : w1[e - 4]);
  *reinterpret_cast<u32x4 *>(x + row * DN_D + c0) =
      u32x4{pack_bf(o[0], o[1]), pack_bf(o[2], o[3]), pack_bf(o[4], o[5]), pack_bf(o[6], o[7])};
}

int gemm_big(const bf16_t *x, const bf16_t *w, void *y, int64_t M, int N, int K, bool swiglu, bool out_f32,
             hipStream_t s);

}  // namespace vk

using namespace vk;

extern "C" int vk_encoder_conv_first(const float *signal, const int64_t *sig_off, const int32_t *start,
                                     const int32_t *hint, const int32_t *len, int32_t n_chunks, int64_t rows,
                                     const float *w, const float *b, int32_t C, int32_t winlen, int32_t stride,
                                     int32_t pad, void *out, void *stream) {
  VK_CHECK_ARG(signal && sig_off && start && hint && len && w && b && out, "encoder_conv_first: null pointer");
  VK_CHECK_ARG(n_chunks > 0 && rows >= 0 && C > 0 && C % 8 == 0 && C <= 512 && winlen > 0 &&
                   winlen <= CF_MAX_WIN && C * winlen <= CF_MAX_W && stride > 0 && pad >= 0,
               "encoder_conv_first: bad sizes (C %d winlen %d stride %d pad %d)", C, winlen, stride, pad);
  VK_CHECK_ARG(vk_aligned16(out), "encoder_conv_first: out must be 16-byte aligned");
  if (rows == 0) return VK_OK;
  const int64_t threads = rows * (C / 8);
  conv_first_kernel<<<static_cast<unsigned>((threads + 255) / 256), 256, 0, VK_STREAM(stream)>>>(
      signal, sig_off, start, hint, len, n_chunks, rows, w, b, C, winlen, stride, pad, static_cast<bf16_t *>(out));
  return launch_status("encoder_conv_first");
}

extern "C" int vk_encoder_conv(const void *a, int64_t lda, const void *w, int32_t K, int32_t N, const float *bias,
                               const int32_t *start, const int32_t *hint, const int32_t *len, const int32_t *dst0,
                               int32_t n_chunks, int64_t rows, int32_t compact, void *out, int64_t ldo, void *stream) {
  VK_CHECK_ARG(a && w && bias && start && hint && len && out && (!compact || dst0), "encoder_conv: null pointer");
  VK_CHECK_ARG(n_chunks > 0 && rows >= 0 && K > 0 && K % CG_BK == 0 && N > 0 && N % CG_BN == 0 && lda % 8 == 0 &&
                   ldo >= N && ldo % 4 == 0,
               "encoder_conv: need K %% 32 == 0, N %% 64 == 0, lda %% 8 == 0 (K %d N %d lda %lld)", K, N,
               static_cast<long long>(lda));
  VK_CHECK_ARG(vk_aligned16(a) && vk_aligned16(w) && vk_aligned16(out), "encoder_conv: pointers must be 16-byte aligned");
  if (rows == 0) return VK_OK;
  const dim3 grid(static_cast<unsigned>((rows + CG_BM - 1) / CG_BM), static_cast<unsigned>(N / CG_BN));
  conv_gemm_kernel<<<grid, 256, 0, VK_STREAM(stream)>>>(static_cast<const bf16_t *>(a), lda,
                                                         static_cast<const bf16_t *>(w), K, N, bias, start, hint, len, dst0,
                                                         n_chunks, rows, compact, static_cast<bf16_t *>(out), ldo);
  return launch_status("encoder_conv");
}

extern "C" int vk_window_attention(const void *qkv, int64_t ld, const int32_t *cu, const int32_t *plan,
                                   int32_t n_blocks, int32_t n_chunks, int32_t max_len, int32_t H, int32_t D,
                                   const float *cos_t, const float *sin_t, int32_t table_len, int32_t left,
                                   int32_t right, void *out, int64_t ldo, void *stream) {
  VK_CHECK_ARG(qkv && cu && plan && out && (cos_t == nullptr) == (sin_t == nullptr), "window_attention: null pointer");
  if (D != WA_D) return fail(VK_ERR_UNSUPPORTED, "window_attention: built for head_dim 64 (got %d)", D);
  VK_CHECK_ARG(H > 0 && n_blocks >= 0 && n_chunks > 0 && left >= 0 && right >= 0 && ld >= 3 * H * WA_D &&
                   ld % 8 == 0 && ldo >= H * WA_D && ldo % 4 == 0,
               "window_attention: bad sizes");
  VK_CHECK_ARG(cos_t == nullptr || max_len <= table_len, "window_attention: chunk of %d frames beyond the rotary table (%d)",
               max_len, table_len);
  VK_CHECK_ARG(vk_aligned16(qkv) && vk_aligned16(out) && vk_aligned16(cos_t) && vk_aligned16(sin_t),
               "window_attention: pointers must be 16-byte aligned");
  if (n_blocks == 0) return VK_OK;
  const int64_t total = static_cast<int64_t>(n_blocks) * H;
  VK_CHECK_ARG(total < (int64_t(1) << 31), "window_attention: too many blocks");
  const float scale_log2 = static_cast<float>(1.0 / sqrt(static_cast<double>(WA_D)) * 1.4426950408889634);
  auto kern = cos_t != nullptr ? window_attn_kernel<true> : window_attn_kernel<false>;
  kern<<<static_cast<unsigned>(total), 256, 0, VK_STREAM(stream)>>>(static_cast<const bf16_t *>(qkv), ld, cu, plan,
                                                                     n_blocks, n_chunks, H, cos_t, sin_t, left, right,
                                                                     scale_log2, static_cast<bf16_t *>(out), ldo);
  return launch_status("window_attention");
}

extern "C" int vk_deepnorm_rmsnorm(const float *y, const float *bias, void *x, float alpha, const float *w, float eps,
                                   int64_t n, int32_t d, void *stream) {
  VK_CHECK_ARG(y && x && w, "deepnorm_rmsnorm: null pointer");
  if (d != DN_D) return fail(VK_ERR_UNSUPPORTED, "deepnorm_rmsnorm: built for d_model 512 (got %d)", d);
  VK_CHECK_ARG(n >= 0, "deepnorm_rmsnorm: bad sizes");
  VK_CHECK_ARG(vk_aligned16(y) && vk_aligned16(x) && vk_aligned16(w) && (bias == nullptr || vk_aligned16(bias)),
               "deepnorm_rmsnorm: pointers must be 16-byte aligned");
  if (n == 0) return VK_OK;
  deepnorm_kernel<<<static_cast<unsigned>((n + 3) / 4), 256, 0, VK_STREAM(stream)>>>(y, bias, static_cast<bf16_t *>(x),
                                                                                     alpha, w, eps, n);
  return launch_status("deepnorm_rmsnorm");
}

extern "C" int vk_gemm_rows(const void *x, const void *w, void *y, int64_t M, int32_t N, int32_t K, int32_t epilogue,
                            void *stream) {
  VK_CHECK_ARG(x && w && y, "gemm_rows: null pointer");
  VK_CHECK_ARG(M >= 0 && N > 0 && N % 8 == 0 && K > 0 && K % 64 == 0, "gemm_rows: need N %% 8 == 0, K %% 64 == 0");
  VK_CHECK_ARG(epilogue >= 0 && epilogue <= 2, "gemm_rows: epilogue 0 (bf16), 1 (fp32) or 2 (SwiGLU)");
  VK_CHECK_ARG(vk_aligned16(x) && vk_aligned16(w) && vk_aligned16(y), "gemm_rows: pointers must be 16-byte aligned");
  VK_CHECK_ARG(M < (int64_t(1) << 31) / 256 * 256, "gemm_rows: M too large");
  if (M == 0) return VK_OK;
  const int rc = gemm_big(static_cast<const bf16_t *>(x), static_cast<const bf16_t *>(w), y, M, N, K, epilogue == 2,
                          epilogue == 1, VK_STREAM(stream));
  if (rc != VK_OK) return rc;
  return launch_status("gemm_rows");
}
