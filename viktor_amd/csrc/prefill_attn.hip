// Variable-length GQA attention of packed queries against per-sequence key ranges, bf16 MFMA with
// fp32 online softmax (the semantics of flash_attn_varlen_func as called at
// viktor/fast_decoder.py:68-73, and of flash_attn_func(causal=True) at viktor/decoder.py:82-87).
//
// MI355X design:
//   * Workgroup = one 64-query block of one sequence x one KV head, 8 wavefronts: the 4 query heads of
//     that KV head x 2 halves of 32 query rows. Every K/V tile staged in LDS serves 4 heads x 64 rows.
//   * Keys advance in 64-row tiles, double buffered in LDS (the next tile's global loads are in flight
//     during the MFMAs on the current one; 16-byte pad per row). Within a tile a wave works in two
//     32-key halves; halves that lie entirely above the causal diagonal of the wave's rows are skipped.
//   * Transposed products as in the decode kernel: S^T = K Q^T (A = key rows from LDS, B = Q^T held in
//     registers for the whole loop) leaves each lane the scores of one query row; O^T = V^T P^T consumes
//     those probabilities in place and the online-softmax rescale stays lane-local. V is staged row-major like
//     K and the V^T operand is two LDS transpose reads (ds_read_b64_tr_b16) per lane.
//   * Per-wave state is 32 query rows (Q^T 16, O^T 32, scores 16 VGPRs) so the kernel fits 4 waves per
//     SIMD: two workgroups per CU.
//   * Keys of sequence i live at base + k_off[i] + j * stride_tok (+ kv head * 64): the same kernel
//     reads packed k/v rows or a KV-cache layer directly.
//   * The host orders the query blocks longest-first (causal blocks near the end of a sequence do the
//     most work) so the tail of the grid is short blocks.
//   * PREFIXED: a sequence's first p_lens[i] keys come from a second buffer (kp / vp + p_off[i] + j * p_stride),
//     the rest from k / v as above (key j at k_off[i] + (j - p_lens[i]) * stride_tok): the key order of one
//     window [prefix | own rows] whose prefix rows are shared with other sequences (a GSPO group's samples).
//     The choice is made per loaded row, so a tile may straddle the two.
#include <math.h>

#include "common.h"

namespace vk {

constexpr int PA_H = 8, PA_HKV = 2, PA_D = 64;
constexpr int PA_Q = 64;      // query rows per workgroup (plan granularity)
constexpr int PA_WAVES = 8;   // 4 query heads x 2 halves of 32 rows
constexpr int PA_KT = 64;     // keys per LDS tile
constexpr int PA_PITCH = 72;  // 64 + 8 bf16
constexpr float PA_SLACK = 8.0f;  // log2 units a row's score may pass its reference max before it moves

struct PaPrefix {
  const bf16_t *kp, *vp;       // prefix keys / values
  const int64_t *p_off;        // per sequence: element offset of its prefix row 0
  const int32_t *p_lens;       // per sequence: keys taken from the prefix buffer
  int64_t p_stride;            // elements between prefix rows
};

template <bool PREFIXED>
__global__ __launch_bounds__(PA_WAVES * 64) void varlen_attn_kernel(
    const bf16_t *__restrict__ q, const bf16_t *__restrict__ k, const bf16_t *__restrict__ v,
    const int32_t *__restrict__ cu_q, const int64_t *__restrict__ k_off, const int32_t *__restrict__ k_lens,
    const int32_t *__restrict__ plan, int n_seq, int64_t stride_tok, bf16_t *__restrict__ out, int causal,
    float scale_log2, float *__restrict__ lse, const PaPrefix pre) {
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][PA_KT * PA_PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[2][PA_KT * PA_PITCH];  // V rows, as K

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int col = lane & 15, g = lane >> 4;
  const int hk = blockIdx.y;
  const int hq = hk * (PA_H / PA_HKV) + (wid & 3);
  const int half = wid >> 2;
  const int seq = plan[2 * blockIdx.x];
  const int qs = plan[2 * blockIdx.x + 1];
  // the sequence's metadata is loaded before the checks below (index clamped into 0 .. n_seq - 1; n_seq > 0 is
  // checked on the host), so these loads go out together instead of one round trip per check
  const int seq_c = seq < 0 ? 0 : (seq >= n_seq ? n_seq - 1 : seq);
  const int64_t q0 = cu_q[seq_c];
  const int q_end = cu_q[seq_c + 1];
  const int klen = k_lens[seq_c];
  const int64_t koff = k_off[seq_c];
  const int plen = PREFIXED ? pre.p_lens[seq_c] : 0;
  const int64_t poff = PREFIXED ? pre.p_off[seq_c] : 0;
  asm volatile("" ::"s"(q0), "s"(q_end), "s"(klen), "s"(koff));  // (kept ahead of the checks: the compiler would sink them)
  if (PREFIXED) asm volatile("" ::"s"(plen), "s"(poff));
  if (seq < 0 || seq >= n_seq || qs < 0) return;
  const int q_len = q_end - static_cast<int>(q0);
  if (q_len <= 0 || klen <= 0 || qs >= q_len) return;
  const int qshift = klen - q_len;  // query r sits at key position qshift + r
  const int nq = min(PA_Q, q_len - qs);
  const int kend = causal ? min(klen, qshift + qs + nq) : klen;
  if (kend <= 0) return;
  const int ntiles = (kend + PA_KT - 1) / PA_KT;

  // this wave's 32 query rows: two blocks of 16 (row = lane % 16 within a block)
  const int r_first = qs + 32 * half;
  int qpos[2];
  bf16x8 bq[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int r = r_first + 16 * qb + col;
    r = r < q_len ? r : q_len - 1;
    qpos[qb] = qshift + r;
    const bf16_t *src = q + ((q0 + r) * PA_H + hq) * PA_D + g * 8;
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) bq[qb][dc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(src + 32 * dc));
  }
  // highest key any row of this wave may see (rows past q_len are clamped copies of the last row)
  const int wave_kmax = causal ? qshift + min(r_first + 31, q_len - 1) : klen - 1;

  f32x4 acc[4][2];  // O^T tiles [d tile][query block]
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};  // raw-score reference max, row sum
  const float slack_raw = PA_SLACK / scale_log2;

  // cooperative tile load: 512 threads -> (key row 0..63, 16-byte chunk 0..7) of K and of V
  const int lrow = tid >> 3, lchunk = tid & 7;
  u32x4 rk, rv;
  auto load_tile = [&](int t) {
    int key = t * PA_KT + lrow;
    key = key < klen ? key : klen - 1;
    const bf16_t *kb = k, *vb = v;
    int64_t off;
    if (PREFIXED && key < plen) {
      kb = pre.kp;
      vb = pre.vp;
      off = poff + static_cast<int64_t>(key) * pre.p_stride;
    } else {
      off = koff + static_cast<int64_t>(key - plen) * stride_tok;
    }
    off += hk * PA_D + lchunk * 8;
    rk = *reinterpret_cast<const u32x4 *>(kb + off);
    rv = *reinterpret_cast<const u32x4 *>(vb + off);
  };
  auto store_tile = [&](int buf) {
    *reinterpret_cast<u32x4 *>(&Ks[buf][lrow * PA_PITCH + lchunk * 8]) = rk;
    *reinterpret_cast<u32x4 *>(&Vs[buf][lrow * PA_PITCH + lchunk * 8]) = rv;
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kbase = t * PA_KT + 32 * ks;
      if (kbase > wave_kmax) continue;  // wave-uniform: every key of this half is masked for every row
      const bf16_t *kt = &Ks[buf][32 * ks * PA_PITCH];
      const bf16_t *vt = &Vs[buf][32 * ks * PA_PITCH];
      // S^T[key][query] for two 16-key blocks x two 16-query blocks
      f32x4 st[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        bf16x8 ka[2];
#pragma unroll
        for (int dc = 0; dc < 2; ++dc)
          ka[dc] = *reinterpret_cast<const bf16x8 *>(&kt[(16 * kb + col) * PA_PITCH + 32 * dc + g * 8]);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          st[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int dc = 0; dc < 2; ++dc)
            st[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[dc], bq[qb][dc], st[kb][qb], 0, 0, 0);
        }
      }
      const bool need_mask = kbase + 31 >= klen || (causal && kbase + 31 > qshift + r_first);
      // softmax step on the raw scores (the scale enters through the exponent's fma, and max commutes with a
      // positive scale); the mask is a compare per score under one wave-uniform branch (a short-circuit test
      // per score compiles to a divergent branch per score)
      bf16x8 pf[2];
      float m_old[2], ps_q[2];
      bool moved_q[2], grew = false;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float sv[8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[kb * 4 + i] = st[kb][qb][i];
        if (need_mask) {
          // last key this row sees, relative to this lane's first key (key kbase + 4 g): one subtraction,
          // then compares against constants
          const int lim = (causal ? min(qpos[qb], klen - 1) : klen - 1) - kbase - 4 * g;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[kb * 4 + i] = 16 * kb + i <= lim ? sv[kb * 4 + i] : -INFINITY;
        }
        // The row's reference max moves only when a score passes it by more than PA_SLACK in log2 units of the
        // scaled scores: the probabilities are then exp2(s c - m c) <= 2^PA_SLACK (bf16 and the fp32 sums carry
        // them with the same relative precision as values <= 1), and the rescale of the row's sum and output
        // (a multiply per accumulator) is rare after the first tiles. m_run = -inf before the first key: any
        // finite score moves it. Tile 0 holds key 0, visible to every query, so m_run is finite after it.
        // The row's max over its 4 lanes is needed only when some lane's own max passes the slack, so the lane
        // swaps run under a wave-uniform test that is rarely true after the first tiles.
        const float mx_lane = vmax3(vmax3(sv[0], sv[1], sv[2]), vmax3(sv[3], sv[4], sv[5]), vmax3(sv[6], sv[7], sv[7]));
        bool moved = false;
        float m_ref = m_run[qb];
        if (__builtin_amdgcn_ballot_w64(mx_lane > m_run[qb] + slack_raw) != 0) {
          const float mx = max_lane_groups(mx_lane);
          moved = mx > m_run[qb] + slack_raw;
          m_ref = moved ? mx : m_run[qb];
        }
        const float nmc = -m_ref * scale_log2;
        float e[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) e[jj] = __builtin_amdgcn_exp2f(fmaf(sv[jj], scale_log2, nmc));
        float ps = e[0];
#pragma unroll
        for (int jj = 1; jj < 8; ++jj) ps += e[jj];
        pf[qb] = __builtin_bit_cast(bf16x8, u32x4{pack_bf(e[0], e[1]), pack_bf(e[2], e[3]), pack_bf(e[4], e[5]),
                                                   pack_bf(e[6], e[7])});
        m_old[qb] = m_run[qb];
        moved_q[qb] = moved;
        ps_q[qb] = ps;
        grew |= moved;
        m_run[qb] = m_ref;
      }
      // the rescale (its two exponentials included) only when some row of the wave moved its reference max
      if (__builtin_amdgcn_ballot_w64(grew) != 0) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float alpha = moved_q[qb] ? __builtin_amdgcn_exp2f((m_old[qb] - m_run[qb]) * scale_log2) : 1.0f;
          l_run[qb] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) acc[dt][qb] *= alpha;
        }
      }
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) l_run[qb] += ps_q[qb];
      // O^T += V^T P^T (key order {4g..4g+3, 16+4g..16+4g+3} in both operands). The V^T operand comes from
      // the row-major V tile through gfx950's transpose read ds_read_b64_tr_b16: in each 16-lane group, source
      // lane s reads 4 consecutive d of key row R0 + s / 4 and output lane j receives d = 16 dt + j at keys
      // R0 .. R0 + 3; two reads (R0 = 4 g and 16 + 4 g) give the lane's 8 keys.
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const bf16x8 va = lds_tr_frag<PA_PITCH>(vt, 0, 16 * dt, lane);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) acc[dt][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[qb], acc[dt][qb], 0, 0, 0);
      }
    }
    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = l_run[qb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int r = r_first + 16 * qb + col;
    if (r >= q_len || r >= qs + nq) continue;
    const float inv = 1.0f / l;
    // the row's log-sum-exp in log2 units of the scaled scores (m c + log2 l), for the backward pass
    if (lse != nullptr && g == 0) lse[(q0 + r) * PA_H + hq] = m_run[qb] * scale_log2 + log2f(l);
    bf16_t *dst = out + ((q0 + r) * PA_H + hq) * PA_D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      u32x2 pk;
      pk[0] = pack_bf(acc[dt][qb][0] * inv, acc[dt][qb][1] * inv);
      pk[1] = pack_bf(acc[dt][qb][2] * inv, acc[dt][qb][3] * inv);
      *reinterpret_cast<u32x2 *>(dst + 16 * dt) = pk;
    }
  }
}

}  // namespace vk

using namespace vk;

static int varlen_launch(const void *q, const void *k, const void *v, const int32_t *cu_q, const int64_t *k_off,
                         const int32_t *k_lens, const int32_t *plan, int32_t n_blocks, int32_t n_seq, int64_t stride_tok,
                         void *out, int32_t causal, int32_t H, int32_t HKV, int32_t D, float *lse, const PaPrefix *pre,
                         void *stream) {
  VK_CHECK_ARG(q && k && v && cu_q && k_off && k_lens && out, "varlen_attention: null pointer");
  if (H != PA_H || HKV != PA_HKV || D != PA_D)
    return fail(VK_ERR_UNSUPPORTED, "varlen_attention: built for H=8 HKV=2 D=64 (got %d/%d/%d)", H, HKV, D);
  VK_CHECK_ARG(n_blocks >= 0 && n_seq >= 0 && stride_tok >= PA_HKV * PA_D && stride_tok % 8 == 0,
               "varlen_attention: bad sizes");
  VK_CHECK_ARG(n_blocks == 0 || (plan != nullptr && n_seq > 0), "varlen_attention: missing plan or sequences");
  VK_CHECK_ARG(vk_aligned16(q) && vk_aligned16(k) && vk_aligned16(v) && vk_aligned16(out),
               "varlen_attention: pointers must be 16-byte aligned");
  if (pre != nullptr) {
    VK_CHECK_ARG(pre->kp && pre->vp && pre->p_off && pre->p_lens, "varlen_attention_prefixed: null pointer");
    VK_CHECK_ARG(pre->p_stride >= PA_HKV * PA_D && pre->p_stride % 8 == 0, "varlen_attention_prefixed: bad prefix stride");
    VK_CHECK_ARG(vk_aligned16(pre->kp) && vk_aligned16(pre->vp), "varlen_attention_prefixed: prefix pointers must be 16-byte aligned");
  }
  if (n_blocks == 0) return VK_OK;
  const float scale_log2 = static_cast<float>(1.0 / sqrt(static_cast<double>(PA_D)) * 1.4426950408889634);
  const dim3 grid(static_cast<unsigned>(n_blocks), PA_HKV);
  const auto qb = static_cast<const bf16_t *>(q), kb = static_cast<const bf16_t *>(k), vb = static_cast<const bf16_t *>(v);
  const auto ob = static_cast<bf16_t *>(out);
  if (pre != nullptr)
    varlen_attn_kernel<true><<<grid, PA_WAVES * 64, 0, VK_STREAM(stream)>>>(
        qb, kb, vb, cu_q, k_off, k_lens, plan, n_seq, stride_tok, ob, causal, scale_log2, lse, *pre);
  else
    varlen_attn_kernel<false><<<grid, PA_WAVES * 64, 0, VK_STREAM(stream)>>>(
        qb, kb, vb, cu_q, k_off, k_lens, plan, n_seq, stride_tok, ob, causal, scale_log2, lse, PaPrefix{});
  return launch_status("varlen_attention");
}

extern "C" int vk_varlen_attention(const void *q, const void *k, const void *v, const int32_t *cu_q,
                                   const int64_t *k_off, const int32_t *k_lens, const int32_t *plan, int32_t n_blocks,
                                   int32_t n_seq, int64_t stride_tok, void *out, int32_t causal, int32_t H,
                                   int32_t HKV, int32_t D, float *lse, void *stream) {
  return varlen_launch(q, k, v, cu_q, k_off, k_lens, plan, n_blocks, n_seq, stride_tok, out, causal, H, HKV, D, lse,
                       nullptr, stream);
}

extern "C" int vk_varlen_attention_prefixed(const void *q, const void *k, const void *v, const int32_t *cu_q,
                                            const int64_t *k_off, const int32_t *k_lens, const int32_t *plan,
                                            int32_t n_blocks, int32_t n_seq, int64_t stride_tok, const void *k_prefix,
                                            const void *v_prefix, const int64_t *p_off, const int32_t *p_lens,
                                            int64_t p_stride, void *out, int32_t causal, int32_t H, int32_t HKV,
                                            int32_t D, float *lse, void *stream) {
  const PaPrefix pre{static_cast<const bf16_t *>(k_prefix), static_cast<const bf16_t *>(v_prefix), p_off, p_lens,
                     p_stride};
  return varlen_launch(q, k, v, cu_q, k_off, k_lens, plan, n_blocks, n_seq, stride_tok, out, causal, H, HKV, D, lse,
                       &pre, stream);
}
