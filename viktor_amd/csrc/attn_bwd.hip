// Backward of causal GQA self-attention over packed sequences (the training-mode attention of the decoder:
// flash_attn_func(causal=True) under autocast at viktor/decoder.py:82-87, whose backward the GSPO update
// runs through at scripts/gspo.py:477).
//
// Per sequence i (rows cu[i] .. cu[i+1]-1 of the packed q [N, 8, 64], k / v [N, 2, 64] at stride_tok),
// query head h uses KV head h / 4, query r sees keys j <= r, S = q k^T / sqrt(64), P = softmax(S),
// o = P v. Given dO, with D_r = sum_d dO_rd o_rd (row dot kernel):
//   dV_j = sum_r P_rj dO_r          dP_rj = dO_r . v_j          dS_rj = P_rj (dP_rj - D_r)
//   dQ_r = sum_j dS_rj k_j / 8      dK_j = sum_r dS_rj q_r / 8  (summed over the 4 query heads of a KV head)
// P is recomputed from the forward's per-row log-sum-exp (log2 units of the scaled scores).
//
// MI355X design: the transposed MFMA products of the forward kernels, so the probabilities computed in one
// product's accumulator layout are consumed in place as the next product's operand:
//   * dQ kernel = the forward's shape: a workgroup per 64-query block x KV head, 8 wavefronts (4 query
//     heads x 2 halves of 32 rows), K / V tiles of 64 keys double buffered in LDS. Per key half:
//     S^T = K Q^T, dP^T = V dO^T (A = key rows from LDS, B = Q^T / dO^T held in registers), dS^T in the
//     accumulator layout, dQ^T += K^T dS^T (A = K^T by LDS transpose reads of the row-major K tile).
//   * dK/dV kernel: a workgroup per 128-key block x KV head, 4 wavefronts of 32 keys (two 16-key blocks;
//     K^T / V^T fragments in registers), looping over the 32-query tiles at or below the diagonal, Q / dO /
//     lse / D of the 4 query heads staged in LDS (the next tile's loads in flight during the current one):
//     S = Q K^T, dP = dO V^T (A = query rows), then dV^T += dO^T P and dK^T += Q^T dS (A = dO^T / Q^T by
//     LDS transpose reads of the row-major tiles) with P / dS consumed in their accumulator layout; the 4
//     heads accumulate in place. Each operand fragment read from LDS feeds both key blocks of the wave, so
//     the LDS reads per MFMA are half those of 16-key waves (the kernel was bound by them). 128 keys per
//     staged tile halve the re-reads of Q / dO against 64.
// Gradients are written in fp32 (the consumers -- QK-norm / RoPE backward, the qkv weight gradient -- work
// in fp32 and round once).
#include <math.h>

#include "common.h"

namespace vk {

constexpr int AB_H = 8, AB_HKV = 2, AB_D = 64;
constexpr int AB_PITCH = 72;  // 64 + 8 bf16 per LDS row
constexpr int AB_KW = 4;      // wavefronts of a dK/dV workgroup (32 keys each: 128 keys per staged query tile)
constexpr int AB_KB = 32 * AB_KW;

typedef short ab_s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ab_s4 ab_lds_s4;

// The MFMA operand "column 16 dt + lane % 16 of a row-major LDS tile (AB_PITCH elements per row) at rows
// r0 + 4 g .. + 3 and r0 + 16 + 4 g .. + 3" (g = lane / 16) as one bf16x8, from two gfx950 transpose reads
// ds_read_b64_tr_b16: in each 16-lane group, source lane s reads 4 consecutive columns 4 (s % 4) .. of row
// R0 + s / 4, and output lane j receives column j at rows R0 .. R0 + 3.
__device__ __forceinline__ bf16x8 ab_tr_frag(const bf16_t *tile, int r0, int dt, int lane) {
  const int g = lane >> 4, s = lane & 15;
  const bf16_t *p0 = tile + (r0 + 4 * g + (s >> 2)) * AB_PITCH + 16 * dt + 4 * (s & 3);
  const ab_s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ab_lds_s4 *)(const __attribute__((address_space(3))) bf16_t *)p0);
  const ab_s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (ab_lds_s4 *)(const __attribute__((address_space(3))) bf16_t *)(p0 + 16 * AB_PITCH));
  typedef short s8 __attribute__((ext_vector_type(8)));
  return __builtin_bit_cast(bf16x8, s8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
}

// D[r, h] = sum_d dO[r, h, d] * o[r, h, d]: one thread per (row, head)
__global__ __launch_bounds__(256) void attn_bwd_dot_kernel(const bf16_t *__restrict__ dout,
                                                          const bf16_t *__restrict__ out, float *__restrict__ dd,
                                                          int64_t n_rows) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // row * 8 + head
  if (i >= n_rows * AB_H) return;
  const u32x4 *a = reinterpret_cast<const u32x4 *>(dout + i * AB_D);
  const u32x4 *b = reinterpret_cast<const u32x4 *>(out + i * AB_D);
  u32x4 av[8], bv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    av[c] = a[c];
    bv[c] = b[c];
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += lo_bf(av[c][e]) * lo_bf(bv[c][e]) + hi_bf(av[c][e]) * hi_bf(bv[c][e]);
  dd[i] = s;
}

// Shared-prefix layout (the GSPO group's samples scored as one window each, their common prefix rows kept once):
// in dQ, sequence i's queries see first p_lens[i] prefix keys, rows of k / v from element p_off[i] (row stride
// stride_tok), then its own rows, query r at key position p_lens[i] + r. In dK / dV a work item is
// (sequence, first key, xr0, xl, slot): xl < 0 takes -xl of the sequence's own query rows from its row xr0
// (causal), xl >= 0 the xl rows from packed row xr0 (of q / dO / lse / D), each of which sees every key of the
// block (the samples' token rows against their prefix keys); slot < 0 writes dk / dv, slot >= 0 the partial rows
// part[slot][r0 + key], which attn_bwd_part_reduce_kernel sums over the slots in order into dk / dv (rows <
// n_part; a slot no item of a row writes must hold zeros). Not PREFIXED: plain causal self-attention with
// (sequence, first key) items.
struct AbPrefix {
  const int32_t *p_lens;
  const int64_t *p_off;
  float *part_k, *part_v;  // [slots, n_part, HKV, D]
  int64_t n_part;
};

// ---- dQ: workgroup = 64 query rows of one sequence x one KV head -----------------------------------------
template <bool PREFIXED>
__global__ __launch_bounds__(512) void attn_bwd_dq_kernel(
    const bf16_t *__restrict__ q, const bf16_t *__restrict__ k, const bf16_t *__restrict__ v,
    const bf16_t *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ dd,
    const int32_t *__restrict__ cu, const int32_t *__restrict__ plan, int n_seq, int64_t stride_tok,
    float *__restrict__ dq, float scale_log2, float scale, const AbPrefix pre) {
  // K and V rows: the A operands of S^T and dP^T, and (through transpose reads of K) of dQ^T = K^T dS^T
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][64 * AB_PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[2][64 * AB_PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int col = lane & 15, g = lane >> 4;
  const int hk = blockIdx.y, hq = hk * 4 + (wid & 3), half = wid >> 2;
  const int seq = plan[2 * blockIdx.x], qs = plan[2 * blockIdx.x + 1];
  if (seq < 0 || seq >= n_seq || qs < 0) return;
  const int64_t r0 = cu[seq];
  const int len = cu[seq + 1] - static_cast<int>(r0);
  if (len <= 0 || qs >= len) return;
  const int nq = min(64, len - qs);
  const int plen = PREFIXED ? pre.p_lens[seq] : 0;  // keys before the sequence's own rows
  const int64_t poff = PREFIXED ? pre.p_off[seq] : 0;
  const int klen = plen + len;
  const int kend = plen + qs + nq;  // causal: the block's last row sees keys < kend
  const int ntiles = (kend + 63) / 64;

  const int r_first = qs + 32 * half;
  int qpos[2];
  bf16x8 bq[2][2], bdo[2][2];
  float lse2[2], dr[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int r = r_first + 16 * qb + col;
    r = r < len ? r : len - 1;
    qpos[qb] = plen + r;
    const int64_t row = (r0 + r) * AB_H + hq;
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) {
      bq[qb][dc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(q + row * AB_D + 32 * dc + 8 * g));
      bdo[qb][dc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(dout + row * AB_D + 32 * dc + 8 * g));
    }
    lse2[qb] = lse[row];
    dr[qb] = dd[row];
  }
  const int wave_kmax = plen + min(r_first + 31, len - 1);

  f32x4 acc[4][2];  // dQ^T tiles [d tile][query block]
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lrow = tid >> 3, lchunk = tid & 7;
  u32x4 rk, rv;
  auto load_tile = [&](int t) {
    int key = t * 64 + lrow;
    key = key < klen ? key : klen - 1;
    const int64_t off = (PREFIXED && key < plen ? poff + static_cast<int64_t>(key) * stride_tok
                                                : (r0 + key - plen) * stride_tok) + hk * AB_D + lchunk * 8;
    rk = *reinterpret_cast<const u32x4 *>(k + off);
    rv = *reinterpret_cast<const u32x4 *>(v + off);
  };
  auto store_tile = [&](int buf) {
    *reinterpret_cast<u32x4 *>(&Ks[buf][lrow * AB_PITCH + lchunk * 8]) = rk;
    *reinterpret_cast<u32x4 *>(&Vs[buf][lrow * AB_PITCH + lchunk * 8]) = rv;
  };
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kbase = t * 64 + 32 * ks;
      if (kbase > wave_kmax) continue;  // wave-uniform: every key of this half is above every row's diagonal
      const bf16_t *kt = &Ks[buf][32 * ks * AB_PITCH];
      const bf16_t *vt = &Vs[buf][32 * ks * AB_PITCH];
      f32x4 st[2][2], dpt[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        bf16x8 ka[2], va[2];
#pragma unroll
        for (int dc = 0; dc < 2; ++dc) {
          ka[dc] = *reinterpret_cast<const bf16x8 *>(&kt[(16 * kb + col) * AB_PITCH + 32 * dc + 8 * g]);
          va[dc] = *reinterpret_cast<const bf16x8 *>(&vt[(16 * kb + col) * AB_PITCH + 32 * dc + 8 * g]);
        }
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          st[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dpt[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int dc = 0; dc < 2; ++dc) {
            st[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[dc], bq[qb][dc], st[kb][qb], 0, 0, 0);
            dpt[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dc], bdo[qb][dc], dpt[kb][qb], 0, 0, 0);
          }
        }
      }
      // dS^T in the accumulator layout (key 16 kb + 4 g + i, query col), as the B operand of K^T dS^T;
      // exponents are <= 0 (the row's log-sum-exp bounds every score), so the bare v_exp_f32 serves. Only a
      // half that reaches a row's diagonal is masked (a wave-uniform branch; a masked score's exponent is -inf)
      const bool need_mask = kbase + 31 > plen + r_first;
      bf16x8 dsf[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int hi_k = min(qpos[qb], klen - 1);
        float x[8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) x[kb * 4 + i] = fmaf(st[kb][qb][i], scale_log2, -lse2[qb]);
        if (need_mask) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[kb * 4 + i] = kbase + 16 * kb + 4 * g + i <= hi_k ? x[kb * 4 + i] : -INFINITY;
        }
        float d[8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            d[kb * 4 + i] = __builtin_amdgcn_exp2f(x[kb * 4 + i]) * (dpt[kb][qb][i] - dr[qb]);
        dsf[qb] = __builtin_bit_cast(bf16x8, u32x4{pack_bf(d[0], d[1]), pack_bf(d[2], d[3]), pack_bf(d[4], d[5]),
                                                    pack_bf(d[6], d[7])});
      }
      // dQ^T += K^T dS^T (key order {4g..4g+3, 16+4g..16+4g+3} in both operands; K^T by transpose reads)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const bf16x8 ka = ab_tr_frag(kt, 0, dt, lane);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) acc[dt][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, dsf[qb], acc[dt][qb], 0, 0, 0);
      }
    }
    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int r = r_first + 16 * qb + col;
    if (r >= len || r >= qs + nq) continue;
    float *dst = dq + ((r0 + r) * AB_H + hq) * AB_D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) *reinterpret_cast<f32x4 *>(dst + 16 * dt) = acc[dt][qb] * scale;
  }
}

// ---- dK / dV: workgroup = AB_KB keys of one sequence x one KV head ----------------------------------------
template <bool PREFIXED>
__global__ __launch_bounds__(AB_KW * 64, 2) void attn_bwd_dkdv_kernel(
    const bf16_t *__restrict__ q, const bf16_t *__restrict__ k, const bf16_t *__restrict__ v,
    const bf16_t *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ dd,
    const int32_t *__restrict__ cu, const int32_t *__restrict__ plan, int n_seq, int64_t stride_tok,
    float *__restrict__ dk, float *__restrict__ dv, float scale_log2, float scale, const AbPrefix pre) {
  // row-major Q / dO tiles [head][row]: the A operands of S and dP, and (through transpose reads) of dK^T and dV^T
  __shared__ __attribute__((aligned(16))) bf16_t Qs[4 * 32 * AB_PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t Os[4 * 32 * AB_PITCH];  // dO
  __shared__ float Ls[4 * 32], Ds[4 * 32];
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int col = lane & 15, g = lane >> 4;
  const int hk = blockIdx.y;
  constexpr int PS = PREFIXED ? 5 : 2;  // plan entry size
  const int seq = plan[PS * blockIdx.x], ks = plan[PS * blockIdx.x + 1];
  const int xl = PREFIXED ? plan[PS * blockIdx.x + 3] : -1;
  const int64_t xr0 = PREFIXED ? plan[PS * blockIdx.x + 2] : 0;
  const int slot = PREFIXED ? plan[PS * blockIdx.x + 4] : -1;
  if (seq < 0 || seq >= n_seq || ks < 0) return;
  const int64_t r0 = cu[seq];
  const int len = cu[seq + 1] - static_cast<int>(r0);
  if (len <= 0 || ks >= len) return;
  // query tiles: the sequence's own rows from the block's first key (causal), or the xl extra rows
  const bool xt = xl >= 0;  // extra rows: every row sees every key of the block
  // own rows (causal): rows r_beg .. r_lim - 1 of the sequence; extra rows: 0 .. xl - 1 from packed row xr0
  const int r_beg = xt ? 0 : (PREFIXED ? static_cast<int>(xr0) : ks);
  const int r_lim = xt ? xl : (PREFIXED ? min(len, r_beg - xl) : len);
  const int ntl = r_lim > r_beg ? (r_lim - r_beg + 31) / 32 : 0;

  // this wave's 32 keys, two blocks of 16 (lane col -> key of each), K^T / V^T fragments of the B operand
  int keyb[2];
  bf16x8 bk[2][2], bv[2][2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    keyb[kb] = ks + 32 * wid + 16 * kb + col;
    const int keyc = keyb[kb] < len ? keyb[kb] : len - 1;
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) {
      const int64_t off = (r0 + keyc) * stride_tok + hk * AB_D + 32 * dc + 8 * g;
      bk[kb][dc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(k + off));
      bv[kb][dc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(v + off));
    }
  }
  // dV^T / dK^T tiles [key block][d tile] (lane col -> key, 4 g + i -> d within the tile)
  f32x4 accv[2][4], acck[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) accv[kb][dt] = acck[kb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int wave_kmin = ks + 32 * wid;  // rows below it see none of this wave's keys

  // staging: thread t loads 16-byte chunks t + NT c (c < 1024 / NT) of the Q tile and of the dO tile:
  // chunk -> (head hh = chunk / 256, row rr = chunk / 8 % 32, d chunk dc8 = chunk % 8), and threads t < 256
  // one lse (t < 128) or D value. Software pipelined: tile rs + 32 is loaded while tile rs is computed.
  constexpr int NT = AB_KW * 64, NC = 1024 / NT;
  u32x4 qv[NC], ov[NC];
  float lv = 0.f;
  // query tile it: rows rs .. rs + 31 of the sequence (rs = ks + 32 it) or of the extra rows (rs = 32 it)
  auto tile_rows = [&](int it, int &rs, int &n, int64_t &base) {
    rs = r_beg + 32 * it;
    n = r_lim;
    base = xt ? xr0 : r0;
  };
  auto load_tile = [&](int it) {
    int rs, n;
    int64_t base;
    tile_rows(it, rs, n, base);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int chunk = tid + NT * c;
      const int hh = chunk >> 8, rr = (chunk >> 3) & 31, dc8 = chunk & 7;
      int r = rs + rr;
      r = r < n ? r : n - 1;
      const int64_t off = ((base + r) * AB_H + hk * 4 + hh) * AB_D + 8 * dc8;
      qv[c] = *reinterpret_cast<const u32x4 *>(q + off);
      ov[c] = *reinterpret_cast<const u32x4 *>(dout + off);
    }
    const int hh = (tid & 127) >> 5, rr = tid & 31;
    int r = rs + rr;
    r = r < n ? r : n - 1;
    const int64_t row = (base + r) * AB_H + hk * 4 + hh;
    lv = tid < 128 ? lse[row] : dd[row];  // (threads >= 256 load a D value they do not store)
  };
  if (ntl > 0) load_tile(0);
  for (int it = 0; it < ntl; ++it) {
    int rs, n;
    int64_t base;
    tile_rows(it, rs, n, base);
    __syncthreads();  // the previous tile's readers are done
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int chunk = tid + NT * c;
      const int hh = chunk >> 8, rr = (chunk >> 3) & 31, dc8 = chunk & 7;
      *reinterpret_cast<u32x4 *>(&Qs[(hh * 32 + rr) * AB_PITCH + 8 * dc8]) = qv[c];
      *reinterpret_cast<u32x4 *>(&Os[(hh * 32 + rr) * AB_PITCH + 8 * dc8]) = ov[c];
    }
    if (tid < 128)
      Ls[tid] = lv;
    else if (tid < 256)
      Ds[tid - 128] = lv;
    __syncthreads();
    if (it + 1 < ntl) load_tile(it + 1);
    if (!xt && rs + 31 < wave_kmin) continue;  // wave-uniform: every row of the tile lies above this wave's keys

#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const bf16_t *qt = &Qs[hh * 32 * AB_PITCH];
      const bf16_t *ot = &Os[hh * 32 * AB_PITCH];
      // S / dP [key block][row 16 rb + 4 g + i][key col]: each Q / dO fragment serves both key blocks
      f32x4 st[2][2], dpt[2][2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) st[kb][rb] = dpt[kb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dc = 0; dc < 2; ++dc) {
          const bf16x8 qa = *reinterpret_cast<const bf16x8 *>(&qt[(16 * rb + col) * AB_PITCH + 32 * dc + 8 * g]);
          const bf16x8 oa = *reinterpret_cast<const bf16x8 *>(&ot[(16 * rb + col) * AB_PITCH + 32 * dc + 8 * g]);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            st[kb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa, bk[kb][dc], st[kb][rb], 0, 0, 0);
            dpt[kb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(oa, bv[kb][dc], dpt[kb][rb], 0, 0, 0);
          }
        }
      }
      // row order {4g..4g+3, 16+4g..16+4g+3}; exponents are <= 0 (bare v_exp_f32). A tile wholly below the
      // diagonal and inside the sequence needs no mask (a wave-uniform branch); else a masked entry's exponent
      // is -inf (exp2 -> 0)
      const bool full = xt ? rs + 31 < n && wave_kmin + 31 < len : wave_kmin + 31 <= rs && rs + 31 < n;
      bf16x8 pf[2], dsf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int key = keyb[kb];
        float x[8];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int i = 0; i < 4; ++i) x[rb * 4 + i] = fmaf(st[kb][rb][i], scale_log2, -Ls[hh * 32 + 16 * rb + 4 * g + i]);
        if (!full) {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int r = rs + 16 * rb + 4 * g + i;
              const bool ok = (r < n) & (xt | (key <= r)) & (key < len);
              x[rb * 4 + i] = ok ? x[rb * 4 + i] : -INFINITY;
            }
        }
        float pv[8], dv8[8];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(x[rb * 4 + i]);
            pv[rb * 4 + i] = p;
            dv8[rb * 4 + i] = p * (dpt[kb][rb][i] - Ds[hh * 32 + 16 * rb + 4 * g + i]);
          }
        pf[kb] = __builtin_bit_cast(bf16x8, u32x4{pack_bf(pv[0], pv[1]), pack_bf(pv[2], pv[3]), pack_bf(pv[4], pv[5]),
                                                   pack_bf(pv[6], pv[7])});
        dsf[kb] = __builtin_bit_cast(bf16x8, u32x4{pack_bf(dv8[0], dv8[1]), pack_bf(dv8[2], dv8[3]),
                                                    pack_bf(dv8[4], dv8[5]), pack_bf(dv8[6], dv8[7])});
      }
      // dV^T += dO^T P, dK^T += Q^T dS (A = dO^T / Q^T by transpose reads of the row-major tiles: lane col -> d,
      // rows {4g..4g+3} and {16+4g..16+4g+3}, the row order of P / dS above; each fragment serves both key blocks)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const bf16x8 qa = ab_tr_frag(qt, 0, dt, lane);
        const bf16x8 oa = ab_tr_frag(ot, 0, dt, lane);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          accv[kb][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(oa, pf[kb], accv[kb][dt], 0, 0, 0);
          acck[kb][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa, dsf[kb], acck[kb][dt], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if (keyb[kb] < len) {
      const int64_t orow = slot < 0 ? r0 + keyb[kb] : slot * pre.n_part + r0 + keyb[kb];
      float *dkp = (slot < 0 ? dk : pre.part_k) + (orow * AB_HKV + hk) * AB_D + 4 * g;
      float *dvp = (slot < 0 ? dv : pre.part_v) + (orow * AB_HKV + hk) * AB_D + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        *reinterpret_cast<f32x4 *>(dkp + 16 * dt) = acck[kb][dt] * scale;
        *reinterpret_cast<f32x4 *>(dvp + 16 * dt) = accv[kb][dt];
      }
    }
  }
}

// dk / dv rows 0 .. n_part - 1 = the sum over slots 0 .. S - 1 of part[slot] (in slot order), 4 values per thread
__global__ __launch_bounds__(256) void attn_bwd_part_reduce_kernel(const float *__restrict__ part_k,
                                                                  const float *__restrict__ part_v,
                                                                  float *__restrict__ dk, float *__restrict__ dv,
                                                                  int64_t n4, int S) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n4) return;
  const f32x4 *pk = reinterpret_cast<const f32x4 *>(part_k), *pv = reinterpret_cast<const f32x4 *>(part_v);
  f32x4 a = pk[i], b = pv[i];
  for (int s = 1; s < S; ++s) {
    a += pk[s * n4 + i];
    b += pv[s * n4 + i];
  }
  reinterpret_cast<f32x4 *>(dk)[i] = a;
  reinterpret_cast<f32x4 *>(dv)[i] = b;
}

}  // namespace vk

using namespace vk;

static int attn_bwd_launch(const void *q, const void *k, const void *v, const void *out, const void *dout,
                           const float *lse, const int32_t *cu, int32_t n_seq, const int32_t *q_plan,
                           int32_t n_qblocks, const int32_t *k_plan, int32_t n_kblocks, int64_t n_rows,
                           int64_t stride_tok, const AbPrefix *pre, int32_t n_slots, float *dd, float *dq,
                           float *dk, float *dv, int32_t H, int32_t HKV, int32_t D, void *stream) {
  VK_CHECK_ARG(q && k && v && out && dout && lse && cu && dd && dq && dk && dv, "attention_backward: null pointer");
  if (H != AB_H || HKV != AB_HKV || D != AB_D)
    return fail(VK_ERR_UNSUPPORTED, "attention_backward: built for H=8 HKV=2 D=64 (got %d/%d/%d)", H, HKV, D);
  VK_CHECK_ARG(n_seq >= 0 && n_rows >= 0 && n_qblocks >= 0 && n_kblocks >= 0 && stride_tok >= AB_HKV * AB_D &&
                   stride_tok % 8 == 0,
               "attention_backward: bad sizes");
  VK_CHECK_ARG((n_qblocks == 0 || q_plan) && (n_kblocks == 0 || k_plan), "attention_backward: missing plan");
  VK_CHECK_ARG(vk_aligned16(q) && vk_aligned16(k) && vk_aligned16(v) && vk_aligned16(out) && vk_aligned16(dout) &&
                   vk_aligned16(dq) && vk_aligned16(dk) && vk_aligned16(dv),
               "attention_backward: pointers must be 16-byte aligned");
  VK_CHECK_ARG(pre == nullptr || (pre->p_lens && pre->p_off && pre->n_part >= 0 &&
                                  (pre->n_part == 0 || (pre->part_k && pre->part_v && vk_aligned16(pre->part_k) &&
                                                        vk_aligned16(pre->part_v)))),
               "attention_backward_prefixed: prefix arrays or partial buffers");
  if (n_rows == 0) return VK_OK;
  hipStream_t s = VK_STREAM(stream);
  const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(AB_D)));
  const float scale_log2 = static_cast<float>(1.0 / sqrt(static_cast<double>(AB_D)) * 1.4426950408889634);
  const auto qb = static_cast<const bf16_t *>(q);
  const auto kb = static_cast<const bf16_t *>(k);
  const auto vb = static_cast<const bf16_t *>(v);
  const auto ob = static_cast<const bf16_t *>(out);
  const auto dob = static_cast<const bf16_t *>(dout);
  const AbPrefix none{nullptr, nullptr, nullptr, nullptr, 0};
  const int64_t nd = n_rows * AB_H;
  attn_bwd_dot_kernel<<<static_cast<unsigned>((nd + 255) / 256), 256, 0, s>>>(dob, ob, dd, n_rows);
  int rc = launch_status("attention_backward dot");
  if (rc != VK_OK) return rc;
  if (n_qblocks > 0) {
    const dim3 grid(static_cast<unsigned>(n_qblocks), AB_HKV);
    if (pre != nullptr)
      attn_bwd_dq_kernel<true><<<grid, 512, 0, s>>>(qb, kb, vb, dob, lse, dd, cu, q_plan, n_seq, stride_tok, dq,
                                                   scale_log2, scale, *pre);
    else
      attn_bwd_dq_kernel<false><<<grid, 512, 0, s>>>(qb, kb, vb, dob, lse, dd, cu, q_plan, n_seq, stride_tok, dq,
                                                    scale_log2, scale, none);
    rc = launch_status("attention_backward dq");
    if (rc != VK_OK) return rc;
  }
  if (n_kblocks > 0) {
    const dim3 grid(static_cast<unsigned>(n_kblocks), AB_HKV);
    if (pre != nullptr)
      attn_bwd_dkdv_kernel<true><<<grid, AB_KW * 64, 0, s>>>(qb, kb, vb, dob, lse, dd, cu, k_plan, n_seq, stride_tok,
                                                            dk, dv, scale_log2, scale, *pre);
    else
      attn_bwd_dkdv_kernel<false><<<grid, AB_KW * 64, 0, s>>>(qb, kb, vb, dob, lse, dd, cu, k_plan, n_seq, stride_tok,
                                                             dk, dv, scale_log2, scale, none);
    rc = launch_status("attention_backward dkdv");
    if (rc != VK_OK) return rc;
  }
  if (pre != nullptr && pre->n_part > 0 && n_slots > 0) {
    const int64_t n4 = pre->n_part * AB_HKV * AB_D / 4;
    attn_bwd_part_reduce_kernel<<<static_cast<unsigned>((n4 + 255) / 256), 256, 0, s>>>(pre->part_k, pre->part_v, dk,
                                                                                        dv, n4, n_slots);
    rc = launch_status("attention_backward partial sums");
  }
  return rc;
}

extern "C" int vk_attention_backward(const void *q, const void *k, const void *v, const void *out, const void *dout,
                                     const float *lse, const int32_t *cu, int32_t n_seq, const int32_t *q_plan,
                                     int32_t n_qblocks, const int32_t *k_plan, int32_t n_kblocks, int64_t n_rows,
                                     int64_t stride_tok, float *dd, float *dq, float *dk, float *dv, int32_t H,
                                     int32_t HKV, int32_t D, void *stream) {
  return attn_bwd_launch(q, k, v, out, dout, lse, cu, n_seq, q_plan, n_qblocks, k_plan, n_kblocks, n_rows, stride_tok,
                         nullptr, 0, dd, dq, dk, dv, H, HKV, D, stream);
}

extern "C" int vk_attention_backward_prefixed(const void *q, const void *k, const void *v, const void *out,
                                              const void *dout, const float *lse, const int32_t *cu, int32_t n_seq,
                                              const int32_t *q_plan, int32_t n_qblocks, const int32_t *k_plan,
                                              int32_t n_kblocks, int64_t n_rows, int64_t stride_tok,
                                              const int32_t *p_lens, const int64_t *p_off, float *part_k,
                                              float *part_v, int64_t n_part, int32_t n_slots, float *dd, float *dq,
                                              float *dk, float *dv, int32_t H, int32_t HKV, int32_t D, void *stream) {
  VK_CHECK_ARG(n_slots >= 0 && n_part <= n_rows, "attention_backward_prefixed: bad partial sizes");
  const AbPrefix pre{p_lens, p_off, part_k, part_v, n_part};
  return attn_bwd_launch(q, k, v, out, dout, lse, cu, n_seq, q_plan, n_qblocks, k_plan, n_kblocks, n_rows, stride_tok,
                         &pre, n_slots, dd, dq, dk, dv, H, HKV, D, stream);
}
