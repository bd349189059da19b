// The GSPO reward on the device: strict identity of each call against its window's label
// (scripts/gspo.py:86-89 with ref_errors, scripts/train.py:170-188):
//   empty label: 1 if len(call) <= empty_max else empty_max / len(call);
//   else 1 - (errors of the global (NW) alignment path that fall on scored label bases) / max(len(call), len(label)),
// where a mismatch or a deletion counts at its label base and an insertion at the label base before it
// (the first base for an insertion before any label base).
//
// The reference takes the path edlib's traceback returns (edlib.align(call, label, "NW", "path")). Here the
// path is fixed by a stated preference among the optimal predecessors of each cell -- diagonal (match or
// mismatch), then up (deletion of a label base), then left (insertion of a call base) -- and the count of
// scored errors is carried forward along each cell's chosen predecessor, which is exactly the count along
// the traceback from the last cell with the same preference (no traceback pass, no per-cell storage). The
// edit distance, and the count when every label base is scored, do not depend on the choice of path.
//
// MI355X design: one wavefront per call; the DP advances by anti-diagonals (cells i + j = k), lane l takes
// the cells l, l + 64, ... of a diagonal, and three rolling diagonals of (distance, count) pairs live in
// LDS as int16, next to the label, its scored mask and the call. Integer work only, a few hundred thousand
// cells per call: every call of a rollout runs concurrently (one wavefront each).
#include "common.h"

namespace vk {

constexpr int RW_MAX_REF = 4096;   // label bases (LDS: 3 diagonals x 2 arrays x int16)
constexpr int RW_MAX_CALL = 8192;  // call bases (distances stay below 32767)

__global__ __launch_bounds__(64) void strict_identity_kernel(
    const uint8_t *__restrict__ calls, const int64_t *__restrict__ call_off, const int32_t *__restrict__ call_len,
    const uint8_t *__restrict__ refs, const int64_t *__restrict__ ref_off, const int32_t *__restrict__ ref_len,
    const uint8_t *__restrict__ scored, const int32_t *__restrict__ ref_of_call, int n_refs, int max_ref,
    int max_call, float empty_max, float *__restrict__ reward, int32_t *__restrict__ dist_out,
    int32_t *__restrict__ err_out) {
  extern __shared__ __attribute__((aligned(16))) char rw_smem[];
  const int lane = threadIdx.x;
  const int c = blockIdx.x;
  int r = ref_of_call[c];
  r = r < 0 ? 0 : (r >= n_refs ? n_refs - 1 : r);
  int n = call_len[c], m = ref_len[r];
  n = n < 0 ? 0 : (n > max_call ? max_call : n);  // (LDS is sized for max_ref / max_call)
  m = m < 0 ? 0 : (m > max_ref ? max_ref : m);
  if (m == 0) {  // a window without DNA
    if (lane == 0) {
      reward[c] = n <= empty_max ? 1.0f : empty_max / static_cast<float>(n);
      dist_out[c] = n;
      err_out[c] = 0;
    }
    return;
  }
  const int W = max_ref + 1;  // diagonal arrays indexed by the label row i = 0 .. m
  int16_t *dg = reinterpret_cast<int16_t *>(rw_smem);    // [3][W] distances
  int16_t *cn = dg + 3 * W;                              // [3][W] scored-error counts
  uint8_t *rs = reinterpret_cast<uint8_t *>(cn + 3 * W);  // label
  uint8_t *sc = rs + max_ref;                             // scored mask of the label
  uint8_t *cs = sc + max_ref;                             // call
  const uint8_t *rg = refs + ref_off[r], *sg = scored + ref_off[r], *cg = calls + call_off[c];
  for (int i = lane; i < m; i += 64) {
    rs[i] = rg[i];
    sc[i] = sg[i] ? 1 : 0;
  }
  for (int j = lane; j < n; j += 64) cs[j] = cg[j];
  __syncthreads();

  // diagonal k = i + j lives in slot k % 3
  for (int k = 0; k <= m + n; ++k) {
    int16_t *d0 = dg + (k % 3) * W, *c0 = cn + (k % 3) * W;
    const int16_t *d1 = dg + ((k + 2) % 3) * W, *c1 = cn + ((k + 2) % 3) * W;  // k - 1
    const int16_t *d2 = dg + ((k + 1) % 3) * W, *c2 = cn + ((k + 1) % 3) * W;  // k - 2
    const int lo = k - n > 0 ? k - n : 0, hi = k < m ? k : m;
    for (int i = lo + lane; i <= hi; i += 64) {
      const int j = k - i;
      int d, e;
      if (i == 0) {  // first label row: j insertions, each counted at label base 0
        d = j;
        e = j > 0 ? c1[0] + sc[0] : 0;
      } else if (j == 0) {  // first call column: i deletions
        d = i;
        e = c1[i - 1] + sc[i - 1];
      } else {
        const int mis = rs[i - 1] != cs[j - 1];
        const int dd = d2[i - 1] + mis, du = d1[i - 1] + 1, dl = d1[i] + 1;
        d = dd < du ? dd : du;
        d = dl < d ? dl : d;
        if (dd == d)
          e = c2[i - 1] + (mis ? sc[i - 1] : 0);  // match / mismatch at label base i - 1
        else if (du == d)
          e = c1[i - 1] + sc[i - 1];  // deletion of label base i - 1
        else
          e = c1[i] + sc[i - 1];  // insertion after label base i - 1
      }
      d0[i] = static_cast<int16_t>(d);
      c0[i] = static_cast<int16_t>(e);
    }
    __syncthreads();  // one wavefront: orders this diagonal's LDS writes before the next one's reads
  }
  if (lane == 0) {
    const int slot = (m + n) % 3;
    const int d = dg[slot * W + m], e = cn[slot * W + m];
    dist_out[c] = d;
    err_out[c] = e;
    reward[c] = 1.0f - static_cast<float>(e) / static_cast<float>(n > m ? n : m);
  }
}

}  // namespace vk

using namespace vk;

extern "C" int vk_strict_identity(const uint8_t *calls, const int64_t *call_off, const int32_t *call_len,
                                  const uint8_t *refs, const int64_t *ref_off, const int32_t *ref_len,
                                  const uint8_t *scored, const int32_t *ref_of_call, int32_t n_calls, int32_t n_refs,
                                  int32_t max_ref_len, int32_t max_call_len, float empty_max, float *reward,
                                  int32_t *edit_distance, int32_t *scored_errors, void *stream) {
  VK_CHECK_ARG(call_off && call_len && ref_off && ref_len && ref_of_call && reward && edit_distance && scored_errors,
               "strict_identity: null pointer");
  VK_CHECK_ARG(n_calls >= 0 && n_refs > 0 && max_ref_len >= 0 && max_call_len >= 0, "strict_identity: bad sizes");
  if (max_ref_len > RW_MAX_REF || max_call_len > RW_MAX_CALL)
    return fail(VK_ERR_UNSUPPORTED, "strict_identity: labels up to %d and calls up to %d bases (got %d / %d)",
                RW_MAX_REF, RW_MAX_CALL, max_ref_len, max_call_len);
  VK_CHECK_ARG((max_call_len == 0 || calls) && (max_ref_len == 0 || (refs && scored)), "strict_identity: null data");
  if (n_calls == 0) return VK_OK;
  // LDS: 3 diagonals x (distance, count) int16 of max_ref_len + 1 rows, the label, its mask and the call
  const size_t lds = 3 * 2 * 2 * static_cast<size_t>(max_ref_len + 1) + 2 * static_cast<size_t>(max_ref_len) +
                     static_cast<size_t>(max_call_len) + 16;
  // labels past about 3.3 kb need more than the default 64 KB of dynamic LDS: the limit is raised once, to what the
  // largest label and call take, so concurrent callers never lower it under each other
  constexpr size_t kMaxLds = 3 * 2 * 2 * static_cast<size_t>(RW_MAX_REF + 1) + 2 * static_cast<size_t>(RW_MAX_REF) +
                             static_cast<size_t>(RW_MAX_CALL) + 16;
  if (lds > 65536) VK_RAISE_LDS_ONCE(strict_identity_kernel, kMaxLds, "strict_identity");
  strict_identity_kernel<<<static_cast<unsigned>(n_calls), 64, lds, VK_STREAM(stream)>>>(
      calls, call_off, call_len, refs, ref_off, ref_len, scored, ref_of_call, n_refs, max_ref_len, max_call_len,
      empty_max, reward, edit_distance, scored_errors);
  return launch_status("strict_identity");
}
