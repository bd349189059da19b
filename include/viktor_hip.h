/*
 * viktor_hip.h -- C ABI of libviktor_hip.so, the gfx950 (MI355X) kernels of the decoder's
 * rollout-and-scoring path.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers (HIP device memory) unless stated otherwise;
 *     bf16 tensors are passed as raw 16-bit storage, row-major and contiguous unless a
 *     stride argument is given;
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream); every kernel is
 *     enqueued on it, nothing synchronises the device, nothing allocates device memory,
 *     so every entry point may be recorded into a HIP graph;
 *   - the return value is VK_OK (0) or a VK_ERR_* code; vk_last_error() returns the
 *     message of the last failure on the calling host thread.
 *   - device-side indices read from memory (token ids, positions, cache rows, lengths)
 *     are bounds-checked inside the kernels against the sizes passed here: an
 *     out-of-range write is skipped, an out-of-range read is clamped.
 *
 * Each declaration names the reference function it replaces (file:line of GHSSHG/Viktor).
 */
#ifndef VIKTOR_HIP_H
#define VIKTOR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VK_OK 0
#define VK_ERR_ARG 1         /* invalid argument: shape, size, alignment or null pointer */
#define VK_ERR_LAUNCH 2      /* the HIP runtime rejected a kernel launch */
#define VK_ERR_UNSUPPORTED 3 /* a configuration these kernels are not built for */

#define VK_DTYPE_BF16 0
#define VK_DTYPE_F32 1

/* Library version (major * 10000 + minor * 100 + patch). */
int vk_version(void);

/* Message of the last non-zero status returned on this host thread ("" if none). */
const char *vk_last_error(void);

/* Number of compute units of the current device (0 on failure); used to size launch grids. */
int vk_device_cus(void);

/*
 * x[n, d] += delta[n, d] (bf16, in place; delta may be NULL), then
 * h[n, d] = bf16(x * rsqrt(mean(x^2) + eps) * w), fp32 inside.
 * Replaces add_rmsnorm, viktor/triton_ops.py:17-40.
 */
int vk_add_rmsnorm(void *x, const void *delta, const void *w, void *h, int64_t n, int32_t d, float eps,
                   void *stream);

/*
 * x[i, :] = emb[tok[i], :] and h = RMSNorm(x) * w (bf16). Token ids outside [0, vocab) give a zero row.
 * Replaces embed_rmsnorm, viktor/triton_ops.py:149-169.
 */
int vk_embed_rmsnorm(const int64_t *tok, const void *emb, int64_t vocab, const void *w, void *x, void *h,
                     int64_t n, int32_t d, float eps, void *stream);

/*
 * Per token t of qkv[n, (H + 2 HKV) * D]: heads 0..H-1 are q, then HKV k heads, then HKV v heads.
 * q and k heads get RMSNorm over D (weights q_norm_w / k_norm_w, result rounded to bf16) and the
 * half-split RoPE rotation at row rope_pos[t] of cos/sin [table_rows, D/2] (table_dtype bf16 or f32).
 * q[n, H, D] receives the rotated q heads; k (rotated) and v go to
 * k_cache/v_cache + seq[t] * stride_cb + pos[t] * stride_cs (+ head * D) when the cache pointers are
 * non-NULL and seq[t] < cache_rows, pos[t] < cache_len; and to k_out/v_out[n, HKV, D] when non-NULL.
 * rope_pos may be NULL (then pos is used). Norm weights bf16 or fp32 per norm_w_dtype (fp32: the master weights
 * autocast keeps in fp32; same rounding points).
 * Replaces qkv_rope_cache, viktor/triton_ops.py:43-108.
 */
int vk_qkv_rope_cache(const void *qkv, const void *q_norm_w, const void *k_norm_w, int32_t norm_w_dtype,
                      const void *cos_t, const void *sin_t, int32_t table_dtype, int64_t table_rows, const int32_t *pos,
                      const int32_t *rope_pos, const int32_t *seq, void *q, void *k_cache, void *v_cache,
                      int64_t stride_cb, int64_t stride_cs, int64_t cache_rows, int64_t cache_len, void *k_out,
                      void *v_out, int64_t n, float eps, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                      void *stream);

/*
 * y[M, N] = x[M, K] @ w[N, K]^T on bf16 MFMA with fp32 accumulation; y is bf16 (out_dtype
 * VK_DTYPE_BF16) or fp32 (VK_DTYPE_F32).
 * swiglu != 0: w is gate_up [2N, K] and y[M, N] = bf16(bf16(silu(bf16(x w_gate^T))) * bf16(x w_up^T)),
 * the rounding points of the unfused linear + SwiGLU path; gu_out (NULL: none, swiglu only) then also receives
 * the gate | up product rows [M, 2N] in bf16, as the plain product stores them (the SwiGLU backward's operand).
 * Requires K % 32 == 0 and 16-byte aligned x, w.
 * Replaces linear (viktor/triton_ops.py:111-146), swiglu (212-229) and the F.linear / nn.Linear
 * projections of viktor/fast_decoder.py:39,56-57 and viktor/decoder.py:58-59,114-115,163-164.
 */
int vk_linear(const void *x, const void *w, void *y, int64_t M, int32_t N, int32_t K, int32_t swiglu,
              int32_t out_dtype, void *gu_out, void *stream);

/*
 * out[n, F] = bf16(bf16(silu(gate)) * up) for gu[n, 2F] = [gate | up] (bf16).
 * Replaces swiglu, viktor/triton_ops.py:212-229.
 */
int vk_swiglu(const void *gu, void *out, int64_t n, int32_t f, void *stream);

/*
 * Group check of DecodeEngine(group_size=G) before its one-prefill-per-window: x holds groups x G members of
 * member_bytes each (16-byte aligned, member_bytes % 16 == 0); stores 1 to *flag when any member differs from its
 * group's first member bit for bit (the caller zeroes *flag first; nothing is stored when all are equal).
 * No reference counterpart: the reference prefills every repeated window (scripts/gspo.py:444).
 */
int vk_group_rows_equal(const void *x, int64_t groups, int32_t G, int64_t member_bytes, int32_t *flag, void *stream);

/*
 * Large-M residual product, in place (a [M, K], w [N, K] bf16, bias fp32 [N] or NULL; N % 128 == 0, K % 64 == 0):
 *   x_dtype bf16: x[M, N] = bf16(bf16(a w^T + bias) + bf16(alpha x)). alpha = 1 without bias is the residual add
 *     of add_rmsnorm (viktor/triton_ops.py:17-31, x += delta after the o / down projections of
 *     viktor/fast_decoder.py:56-58); with the out_proj bias and the DeepNorm alpha it is the encoder's norm input
 *     (viktor/encoder.py:106-108);
 *   x_dtype f32: x[M, N] = alpha x + bf16(a w^T + bias) in fp32, the residual add x + sublayer(x) of an fp32 stream
 *     under torch.autocast bf16 (viktor/decoder.py:118-120 as scripts/gspo.py:345-347 runs it).
 * ss_out[M, N / 64] = the fp32 sum of squares of each row's new values per 64-column block.
 * x_in (NULL: x itself): where the old residual is read, so x may be a fresh buffer and x_in the previous layer's
 * stream, kept for the backward (the autograd graph of the reference keeps every layer's input alive).
 */
int vk_linear_residual_big(const void *a, const void *w, void *x, int32_t x_dtype, int64_t M, int32_t N, int32_t K,
                           const float *bias, float alpha, float *ss_out, const void *x_in, void *stream);

/*
 * RMSNorm from handed-over sums of squares: h = bf16(x * rsqrt(sum_b ss[row, b] / d + eps) * w) (x and w bf16 or
 * fp32 per x_dtype / w_dtype, h bf16, ss [n, nb] fp32 summed in block order; h may be x when x is bf16). The norm
 * half of add_rmsnorm (viktor/triton_ops.py:28-31) after vk_linear_residual_big; with fp32 x and w, nn.RMSNorm of
 * the fp32 residual stream rounded once at the next product's autocast input (viktor/decoder.py:119, 144).
 */
int vk_rmsnorm_apply_ss(const void *x, int32_t x_dtype, const float *ss, int32_t nb, const void *w, int32_t w_dtype,
                        void *h, int64_t n, int32_t d, float eps, void *stream);

/*
 * RMSNorm of an fp32 residual stream with fp32 weights, rounded once to bf16: h = bf16(x rsqrt(mean x^2 + eps) w)
 * (x [n, d], w [d] fp32; d % 8 == 0, d <= 2048). The first attention norm of the autocast teacher-forced forward
 * (nn.RMSNorm at viktor/decoder.py:118 on the fp32 rows viktor/model.py:81-84 builds, cast to bf16 by autocast at
 * qkv_proj).
 */
int vk_rmsnorm_f32(const float *x, const float *w, void *h, int64_t n, int32_t d, float eps, void *stream);

/*
 * The Wqkv product with vk_qkv_rope_cache fused into its epilogue (prefill and the encoder): qkv = x w^T
 * (x [M, K], w [(H + 2 HKV) 64, K] bf16, K % 64 == 0) rounded to bf16 as the unfused product stores it; the
 * q and k heads get the per-head RMSNorm (q_norm_w / k_norm_w, both NULL: none) and the half-split RoPE at
 * rope_pos[t] (NULL: pos[t]) of cos/sin [table_rows, 32] (table_dtype bf16 or f32), with the rounding points
 * of vk_qkv_rope_cache; q head h of row t goes to q + t q_ld + 64 h; k / v head h to the cache
 * (k_cache + seq[t] stride_cb + pos[t] stride_cs + 64 h, when seq[t] < cache_rows and pos[t] < cache_len) and /
 * or to k_out / v_out + t kv_ld + 64 h. head_dim must be 64; 16-byte aligned pointers, strides % 8 == 0.
 * Replaces linear + qkv_rope_cache (viktor/triton_ops.py:43-108, 138-146; viktor/fast_decoder.py:39-47) and
 * the Wqkv product + apply_rope of the encoder (viktor/encoder.py:71-75). norm_w_dtype f32 (with f32 tables):
 * fp32 norm weights, the autocast forward's Attention.project (viktor/decoder.py:63-67): nn.RMSNorm of a bf16 head
 * with fp32 weights returns bf16(x / rms * w), then apply_rope in fp32 rounds back to bf16.
 * qkv_out (NULL: none): also the product itself, rounded to bf16, as rows [M, (H + 2 HKV) 64] (the unrotated
 * projection output the QK-norm + RoPE backward takes).
 */
int vk_linear_qkv_rope(const void *x, const void *w, int64_t M, int32_t K, const void *q_norm_w, const void *k_norm_w,
                       int32_t norm_w_dtype, float eps, const void *cos_t, const void *sin_t, int32_t table_dtype, int64_t table_rows,
                       const int32_t *pos, const int32_t *rope_pos, const int32_t *seq, void *q, int64_t q_ld,
                       void *k_cache, void *v_cache, int64_t stride_cb, int64_t stride_cs, int64_t cache_rows,
                       int64_t cache_len, void *k_out, void *v_out, int64_t kv_ld, void *qkv_out, int32_t n_heads,
                       int32_t n_kv_heads, int32_t head_dim, void *stream);

/*
 * Single-query GQA attention against one layer of the KV cache:
 * out[b, h, :] = softmax(q[b, h] . K[r, :len_b, h / (H/HKV)]^T / sqrt(D)) V[r, :len_b, ...]
 * with len_b = clamp(lengths[b], 1, max_len) and cache row r = rows[b] (rows NULL: r = b);
 * k_cache/v_cache element (r, s, hk, d) at r * stride_b + s * stride_s + hk * D + d, for
 * 0 <= r < cache_rows (a sequence whose row falls outside gets a zero output; with rows NULL,
 * cache_rows must be >= B). fp32 online softmax, probabilities rounded to bf16 before the PV product
 * (as the reference kernel). Each K/V row is read once for its query-head group.
 * Built for H = 8, HKV = 2, D = 64. workspace: vk_decode_attention_workspace() bytes (may be 0 bytes
 * when no split of the key range is needed; then workspace may be NULL).
 * Replaces decode_attention, viktor/decode_attention.py:11-53, and the flash_attn_with_kvcache decode
 * with cache_batch_idx = seq of viktor/fast_decoder.py:86-89 (rows).
 */
int vk_decode_attention(const void *q, const void *k_cache, const void *v_cache, const int32_t *lengths,
                        const int32_t *rows, int64_t cache_rows, void *out, int64_t B, int32_t H, int32_t HKV,
                        int32_t D, int64_t stride_b, int64_t stride_s, int64_t max_len, void *workspace,
                        int64_t workspace_bytes, void *stream);

/* Workspace bytes vk_decode_attention needs for this batch and cache length. */
int vk_decode_attention_workspace(int64_t B, int32_t H, int64_t max_len, int64_t *bytes);

/*
 * vk_decode_attention without a workspace argument and without any allocation: the key-split partials go to a
 * 4 MiB static device array of the library (one per GPU, held until the process ends; its device address is
 * looked up once per device, on the first call there). Same arguments (minus workspace), kernels and results,
 * bit for bit, as vk_decode_attention. Returns VK_ERR_ARG when the split needs more than 4 MiB of partials
 * (B x splits x 8 heads x 66 floats; at most ~2 x CUs + B rows of them, so never on a 256-CU MI355X).
 * Calls that overlap on one GPU (two streams, or two host threads) share that array and race: serialise them.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 */
int vk_decode_attention_noalloc(const void *q, const void *k_cache, const void *v_cache, const int32_t *lengths,
                                const int32_t *rows, int64_t cache_rows, void *out, int64_t B, int32_t H, int32_t HKV,
                                int32_t D, int64_t stride_b, int64_t stride_s, int64_t max_len, void *stream);

/*
 * Decode attention for groups of G consecutive sequences that share a prefix (GSPO: the G samples of one
 * window). Sequence b (group p = b / G) attends to prefix rows [0, prefix_len[p]) of k_prefix/v_prefix
 * (row r of group p at p * stride_pb + r * stride_ps) followed by its own rows [0, suffix_len[b]) of
 * k_suffix/v_suffix (b * stride_sb + r * stride_ss); softmax over the union, same numerics as
 * vk_decode_attention. Each prefix row is read once per group (not once per sequence).
 * G in {2, 4, 8, 16}; H = 8, HKV = 2, D = 64; workspace: vk_decode_attention_grouped_workspace() bytes.
 * Replaces decode_attention (viktor/decode_attention.py:11-53) for rollouts that repeat each window G
 * times (scripts/gspo.py:444); no reference counterpart for the sharing itself.
 */
int vk_decode_attention_grouped(const void *q, const void *k_prefix, const void *v_prefix,
                                const int32_t *prefix_len, int64_t stride_pb, int64_t stride_ps, int64_t pre_max,
                                const void *k_suffix, const void *v_suffix, const int32_t *suffix_len,
                                int64_t stride_sb, int64_t stride_ss, int64_t suf_max, void *out, int64_t B,
                                int32_t G, int32_t H, int32_t HKV, int32_t D, void *workspace,
                                int64_t workspace_bytes, void *stream);

int vk_decode_attention_grouped_workspace(int64_t B, int32_t G, int64_t pre_max, int64_t suf_max, int64_t *bytes);

/* How vk_decode_attention_grouped runs at these sizes: query members per workgroup (G, or G / 2 when the
 * groups are split by member) and parts per subgroup (1: one launch; > 1: a merge launch follows). */
int vk_decode_attention_grouped_layout(int64_t B, int32_t G, int64_t pre_max, int64_t suf_max, int32_t *members,
                                       int32_t *parts);

/*
 * Variable-length GQA attention over packed queries (flash_attn_varlen_func semantics, scale 1/sqrt(D)).
 * Sequence i has q_len_i = cu_q[i+1] - cu_q[i] queries (rows cu_q[i].. of q[*, H, D]) and
 * k_len_i = k_lens[i] keys; key j of sequence i is at k + k_off[i] + j * stride_tok (+ hk * D), same for v.
 * causal != 0: query r of sequence i sits at position k_len_i - q_len_i + r and sees keys <= it
 * (bottom-right alignment). out[*, H, D] bf16. lse (NULL: not written): [*, H] fp32, each row's
 * log-sum-exp of its scaled scores in log2 units, log2(sum_j 2^(s_j * log2(e) / sqrt(D))), for the backward.
 * plan: n_blocks entries of (sequence, first query row) built by the host, one per 64-query block
 * (n_blocks > 0 needs n_seq > 0).
 * Built for H = 8, HKV = 2, D = 64.
 * Replaces flash_attn_varlen_func (viktor/fast_decoder.py:68-73) and flash_attn_func (viktor/decoder.py:82-87).
 */
int vk_varlen_attention(const void *q, const void *k, const void *v, const int32_t *cu_q, const int64_t *k_off,
                        const int32_t *k_lens, const int32_t *plan, int32_t n_blocks, int32_t n_seq,
                        int64_t stride_tok, void *out, int32_t causal, int32_t H, int32_t HKV, int32_t D,
                        float *lse, void *stream);

/*
 * vk_varlen_attention with each sequence's first p_lens[i] keys taken from a second buffer: key j < p_lens[i] at
 * k_prefix + p_off[i] + j * p_stride (+ hk * D), key j >= p_lens[i] at k + k_off[i] + (j - p_lens[i]) * stride_tok,
 * same for v; k_lens[i] counts both. The sequences of a GSPO group score one window [prefix | own tokens] each
 * and keep the shared prefix's keys once (scripts/gspo.py:340-353 over the repeated windows of
 * scripts/gspo.py:444, where the reference recomputes the prefix per sample). No reference counterpart of its
 * own: the key order is flash_attn_varlen_func's over the window (viktor/fast_decoder.py:68-73).
 */
int vk_varlen_attention_prefixed(const void *q, const void *k, const void *v, const int32_t *cu_q,
                                 const int64_t *k_off, const int32_t *k_lens, const int32_t *plan, int32_t n_blocks,
                                 int32_t n_seq, int64_t stride_tok, const void *k_prefix, const void *v_prefix,
                                 const int64_t *p_off, const int32_t *p_lens, int64_t p_stride, void *out,
                                 int32_t causal, int32_t H, int32_t HKV, int32_t D, float *lse, void *stream);

/*
 * One decode step's token choice and bookkeeping for B sequences (DecodeEngine._select + state update):
 *   z = (logits[b] + bias) (fp32 logits, or bf16-rounded when h/w are given with round_bf16) ;
 *   greedy (temperature <= 0): nxt = first argmax of z;
 *   sampled: p = softmax(z / temperature) in fp32, nxt = first v with u < sum_{w<=v} p_w, u = uniforms[b * u_stride + col];
 *   sampled with gumbel != 0 (the reference's formula, viktor/engine.py:80-83): nxt = first argmax over v of
 *   z_v / temperature - log(-log(max(u_v, 1e-20))), u_v = uniforms[b * u_stride + col * V + v] (u_stride >= u_cols V);
 *   tail rule: EOS after a tail token; homopolymer rule (homo_stop > 0): run = (nxt == prev && is_homo[nxt]) ? run + 1 : 0,
 *   EOS when run + 1 >= homo_stop; PAD after EOS or PAD.
 *   out[b * out_stride + col] = nxt with col = pos[b] - plen[b]; tok[b] = nxt; pos[b] += 1;
 *   pos32 = pos - base, seqlens = pos - base + 1, rpos32 = pos + rope_off (each optional, NULL to skip), with
 *   base = cache_base[b] (NULL: 0) -- the cache row of position pos when the sequence's cache starts there.
 * Logits come either from `logits` [B, V] fp32 (h and w_head NULL), or are computed here as
 * h[B, d] @ w_head[V, d]^T (bf16 inputs, fp32 accumulation), the fused LM head; with norm_w non-NULL, h is
 * the residual stream and the final RMSNorm (weight norm_w, eps) is applied to it first (rounded to bf16).
 * logp_out (optional): log softmax(z / T or z)[nxt] of the chosen token before the grammar rules, stored to
 * logp_out[b] when logp_stride == 0, else to logp_out[b * logp_stride + col] (the output column, when
 * 0 <= col < out_cols): one row of per-token log-probabilities per sequence over a whole rollout.
 * Replaces greedy_update (viktor/triton_ops.py:172-209), DecodeEngine._select (viktor/engine.py:79-89)
 * and the head + index_copy bookkeeping of DecodeEngine._step (viktor/engine.py:91-116).
 */
int vk_select_update(const float *logits, const void *h, const void *norm_w, float eps, const void *w_head,
                     int32_t d, int32_t round_bf16,
                     const float *bias, const uint8_t *is_tail, const uint8_t *is_homo, int32_t homo_stop,
                     float temperature, const float *uniforms, int64_t u_stride, int64_t u_cols, int32_t gumbel,
                     int64_t *tok,
                     int64_t *run, int64_t *pos, const int64_t *plen, const int64_t *rope_off,
                     const int64_t *cache_base, int64_t *out,
                     int64_t out_stride, int64_t out_cols, int32_t *pos32, int32_t *seqlens, int32_t *rpos32,
                     float *logp_out, int64_t logp_stride, int64_t B, int32_t V, int32_t eos, int32_t pad,
                     void *stream);

/*
 * Decode-step fusions (small M: one row per sequence). Same rounding points as the unfused ops.
 *
 * vk_norm_qkv_rope_cache: h = RMSNorm(x) * norm_w (x [M, K] bf16; or, with tok non-NULL, x = emb[tok] with
 * emb = the `x` argument [vocab, K], and the gathered rows are also stored to x_store; norm_w NULL: h = x,
 * the activation normalised by vk_add_rmsnorm / vk_embed_rmsnorm beforehand), then
 * qkv = bf16(h @ w_qkv^T) and the vk_qkv_rope_cache transform of qkv: q -> q [M, H, 64], k / v -> caches.
 * ss_in (may be NULL): the row sums of squares of x left by vk_linear_residual ([M, K / 32] fp32, K = 512);
 * then 1 / rms comes from them instead of a pass over x.
 * Replaces embed_rmsnorm / add_rmsnorm + linear + qkv_rope_cache (viktor/triton_ops.py:17-108, 149-169;
 * viktor/fast_decoder.py:41-46, 76-90).
 */
int vk_norm_qkv_rope_cache(const void *x, const int64_t *tok, int64_t vocab, void *x_store, const void *norm_w,
                           float eps, const void *w_qkv, const void *q_norm_w, const void *k_norm_w, const void *cos_t,
                           const void *sin_t, int32_t table_dtype, int64_t table_rows, const int32_t *pos,
                           const int32_t *rope_pos, const int32_t *seq, void *q, void *k_cache, void *v_cache,
                           int64_t stride_cb, int64_t stride_cs, int64_t cache_rows, int64_t cache_len, int64_t M,
                           int32_t K, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const float *ss_in,
                           void *stream);

/*
 * vk_linear_residual: x[M, N] = bf16(x + bf16(a[M, K] @ w[N, K]^T)) in place (the o / down projections
 * followed by the residual add of add_rmsnorm, viktor/triton_ops.py:24-27, viktor/fast_decoder.py:51-57).
 * ss_out (may be NULL; N = 512): per-row partial sums of squares of the updated x, one per 32-column
 * block ([M, N / 32] fp32, each block's sum in a fixed order), for the next norm (the norm half of
 * add_rmsnorm, viktor/triton_ops.py:28-40).
 */
int vk_linear_residual(const void *a, const void *w, void *x, int64_t M, int32_t N, int32_t K, float *ss_out,
                       void *stream);

/*
 * vk_norm_linear: y = act(bf16(RMSNorm(x) * norm_w) @ w^T) (norm_w may be NULL: no norm), act = SwiGLU over
 * w = [gate; up] when swiglu != 0 (bf16 out), else identity (bf16 or fp32 out). The mlp norm + gate_up +
 * SwiGLU of a decode step (viktor/triton_ops.py:17-40, 111-146). ss_in as for vk_norm_qkv_rope_cache.
 * The three entry points above take K in {256, 512, 1024, 1536} and N % 4 == 0.
 */
int vk_norm_linear(const void *x, const void *norm_w, float eps, const void *w, void *y, int64_t M, int32_t N,
                   int32_t K, int32_t swiglu, int32_t out_dtype, const float *ss_in, void *stream);

/*
 * GSPO scoring of B sequences of T target tokens (scripts/gspo.py:340-353 and 459-477):
 *   lp[b,t]   = log_softmax(logits[b,t,:])[targets[b,t]]           (fp32; logits bf16 or fp32)
 *   s[b]      = exp(sum_t mask[b,t] (lp[b,t] - old_lp[b,t]) / n_bases[b])
 *   pg[b]     = -min(s A, clamp(s, 1 - eps_lo, 1 + eps_hi) A), A = adv[b]
 *   loss[0]   = inv_n * sum_b pg[b]                                  (fixed summation order)
 *   dlogits[b,t,v] = inv_n * g_b * s_b * mask[b,t] / n_bases[b] * (1[v = y] - softmax(logits[b,t])_v),
 *   g_b = d pg_b / d s_b with torch.minimum / clamp subgradients (ties split evenly, clamp passes at its ends).
 * Targets outside [0, V) are scored as token 0 (the reference clamps PAD targets to 0) and must be masked.
 * dlogits may be NULL (scoring only); old_lp/adv may be NULL when only lp is wanted (then s, pg, loss untouched).
 */
int vk_gspo_score(const void *logits, int32_t logits_dtype, const int64_t *targets, const uint8_t *mask,
                  const float *old_lp, const float *n_bases, const float *adv, float eps_lo, float eps_hi,
                  float inv_n, float *lp, float *s, float *pg, float *loss, float *dlogits, int64_t B, int64_t T,
                  int32_t V, void *stream);

/*
 * Group-normalised advantages of rewards [G, n] (fp32), population std (ddof 0):
 *   mode 0 (reference, scripts/gspo.py:447-450): adv = (r - mean) / max(std, param); live[g] = std > 1e-6
 *   mode 1 (std + eps):                          adv = (r - mean) / (std + param);   live[g] = std > 1e-6
 */
int vk_group_advantage(const float *reward, int64_t groups, int32_t n, int32_t mode, float param, float *adv,
                       uint8_t *live, void *stream);

/* ---- the GSPO update's backward and optimizer step (scripts/gspo.py:477-493) ----------------------- */

/*
 * Backward of causal GQA self-attention over packed sequences (flash_attn_func(causal=True) under autocast,
 * viktor/decoder.py:82-87, differentiated by the update's backward at scripts/gspo.py:477). Sequence i is
 * rows cu[i] .. cu[i+1]-1 of q / out / dout [n_rows, 8, 64] bf16 and of k / v (row j at j * stride_tok,
 * + kv head * 64); query r sees keys <= r. lse [n_rows, 8]: the forward's vk_varlen_attention log-sum-exp
 * (log2 units). q_plan: (sequence, first row) per 64-query block (as vk_varlen_attention's plan); k_plan:
 * (sequence, first key) per 128-key block. dd [n_rows, 8] fp32 scratch (written: sum_d dout * out);
 * dq [n_rows, 8, 64], dk / dv [n_rows, 2, 64] fp32 (written). H = 8, HKV = 2, D = 64.
 */
int vk_attention_backward(const void *q, const void *k, const void *v, const void *out, const void *dout,
                          const float *lse, const int32_t *cu, int32_t n_seq, const int32_t *q_plan, int32_t n_qblocks,
                          const int32_t *k_plan, int32_t n_kblocks, int64_t n_rows, int64_t stride_tok, float *dd,
                          float *dq, float *dk, float *dv, int32_t H, int32_t HKV, int32_t D, void *stream);

/*
 * vk_attention_backward for the shared-prefix layout of a GSPO group's samples (the prefix rows kept once, each
 * sample's token rows after them in the key order of its window). dQ: sequence i's queries first see p_lens[i]
 * prefix keys, rows of k / v from element p_off[i] (row stride stride_tok), then its own rows (query r at key
 * position p_lens[i] + r). dK / dV: k_plan holds n_kblocks entries (sequence, first key of a 128-key block, xr0,
 * xl, slot): xl < 0 takes -xl of the sequence's own query rows from its row xr0 (causal), xl >= 0 the xl query
 * rows from packed row xr0 (of q / out / dout / lse), each of which sees every key of the block; slot < 0 writes
 * dk / dv, slot >= 0 the partial rows [slot][row] of part_k / part_v ([n_slots, n_part, HKV, D] fp32, a caller's
 * workspace whose slots no entry writes for a row hold zeros; those sequences' rows < n_part), which are then
 * summed in slot order into dk / dv rows 0 .. n_part - 1. So dK / dV
 * of the prefix rows sum the gradients of the prefix's own queries and of every sample's token queries, in a
 * fixed order. No reference counterpart of its own: the reference differentiates every sample's full window
 * (scripts/gspo.py:477); these are the same sums, regrouped.
 */
int vk_attention_backward_prefixed(const void *q, const void *k, const void *v, const void *out, const void *dout,
                                   const float *lse, const int32_t *cu, int32_t n_seq, const int32_t *q_plan,
                                   int32_t n_qblocks, const int32_t *k_plan, int32_t n_kblocks, int64_t n_rows,
                                   int64_t stride_tok, const int32_t *p_lens, const int64_t *p_off, float *part_k,
                                   float *part_v, int64_t n_part, int32_t n_slots, float *dd, float *dq, float *dk,
                                   float *dv, int32_t H, int32_t HKV, int32_t D, void *stream);

/*
 * Weight gradient of a linear layer over packed rows: out[Ka, Kb] = a^T b = sum_r a[r, ka] b[r, kb] for a [N, Ka]
 * (the layer's output gradient) and b [N, Kb] (its input), bf16 row-major with row strides lda / ldb (elements,
 * multiples of 8); fp32 accumulation, the N rows split into slices whose fp32 partials are summed in slice order
 * (deterministic), then rounded to bf16 (out_dtype VK_DTYPE_BF16, the autocast matmul output) or kept fp32.
 * Ka % 256 == 0, Kb % 128 == 0; workspace: vk_wgrad_workspace() bytes.
 * Replaces the weight-gradient products of nn.Linear under autocast in the update's backward
 * (viktor/decoder.py:58-59, 114-115, viktor/model.py:35 differentiated by loss.backward(), scripts/gspo.py:477).
 */
int vk_wgrad(const void *a, int64_t lda, const void *b, int64_t ldb, int64_t N, int32_t Ka, int32_t Kb, void *out,
             int32_t out_dtype, void *workspace, int64_t workspace_bytes, void *stream);

int vk_wgrad_workspace(int64_t N, int32_t Ka, int32_t Kb, int64_t *bytes);

/*
 * Epilogue of the per-frame projector's linears (viktor/model.py:35: nn.Linear -> nn.GELU() -> nn.Linear under
 * torch.autocast bf16, applied at viktor/model.py:74): over an fp32 product y [n, d] and an fp32 bias [d],
 * gelu == 0: out = bf16(y + b); gelu != 0: pre = bf16(y + b) and out = bf16(gelu(pre)), the exact erf GELU.
 * d % 8 == 0; 16-byte aligned tensors.
 */
int vk_bias_act(const float *y, const float *bias, void *pre, void *out, int64_t n, int32_t d, int32_t gelu,
                void *stream);

/* Workgroups (= rows of the column-sum partials) vk_act_backward uses for n rows of width d. */
int vk_act_backward_blocks(int64_t n, int32_t d, int32_t *blocks);

/*
 * Backward rows of the projector (the backward of vk_bias_act's forward): gelu != 0: din = bf16(dout gelu'(pre))
 * [n, d] bf16 and part[blocks, d] = per-workgroup column sums of din (the first linear's bias gradient);
 * gelu == 0: part = per-workgroup column sums of dout (the second linear's bias gradient; pre / din unused).
 * blocks from vk_act_backward_blocks; reduce part with vk_colsum. d % 8 == 0, d <= 2048.
 */
int vk_act_backward(const void *pre, const void *dout, void *din, float *part, int32_t blocks, int64_t n, int32_t d,
                    int32_t gelu, void *stream);

/* Bytes of workspace vk_embed_grad needs for n rows, V token ids and width d. */
int vk_embed_grad_workspace(int64_t n, int32_t V, int32_t d, int64_t *bytes);

/*
 * Token-embedding gradient (the backward of nn.Embedding, viktor/decoder.py:127, gathered at viktor/model.py:77):
 * out[v, :] = sum of d_rows[r, :] over the rows r with tokens[r] == v, fp32 [V, d], from d_rows [n, d] bf16 or fp32
 * per d_dtype (row stride ld elements) and tokens [n] int64. Row slices summed in a fixed order (deterministic, no atomics); ids
 * outside [0, V) add nothing. d % 8 == 0; workspace: vk_embed_grad_workspace() bytes.
 */
int vk_embed_grad(const void *d_rows, int32_t d_dtype, int64_t ld, const int64_t *tokens, int64_t n, int32_t V, int32_t d,
                  float *out, void *workspace, int64_t workspace_bytes, void *stream);

/* Workgroups (= rows of the weight-gradient partials) vk_rmsnorm_backward uses for n rows. */
int vk_rmsnorm_backward_blocks(int64_t n, int32_t *blocks);

/*
 * RMSNorm backward (nn.RMSNorm of the decoder blocks, viktor/decoder.py:110-124), d = 512: given x [n, d] and
 * weight w [d] (both bf16, or both fp32: the autocast forward's residual stream and master weights) and dy [n, d]
 * (bf16 or fp32 per dy_dtype): dx = r w dy - x r^3 mean(w dy x)
 * (+ dres when not NULL: the residual stream's incoming gradient; dx may alias dres), fp32, and when dx_bf16 is
 * not NULL also dx rounded to bf16 (nearest even) there: the operand the next products of the backward take;
 * dw_part [vk_rmsnorm_backward_blocks(n), d] fp32: per-workgroup sums of dy x r (reduce with vk_colsum).
 */
int vk_rmsnorm_backward(const void *x, int32_t x_dtype, const void *w, int32_t w_dtype, const void *dy,
                        int32_t dy_dtype, const float *dres, float *dx, void *dx_bf16, float *dw_part, int64_t n,
                        int32_t d, float eps, void *stream);

/* out[c] = sum_r part[r, c] (+ out[c] when accumulate), fixed order. */
int vk_colsum(const float *part, float *out, int32_t rows, int32_t cols, int32_t accumulate, void *stream);

/*
 * Backward of the QK-norm + RoPE stage (viktor/decoder.py:62-66 with apply_rope, viktor/encoder.py:36-40):
 * qkv [n, (H + 2 HKV) 64] bf16 (the projection output), dq [n, H, 64] / dk / dv [n, HKV, 64] fp32 (the
 * attention's input gradients), RoPE rows rope_pos [n] of cos/sin [table_rows, 32]. Writes dqkv [n, (H + 2 HKV) 64]
 * bf16 (q / k heads through the rotation and the 64-wide norm, v heads copied) and dw_part
 * [vk_rmsnorm_backward_blocks(n), 128] fp32 (q-norm weight partials 0..63, k-norm 64..127). D = 64. Norm weights
 * bf16 or fp32 per norm_w_dtype. Every pointer 16-byte aligned.
 */
int vk_qknorm_rope_backward(const void *qkv, const void *q_norm_w, const void *k_norm_w, int32_t norm_w_dtype,
                            const void *cos_t, const void *sin_t, int32_t table_dtype, int64_t table_rows, const int32_t *rope_pos,
                            const float *dq, const float *dk, const float *dv, void *dqkv, float *dw_part, int64_t n,
                            int32_t H, int32_t HKV, int32_t D, float eps, void *stream);

/* SwiGLU backward (F.silu(gate) * up, viktor/decoder.py:127): gu [n, 2F] (gate | up) bf16, dout [n, F] bf16
 * -> dgu [n, 2F] bf16. F % 8 == 0. */
int vk_swiglu_backward(const void *gu, const void *dout, void *dgu, int64_t n, int32_t F, void *stream);

/*
 * Global gradient norm and clip coefficient of nn.utils.clip_grad_norm_ (scripts/gspo.py:492) over the flat
 * fp32 gradient g [n]: norm_out[0] = ||g||_2, norm_out[1] = min(1, max_norm / (||g|| + 1e-6)), on the device.
 * partials: n_partials floats of scratch.
 */
int vk_grad_norm_clip(const float *g, int64_t n, float max_norm, float *partials, int32_t n_partials,
                      float *norm_out, void *stream);

/*
 * AdamW step (torch.optim.AdamW, scripts/gspo.py:368, 493) over flat fp32 params p, grads g (scaled by
 * coef[1] when coef is not NULL: the clip coefficient of vk_grad_norm_clip) and moments m, v:
 * m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g^2, p = p (1 - lr wd) - lr / (1 - b1^step) m / (sqrt(v / (1 - b2^step)) + eps).
 */
int vk_adamw(float *p, const float *g, float *m, float *v, int64_t n, const float *coef, float lr, float b1, float b2,
             float eps, float wd, int64_t step, void *stream);

/*
 * The GSPO reward on the device: strict identity of call c (bases calls[call_off[c] ..], call_len[c] of them)
 * against label r = ref_of_call[c] (refs[ref_off[r] ..], ref_len[r] bases, scored[ref_off[r] ..] its mask of
 * counted bases) -- scripts/gspo.py:86-89 with ref_errors (scripts/train.py:170-188):
 *   empty label: 1 if len(call) <= empty_max else empty_max / len(call);
 *   else 1 - (errors of a global alignment path on scored label bases) / max(len(call), len(label)),
 * a mismatch or deletion counted at its label base, an insertion at the label base before it. The path is the
 * traceback that prefers diagonal, then deletion, then insertion at each cell (edlib's own order is not
 * available; the edit distance, and the count when every base is scored, do not depend on it).
 * Bases are any byte codes compared for equality. Writes reward, edit_distance and scored_errors [n_calls].
 * max_ref_len / max_call_len: the longest label / call (at most 4096 / 8192).
 */
int vk_strict_identity(const uint8_t *calls, const int64_t *call_off, const int32_t *call_len, const uint8_t *refs,
                       const int64_t *ref_off, const int32_t *ref_len, const uint8_t *scored, const int32_t *ref_of_call,
                       int32_t n_calls, int32_t n_refs, int32_t max_ref_len, int32_t max_call_len, float empty_max,
                       float *reward, int32_t *edit_distance, int32_t *scored_errors, void *stream);

/*
 * The encoder (frames producer): the Dorado SUP conv stack + sliding-window DeepNorm transformer of
 * viktor/encoder.py:43-192, which the reference runs on koi (viktor/csrc/koi_tx.cpp:253-414: koi_vcs_tx_cnn,
 * koi_qkv_rotary + koi_vcs_attn, koi_linear, koi_rmsnorm_residual, koi_mm_swiglu).
 *
 * Padded chunk layout of a convolution's activations: channels-last [rows, C] bf16, chunk c's data rows at
 * [start[c], start[c] + len[c]), zero margin rows between chunks; the input row of output row g is
 * stride * g - pad for every row (margins scale by the strides), so the zero margins are each chunk's
 * Conv1d padding. hint[i] = the chunk of output row 256 i (the last c with start[c] <= 256 i, else 0),
 * ceil(rows / 256) entries.
 *
 * First convolution (C_in = 1; viktor/encoder.py:43-49 and the first koi_vcs_tx_cnn call, koi_tx.cpp:296-315):
 * out[g, co] = bf16(silu(bf16(b[co] + sum_k w[co, k] signal[sig_off[c] + stride t - pad + k]))) for data row
 * g = start[c] + t (samples outside the chunk read as 0), zeros for margin rows; signal, w [C, winlen], b fp32;
 * out [rows, C] bf16 (C % 8 == 0, C <= 512, winlen <= 32, C * winlen <= 4096).
 */
int vk_encoder_conv_first(const float *signal, const int64_t *sig_off, const int32_t *start, const int32_t *hint,
                          const int32_t *len, int32_t n_chunks, int64_t rows, const float *w, const float *b, int32_t C,
                          int32_t winlen, int32_t stride, int32_t pad, void *out, void *stream);

/*
 * Later convolutions (viktor/encoder.py:43-49; koi_vcs_tx_cnn, koi_tx.cpp:296-315) as one strided GEMM:
 * out[dst(g), n] = bf16(silu(bf16(sum_k a[g lda + k] w[n, k] + bias[n]))), k = tap * C_in + channel,
 * K = winlen * C_in (% 32), N = C_out (% 64), lda = stride * C_in; a points at input row -pad of the padded
 * layout (the buffer holds guard rows around it). compact = 0: dst(g) = g, margin rows written as zeros;
 * compact = 1: only data rows, dst(g) = dst0[c] + t (the transformer's [frames, C] input).
 */
int vk_encoder_conv(const void *a, int64_t lda, const void *w, int32_t K, int32_t N, const float *bias,
                    const int32_t *start, const int32_t *hint, const int32_t *len, const int32_t *dst0,
                    int32_t n_chunks, int64_t rows, int32_t compact, void *out, int64_t ldo, void *stream);

/*
 * Sliding-window self-attention with rotary embedding (viktor/encoder.py:71-84: Wqkv output
 * .view(N, T, 3, H, D), apply_rope on q and k at positions 0 .. T - 1 of each chunk, flash_attn_func with
 * window_size = (left, right) or SDPA with the band mask of encoder.py:64-69; koi_qkv_rotary + koi_vcs_attn,
 * koi_tx.cpp:395-400). qkv [rows, ld] bf16 (q heads, k heads, v heads of 64), chunk c = rows cu[c] ..
 * cu[c + 1] - 1; plan = n_blocks pairs (chunk, first query row of a 128-row block); cos_t / sin_t fp32
 * [table_len, 32] (rope_tables), or both NULL when q and k are already rotated (vk_linear_qkv_rope);
 * out [rows, ldo] bf16 (heads concatenated). D must be 64.
 */
int vk_window_attention(const void *qkv, int64_t ld, const int32_t *cu, const int32_t *plan, int32_t n_blocks,
                        int32_t n_chunks, int32_t max_len, int32_t H, int32_t D, const float *cos_t,
                        const float *sin_t, int32_t table_len, int32_t left, int32_t right, void *out, int64_t ldo,
                        void *stream);

/*
 * DeepNorm residual + RMSNorm, in place (viktor/encoder.py:106-108: norm(sublayer(x) + alpha x);
 * koi_rmsnorm_residual, koi_tx.cpp:404-405, 412-413): x = bf16(rmsnorm(bf16(bf16(y + bias) + bf16(alpha x))) * w) with
 * y fp32 [n, d] (a product before rounding), bias fp32 [d] or NULL, w fp32 [d]; d must be 512.
 */
int vk_deepnorm_rmsnorm(const float *y, const float *bias, void *x, float alpha, const float *w, float eps, int64_t n,
                        int32_t d, void *stream);

/*
 * Row-deterministic GEMM y = x w^T (x [M, K], w [N, K] bf16; K % 64 == 0, N % 8 == 0, 16-byte aligned
 * pointers): every row is computed by the same
 * tile code whatever M is, so a chunk's frames do not depend on its batch (the koi VCS property checked at
 * tests/gpu_check.py:103-105). epilogue 0: bf16 out; 1: fp32 out; 2: SwiGLU, w holds 2N rows and
 * y[:, n] = bf16(bf16(silu(bf16(x w[n]))) * bf16(x w[N + n])) (koi_linear / koi_mm_swiglu, koi_tx.cpp:401-411).
 */
int vk_gemm_rows(const void *x, const void *w, void *y, int64_t M, int32_t N, int32_t K, int32_t epilogue,
                 void *stream);

/*
 * Timing support, no counterpart in the reference (its benchmark times whole replays): vk_timestamp stores the
 * device's constant-rate wall clock, read when its one-thread kernel runs, to stamps[index] (uint64, device
 * memory). Launched on a capturing stream it becomes a graph node, so a pair around another node times that node
 * inside the captured graph (less the dispatch gap a back-to-back pair measures). vk_timestamp_rate_khz: the
 * clock's rate.
 */
int vk_timestamp(uint64_t *stamps, int64_t index, void *stream);
int vk_timestamp_rate_khz(int64_t *khz);

#ifdef __cplusplus
}
#endif

#endif /* VIKTOR_HIP_H */
