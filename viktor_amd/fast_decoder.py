"""Inference forward of the Decoder on the gfx950 HIP kernels (same weights as decoder.Decoder).

Tokens are packed [n_tokens, d]: a prefill packs the prefixes of many variable-length sequences, a
decode step is one token per sequence. Per layer (reference: viktor/fast_decoder.py:33-60):
  qkv GEMM -> QK-norm + RoPE + KV-cache write -> attention -> o GEMM + residual add + RMSNorm
  -> gate_up GEMM with SwiGLU epilogue -> down GEMM + residual add + next RMSNorm.
Every GEMM, norm and attention runs on libviktor_hip.so; there is no other backend.
Prefill attention reads K/V straight from the KV cache when one is given (packed k/v otherwise); the
last layer of a prefill can keep only some rows of each sequence (the BOS row for the engine, the
response rows for teacher-forced scoring), which then attend to their whole sequence.
"""

from collections import OrderedDict

import numpy as np
import torch

from . import hip_ops as ops
from ._lib import HipLibraryError, require_device

BF16 = torch.bfloat16


def _require(cond, msg):
    if not cond:
        raise AssertionError(msg)


class PrefillPlan:
    """Host-side layout of one packed prefill (built from Python ints; no device reads).

    seq_lens[j]: tokens of sequence j (packed back to back); rows[j]: its KV-cache row (None without a
    cache); keep[j]: rows of sequence j kept by the last layer (its final keep[j] positions), None to keep
    all. last_rows[j] (instead of keep): the one packed row of sequence j that finishes the last layer, any of
    its rows, attending to the whole sequence (the reference's last-layer call, viktor/fast_decoder.py:64-69:
    flash_attn_varlen_func(q[last_indices], ..., max_seqlen_q=1, causal=False)). Construction uploads the few
    small index tensors once; engines cache plans per layout."""

    def __init__(self, seq_lens, device, rows=None, keep=None, cache=None, last_rows=None):
        seq_lens = [int(n) for n in seq_lens]
        _require(all(n > 0 for n in seq_lens), "PrefillPlan: empty sequence")
        self.seq_lens = seq_lens
        self.n_seq = len(seq_lens)
        cu = [0]
        for n in seq_lens:
            cu.append(cu[-1] + n)
        self.cu = cu
        self.total = cu[-1]
        self.max_len = max(seq_lens) if seq_lens else 0
        self.rows = None if rows is None else [int(r) for r in rows]
        self.device = device
        if cache is not None:
            _require(self.rows is not None and len(self.rows) == self.n_seq, "PrefillPlan: rows for the cache")
            sb, ss = cache.k.stride(1), cache.k.stride(2)
            k_off = [r * sb for r in self.rows]
            self.stride_tok = ss
        else:
            hkv_d = None
            k_off = None
            self.stride_tok = None
        self.from_cache = cache is not None
        self._k_off = k_off
        self.full = None if cache is None else ops.AttentionPlan(seq_lens, seq_lens, k_off, device, causal=True)
        self.keep = None if keep is None else [int(k) for k in keep]
        self.last = None
        self.last_idx = None
        self.bos_lengths = None
        self.last_causal = True
        if last_rows is not None:
            _require(keep is None, "PrefillPlan: keep and last_rows are exclusive")
            lr = [int(r) for r in last_rows]
            _require(len(lr) == self.n_seq and all(cu[j] <= r < cu[j + 1] for j, r in enumerate(lr)),
                     "PrefillPlan: last_rows must name one row inside each sequence")
            self.keep = [1] * self.n_seq
            self.last_causal = False  # the one query attends to every key of its sequence
            self.last_idx = torch.tensor(lr, dtype=torch.int64).to(device)
            if cache is not None:
                self.last = ops.AttentionPlan(self.keep, seq_lens, k_off, device, causal=False)
                if all(r == self.rows[0] + j for j, r in enumerate(self.rows)):
                    # one query per sequence over its whole cached row: the single-query decode kernel
                    self.bos_lengths = torch.tensor(seq_lens, dtype=torch.int32).to(device)
        elif self.keep is not None:
            _require(len(self.keep) == self.n_seq and all(0 < k <= n for k, n in zip(self.keep, seq_lens)),
                     "PrefillPlan: keep counts")
            # rows cu[j + 1] - keep[j] .. cu[j + 1] - 1 of every sequence j, in order
            kp = np.asarray(self.keep, dtype=np.int64)
            idx = np.repeat(np.asarray(cu[1:], dtype=np.int64) - kp, kp) + (
                np.arange(int(kp.sum()), dtype=np.int64) - np.repeat(np.cumsum(kp) - kp, kp))
            self.last_idx = torch.from_numpy(idx).to(device)
            if cache is not None:
                self.last = ops.AttentionPlan(self.keep, seq_lens, k_off, device, causal=True)
                contiguous_rows = all(r == self.rows[0] + j for j, r in enumerate(self.rows))
                if all(k == 1 for k in self.keep) and contiguous_rows:
                    # one query per sequence (its last position): single-query decode kernel on the cache
                    self.bos_lengths = torch.tensor(seq_lens, dtype=torch.int32).to(device)

    def packed_plans(self, hkv_d):
        """Attention plans over packed k/v rows [total, HKV, D] (no cache); built once per hkv_d."""
        memo = self.__dict__.setdefault("_packed", {})
        if hkv_d not in memo:
            k_off = [c * hkv_d for c in self.cu[:-1]]
            full = ops.AttentionPlan(self.seq_lens, self.seq_lens, k_off, self.device, causal=True)
            last = None if self.keep is None else ops.AttentionPlan(self.keep, self.seq_lens, k_off, self.device,
                                                                    causal=self.last_causal)
            memo[hkv_d] = (full, last)
        return memo[hkv_d]


class SharedPrefixPlan:
    """Host-side layout of a teacher-forced forward over groups of G sequences that share their prefix rows
    (a GSPO rollout's repeated windows, scripts/gspo.py:444): group g's pre_lens[g] prefix rows are packed once
    (back to back, as a PrefillPlan), and every member b = g G + m has T token rows (packed at b T). A token row
    attends, in the key order of its window [prefix | tokens], to its group's packed prefix keys and then to its
    member's own token keys (vk_varlen_attention_prefixed), so no prefix key is copied per member."""

    def __init__(self, pre_lens, group_size, T, hkv_d, device):
        pre_lens = [int(p) for p in pre_lens]
        G, T = int(group_size), int(T)
        _require(G >= 1 and T > 0 and len(pre_lens) > 0 and all(p > 0 for p in pre_lens), "SharedPrefixPlan: sizes")
        self.pre_lens, self.G, self.T = pre_lens, G, T
        self.n_groups = len(pre_lens)
        self.B = self.n_groups * G
        self.pre = PrefillPlan(pre_lens, device)
        self.pre_full, _ = self.pre.packed_plans(hkv_d)
        member_pre = np.repeat(np.asarray(pre_lens, dtype=np.int64), G)
        cu = np.asarray(self.pre.cu[:-1], dtype=np.int64)
        self.tok = ops.AttentionPlan([T] * self.B, (member_pre + T).tolist(), [b * T * hkv_d for b in range(self.B)],
                                     device, causal=True, p_lens=member_pre.tolist(),
                                     p_off=(np.repeat(cu, G) * hkv_d).tolist())
        t = np.arange(T, dtype=np.int64)
        # a token row's position in its window (pre_len + t) and the prefix rows' (0 .. pre_len - 1)
        self.pos_tok = torch.from_numpy((member_pre[:, None] + t[None, :]).reshape(-1).astype(np.int32)).to(device)
        self.pos_pre = torch.from_numpy(np.concatenate([np.arange(p, dtype=np.int32) for p in pre_lens])).to(device)


class FastDecoder:
    """Packed-token forward of a Decoder on the HIP kernels (reference: viktor/fast_decoder.py:17-90)."""

    def __init__(self, dec, attention_backend="auto"):
        cfg = dec.cfg
        if attention_backend not in ("auto", "hip", "triton"):
            raise ValueError(f"unknown decode attention backend: {attention_backend}")
        if (cfg.n_heads, cfg.n_kv_heads, cfg.head_dim) != (8, 2, 64):
            raise ValueError("the HIP attention kernels are built for 8 query heads, 2 KV heads, head_dim 64 "
                             f"(got {cfg.n_heads}/{cfg.n_kv_heads}/{cfg.head_dim})")
        _require(cfg.d_model % 64 == 0 and cfg.ffn_dim % 32 == 0, "FastDecoder: d_model % 64, ffn_dim % 32")
        self.dec, self.cfg = dec, cfg
        self.attention_backend = "hip"
        self._wcache = {}
        self._plans = {}
        self._layouts = OrderedDict()
        self.decode_workspace = None
        # optional attn_marks(layer, k): called right before (k = 0) and after (k = 1) each decode step's attention
        # launch, on the launching stream -- the benchmark records timing events there, inside the captured step
        self.attn_marks = None

    # weights: bf16 views of the module's parameters (in place when the module is bf16, so weight syncs
    # into it stay visible to captured graphs; converted copies, refreshed on change, otherwise)
    def w(self, p):
        if p.dtype == BF16 and p.is_contiguous():
            return p
        key = id(p)
        ver = (p.data_ptr(), p._version)
        hit = self._wcache.get(key)
        if hit is not None and hit[0] == ver:
            return hit[1]
        conv = p.detach().to(BF16).contiguous()
        self._wcache[key] = (ver, conv)
        return conv

    def w32(self, p):
        """fp32 contiguous view of a parameter (the module's own tensor when it is fp32; a converted copy,
        refreshed on change, otherwise): the norm weights autocast leaves in fp32."""
        if p.dtype == torch.float32 and p.is_contiguous():
            return p
        key = ("f32", id(p))
        ver = (p.data_ptr(), p._version)
        hit = self._wcache.get(key)
        if hit is not None and hit[0] == ver:
            return hit[1]
        conv = p.detach().float().contiguous()
        self._wcache[key] = (ver, conv)
        return conv

    def _tables(self):
        return self.dec.cos, self.dec.sin

    def layout(self, key, build, cap=4):
        """The host-built layout of a packed batch (plans and their small index tensors on the device) for key,
        built by build() on a miss; the cap most recent are kept. A batch of a layout seen before then starts
        without host work or host-to-device copies (each copy from pageable memory waits for the stream)."""
        hit = self._layouts.get(key)
        if hit is None:
            hit = build()
            self._layouts[key] = hit
            while len(self._layouts) > cap:
                self._layouts.popitem(last=False)
        else:
            self._layouts.move_to_end(key)
        return hit

    def teacher_forced(self, x, pos, plan, rope_pos=None):
        """The teacher-forced causal forward of packed windows with the rounding points of the reference's
        scoring path, Basecaller.logits under torch.autocast bf16 over fp32 master weights (scripts/gspo.py:345-347,
        viktor/model.py:55-60, viktor/decoder.py:63-67, 82-87, 117-120, 144):
          * the residual stream x [n, d] is fp32 (updated in place); every sublayer output is a bf16 product
            added to it in fp32 (vk_linear_residual_big on an fp32 stream);
          * each RMSNorm runs in fp32 with fp32 weights and is rounded once, to the bf16 operand of the next
            product (vk_rmsnorm_f32, vk_rmsnorm_apply_ss on fp32);
          * the GEMM weights are the parameters cast to bf16; the QK-norm keeps fp32 weights and returns
            bf16(x / rms * w) for a bf16 head, the rotation runs in fp32 with fp32 tables, rounded to bf16
            (vk_linear_qkv_rope with fp32 norm weights);
          * attention as flash-attention: bf16 q / k / v, fp32 scores, bf16 probabilities in the PV product.
        pos [n] int32: each row's position in its window (the rotary row unless rope_pos is given); plan: a
        PrefillPlan without a cache (its keep rows finish the last layer). Returns the final-normed hidden state
        of the kept rows (all rows without keep), bf16, the operand of the LM head."""
        require_device(x, "FastDecoder.teacher_forced")
        cfg, layers, W, F = self.cfg, self.dec.layers, self.w, self.w32
        _require(x.dtype == torch.float32 and x.is_contiguous() and x.shape == (plan.total, cfg.d_model),
                 "teacher_forced: x fp32 [plan rows, d]")
        _require(not plan.from_cache, "teacher_forced: a plan without a cache")
        eps = cfg.norm_eps
        H, HKV, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        cos, sin = (F(t) for t in self._tables())
        full, lastp = plan.packed_plans(HKV * D)
        n_layers = len(layers)
        h = ops.rmsnorm_f32(x, F(layers[0].attn_norm.weight), eps)
        for i, blk in enumerate(layers):
            a = blk.attn
            q, k, v = ops.linear_qkv_rope(h, W(a.qkv_proj.weight), F(a.q_norm.weight), F(a.k_norm.weight), cos, sin,
                                          pos, None, None, None, eps, H, HKV, D, return_kv=True, rope_pos=rope_pos)
            last = plan.last_idx is not None and i == n_layers - 1
            if last:  # only the kept rows finish the last layer; they attend to every key of their window
                x = x[plan.last_idx]
                q = q[plan.last_idx]
            o = ops.varlen_attention(q, k, v, lastp if last else full, stride_tok=k.stride(0))
            w_next = layers[i + 1].attn_norm.weight if i + 1 < n_layers else self.dec.norm.weight
            h = self._tf_block(x, o, blk, w_next)
        return h

    def _tf_block(self, x, o, blk, w_next):
        """The rest of a teacher-forced layer after its attention output o: x += o Wo^T (fp32 stream, bf16
        product), the MLP norm, gate_up with SwiGLU, x += down, and the next norm (w_next), which it returns."""
        W, F, eps = self.w, self.w32, self.cfg.norm_eps
        ss = ops.linear_residual_big(o.reshape(x.shape[0], -1), W(blk.attn.o_proj.weight), x)
        h = ops.rmsnorm_apply(x, ss, F(blk.mlp_norm.weight), eps)
        g = ops.linear(h, W(blk.gate_up.weight), swiglu=True)
        ss = ops.linear_residual_big(g, W(blk.down.weight), x)
        return ops.rmsnorm_apply(x, ss, F(w_next), eps)

    def teacher_forced_shared(self, x_pre, x_tok, plan, rope_pre=None, rope_tok=None):
        """teacher_forced over groups of sequences that share their prefix (plan: a SharedPrefixPlan): x_pre
        [n_pre, d] fp32 holds each group's prefix rows once, x_tok [B T, d] fp32 every member's token rows. The
        prefix rows run the layers once per group (the last layer only to its K / V), and the token rows attend to
        their group's prefix keys, then to their member's own (vk_varlen_attention_prefixed). Every step of a row is that of teacher_forced over the unshared windows
        [prefix | tokens]: the products and norms are row by row, and a token row's attention meets the same keys
        in the same order. So the token rows' hidden states are the unshared forward's, bit for bit wherever both
        forwards run a product on the same kernel (each product with at least 4096 rows in both). Returns the
        final-normed hidden of the token rows [B T, d] bf16. rope_pre / rope_tok [n_pre] / [B T] int32: the
        rotary rows when they are not the positions (prefix row j at j, token t of a member at pre_len + t)."""
        require_device(x_tok, "FastDecoder.teacher_forced_shared")
        cfg, layers, W, F = self.cfg, self.dec.layers, self.w, self.w32
        d = cfg.d_model
        _require(x_pre.dtype == torch.float32 and x_pre.is_contiguous() and x_pre.shape == (plan.pre.total, d),
                 "teacher_forced_shared: x_pre fp32 [prefix rows, d]")
        _require(x_tok.dtype == torch.float32 and x_tok.is_contiguous() and x_tok.shape == (plan.B * plan.T, d),
                 "teacher_forced_shared: x_tok fp32 [B T, d]")
        eps = cfg.norm_eps
        H, HKV, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        cos, sin = (F(t) for t in self._tables())
        n_layers = len(layers)
        w0 = F(layers[0].attn_norm.weight)
        hp = ops.rmsnorm_f32(x_pre, w0, eps)
        ht = ops.rmsnorm_f32(x_tok, w0, eps)
        for i, blk in enumerate(layers):
            a = blk.attn
            wqkv, qn, kn = W(a.qkv_proj.weight), F(a.q_norm.weight), F(a.k_norm.weight)
            qp, kp, vp = ops.linear_qkv_rope(hp, wqkv, qn, kn, cos, sin, plan.pos_pre, None, None, None, eps, H, HKV,
                                             D, return_kv=True, rope_pos=rope_pre)
            qt, kt, vt = ops.linear_qkv_rope(ht, wqkv, qn, kn, cos, sin, plan.pos_tok, None, None, None, eps, H, HKV,
                                             D, return_kv=True, rope_pos=rope_tok)
            w_next = layers[i + 1].attn_norm.weight if i + 1 < n_layers else self.dec.norm.weight
            if i + 1 < n_layers:  # the prefix rows feed the next layer's prefix keys
                op = ops.varlen_attention(qp, kp, vp, plan.pre_full, stride_tok=kp.stride(0))
                hp = self._tf_block(x_pre, op, blk, w_next)
            ot = ops.varlen_attention(qt, kt, vt, plan.tok, stride_tok=kt.stride(0), prefix=(kp, vp))
            ht = self._tf_block(x_tok, ot, blk, w_next)
        return ht

    def _layers(self, x, pos, seq, cache, attend, return_kv, last_idx=None, rope_pos=None, h=None):
        """x [n, d] residual stream (updated in place); h: its first attention norm when already computed.
        Returns the final-normed hidden [n or len(last_idx), d]."""
        cfg, layers, W = self.cfg, self.dec.layers, self.w
        eps = cfg.norm_eps
        cos, sin = self._tables()
        if h is None:
            h = ops.add_rmsnorm(x, W(layers[0].attn_norm.weight), eps)
        n_layers = len(layers)
        for i, blk in enumerate(layers):
            a = blk.attn
            kc = cache.k[i] if cache is not None else None
            vc = cache.v[i] if cache is not None else None
            if h.shape[0] >= 4096:  # large packed batches: QK-norm + RoPE + cache write in the product's epilogue
                r = ops.linear_qkv_rope(h, W(a.qkv_proj.weight), W(a.q_norm.weight), W(a.k_norm.weight), cos, sin, pos,
                                        seq, kc, vc, eps, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                        return_kv=return_kv, rope_pos=rope_pos)
            else:
                qkv = ops.linear(h, W(a.qkv_proj.weight))
                r = ops.qkv_rope_cache(qkv, W(a.q_norm.weight), W(a.k_norm.weight), cos, sin, pos, seq, kc, vc, eps,
                                       cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, return_kv=return_kv,
                                       rope_pos=rope_pos)
            last = last_idx is not None and i == n_layers - 1
            if last:
                # rows without a consumer are dropped: all K/V are kept, only the kept rows finish the layer
                x = x[last_idx]
                if return_kv:
                    q, k, v = r
                    r = (q[last_idx], k, v)
                else:
                    r = r[last_idx]
            o = attend(i, r, last)
            h = self._residual_norm(x, o.reshape(x.shape[0], -1), W(a.o_proj.weight), W(blk.mlp_norm.weight))
            g = ops.linear(h, W(blk.gate_up.weight), swiglu=True)
            w_next = layers[i + 1].attn_norm.weight if i + 1 < n_layers else self.dec.norm.weight
            h = self._residual_norm(x, g, W(blk.down.weight), W(w_next))
        return h

    def _residual_norm(self, x, a, w, norm_w):
        """x += a @ w^T in place, then RMSNorm(x) * norm_w (viktor/fast_decoder.py:56-58 with
        viktor/triton_ops.py:34-40). Large batches add the residual in the product's epilogue, which hands the
        row sums of squares to the norm; the bf16 product never goes through HBM."""
        eps = self.cfg.norm_eps
        if x.shape[0] >= 4096 and x.shape[1] % 128 == 0 and a.shape[1] % 64 == 0:
            return ops.rmsnorm_apply(x, ops.linear_residual_big(a, w, x), norm_w, eps)
        return ops.add_rmsnorm(x, norm_w, eps, delta=ops.linear(a, w))

    def prefill(self, x, pos, seq, cu_seqlens, max_seqlen, cache, last_indices=None, cu_queries=None, rope_pos=None,
                plan=None):
        """x [n, d] packed prefix embeddings of several sequences; pos/seq [n] int32 (position, cache row);
        cu_seqlens [b+1] int32. Fills the cache rows of those sequences. Returns hidden [n, d], or the kept
        rows when last_indices and cu_queries are given together (e.g. [b, d] at each sequence's last
        position). plan: a PrefillPlan of this layout (built here from cu_seqlens / seq / cu_queries
        otherwise, which reads them back to the host). With last_indices, the last layer finishes row
        last_indices[j] of each sequence j (any of its rows: the reference's engine passes the BOS rows), which
        attends to the whole sequence, as the reference's last-layer attention (non-causal, one query per
        sequence: cu_queries must be 0, 1, .., n; anything else raises ValueError). Reference:
        viktor/fast_decoder.py:62-74."""
        require_device(x, "FastDecoder.prefill")
        _require((last_indices is None) == (cu_queries is None), "prefill: last_indices and cu_queries go together")
        if plan is None:
            cu = [int(c) for c in cu_seqlens.tolist()]
            lens = [b - a for a, b in zip(cu[:-1], cu[1:])]
            last_rows = None
            if cu_queries is not None:
                cq = [int(c) for c in cu_queries.tolist()]
                if cq != list(range(len(lens) + 1)):
                    raise ValueError("prefill: cu_queries must hold one query per sequence (0, 1, .., n), as the "
                                     "reference's last-layer call reads it with max_seqlen_q = 1")
                last_rows = [int(r) for r in last_indices.tolist()]
                if len(last_rows) != len(lens) or not all(cu[j] <= r < cu[j + 1] for j, r in enumerate(last_rows)):
                    raise ValueError("prefill: last_indices must name one row inside each sequence")
            rows = None
            if cache is not None:
                seq_h = seq.tolist()
                rows = [int(seq_h[c]) for c in cu[:-1]]
            plan = PrefillPlan(lens, x.device, rows=rows, cache=cache, last_rows=last_rows)
        _require(x.shape[0] == plan.total, "prefill: x rows != plan tokens")
        x = x.to(BF16).contiguous() if x.dtype != BF16 else x
        if cache is not None:
            full, lastp = plan.full, plan.last
            return_kv = False
        else:
            full, lastp = plan.packed_plans(self.cfg.n_kv_heads * self.cfg.head_dim)
            return_kv = True

        def attend(i, r, last):
            if return_kv:
                q, k, v = r
            else:
                q = r
                k, v = cache.k[i], cache.v[i]
            if last and plan.bos_lengths is not None:
                r0 = plan.rows[0]
                return ops.decode_attention(q, k[r0:r0 + plan.n_seq], v[r0:r0 + plan.n_seq], plan.bos_lengths)
            p = lastp if last else full
            if return_kv:
                return ops.varlen_attention(q, k, v, p, stride_tok=k.stride(0))
            return ops.varlen_attention(q, k, v, p, stride_tok=k.stride(1))

        return self._layers(x, pos, seq, cache, attend, return_kv, last_idx=plan.last_idx, rope_pos=rope_pos)

    def decode(self, x, pos, seq, cache_seqlens, cache, rope_pos=None, tok=None):
        """One token per sequence: x [B, d] (or tok [B] token ids with x None: the embedding is looked up in
        the first layer's kernel), pos/seq [B] int32 (sequence b's token goes to cache row seq[b], position
        pos[b], and attends to that row's positions < cache_seqlens[b]), cache_seqlens = pos + 1 (int32).
        Returns the final-normed hidden [B, d]. Reference: viktor/fast_decoder.py:76-90."""
        xr = self.decode_residual(pos, seq, cache_seqlens, cache, rope_pos=rope_pos, tok=tok, x=x)
        return ops.add_rmsnorm(xr, self.w(self.dec.norm.weight), self.cfg.norm_eps)

    def decode_residual(self, pos, seq, cache_seqlens, cache, rope_pos=None, tok=None, x=None, prefix=None):
        """The decoder layers of one decode step on the small-M kernels, five launches per layer:
        norm_qkv_rope_cache (attn norm + qkv GEMM + QK-norm + RoPE + cache write; in layer 0 with the
        token-embedding gather in its prologue), decode_attention, linear_residual
        (o proj + residual add), norm_linear (mlp norm + gate_up + SwiGLU), linear_residual (down proj +
        residual add). The residual GEMMs leave the row sums of squares of x (per 32-column block), so the
        norms inside the next GEMMs need no pass of their own over x.
        Returns the residual stream [B, d] after the last layer (x, updated in place, when given); the
        final RMSNorm is left to the consumer (the LM-head kernel applies it).
        prefix = (prefix_cache, prefix_len32, G, workspace): groups of G consecutive sequences share the
        prefix rows [0, prefix_len32[b // G]) of prefix_cache; `cache` then holds each sequence's own tokens
        (pos / cache_seqlens index it) and attention runs over prefix + own rows."""
        cfg, W, layers = self.cfg, self.w, self.dec.layers
        eps = cfg.norm_eps
        H, HKV, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        cos, sin = self._tables()
        if tok is not None:
            require_device(tok, "FastDecoder.decode")
            B, xr = tok.shape[0], None
        else:
            require_device(x, "FastDecoder.decode")
            _require(x.dtype == BF16 and x.is_contiguous(), "decode: x must be contiguous bf16")
            B, xr = x.shape[0], x
        ws = self.decode_workspace
        # row sums of squares of the residual, left by each residual GEMM for the next norm (one per 32-column
        # block): the norms run inside the qkv / gate_up GEMMs without a pass of their own over x
        ss_attn = torch.empty(B, cfg.d_model // 32, dtype=torch.float32, device=(tok if tok is not None else x).device)
        ss_mlp = torch.empty_like(ss_attn)
        for i, blk in enumerate(layers):
            a = blk.attn
            kc, vc = cache.k[i], cache.v[i]
            if xr is None:  # layer 0 of a step fed with token ids: the embedding gather + norm in the qkv launch,
                # which also stores the gathered rows as the residual stream
                emb = W(self.dec.embed.weight)
                xr = torch.empty(B, emb.shape[1], dtype=BF16, device=tok.device)
                q = ops.norm_qkv_rope_cache(emb, W(blk.attn_norm.weight), eps, W(a.qkv_proj.weight), W(a.q_norm.weight),
                                            W(a.k_norm.weight), cos, sin, pos, seq, kc, vc, H, HKV, D, rope_pos=rope_pos,
                                            tok=tok, x_store=xr)
            elif i == 0:  # x handed in by the caller: no row sums yet
                h = ops.add_rmsnorm(xr, W(blk.attn_norm.weight), eps)
                q = ops.norm_qkv_rope_cache(h, None, eps, W(a.qkv_proj.weight), W(a.q_norm.weight),
                                            W(a.k_norm.weight), cos, sin, pos, seq, kc, vc, H, HKV, D, rope_pos=rope_pos)
            else:
                q = ops.norm_qkv_rope_cache(xr, W(blk.attn_norm.weight), eps, W(a.qkv_proj.weight), W(a.q_norm.weight),
                                            W(a.k_norm.weight), cos, sin, pos, seq, kc, vc, H, HKV, D, rope_pos=rope_pos,
                                            ss=ss_attn)
            if self.attn_marks is not None:
                self.attn_marks(i, 0)
            if prefix is None:
                o = ops.decode_attention(q, kc, vc, cache_seqlens, workspace=ws, rows=seq)
            else:
                pc, plen32, G, gws = prefix
                o = ops.decode_attention_grouped(q, pc.k[i], pc.v[i], plen32, kc, vc, cache_seqlens, G, workspace=gws)
            if self.attn_marks is not None:
                self.attn_marks(i, 1)
            ops.linear_residual(o.view(B, H * D), W(a.o_proj.weight), xr, ss_out=ss_mlp)
            g = ops.norm_linear(xr, W(blk.mlp_norm.weight), eps, W(blk.gate_up.weight), swiglu=True, ss=ss_mlp)
            last = i == len(layers) - 1
            ops.linear_residual(g, W(blk.down.weight), xr, ss_out=None if last else ss_attn)
        return xr

    # ---- Decoder.forward on this path ----------------------------------------------------------
    def forward(self, x, cache=None, batch_slice=slice(None), pos=None, positions=None):
        """Decoder.forward on this path (reference: viktor/decoder.py:135-144 with Attention.forward at 69-79).
        Prefill mode (pos None): a causal pass over x [B, T, d]; with a cache, k / v of position t go to cache
        rows batch_slice (B of them) at positions 0..T-1. Decode mode (pos [B]): T == 1, one row per cache
        sequence (the reference writes cache rows 0..B-1 at pos and ignores batch_slice)."""
        require_device(x, "Decoder.forward")
        B, T, d = x.shape
        dev = x.device
        xb = x.to(BF16).reshape(B * T, d).contiguous()
        _require(batch_slice.step in (None, 1), "Decoder.forward: batch_slice must be contiguous")
        row0 = 0 if batch_slice.start is None else int(batch_slice.start)
        if pos is not None:
            _require(T == 1 and cache is not None, "Decoder.forward: decode mode needs T == 1 and a cache")
            _require(cache.k.shape[1] == B, f"Decoder.forward: decode mode needs one cache row per sequence "
                                            f"({B} sequences, {cache.k.shape[1]} cache rows)")
            _require(pos.shape == (B,), "Decoder.forward: pos [B]")
            pos32 = pos.to(torch.int32).contiguous()
            rows = torch.arange(B, dtype=torch.int32, device=dev)
            seqlens = (pos32 + 1).contiguous()
            rp = None if positions is None else positions.reshape(B).to(torch.int32).contiguous()
            if cache is not None and self.decode_workspace is None:
                self.decode_workspace = ops.decode_attention_workspace(cache.k.shape[1], self.cfg.n_heads,
                                                                       cache.k.shape[2], dev)
            h = self.decode(xb, pos32, rows, seqlens, cache, rope_pos=rp)
            return h.view(B, 1, d)
        if cache is not None:
            stop = row0 + B if batch_slice.stop is None else int(batch_slice.stop)
            _require(stop - row0 == B and 0 <= row0 and stop <= cache.k.shape[1],
                     "Decoder.forward: batch_slice must select B rows of the cache")
            _require(T <= cache.k.shape[2], "Decoder.forward: T exceeds the cache length")
        key = (B, T, row0, cache is not None)
        plan = self._plans.get(key)
        if plan is None:
            rows = list(range(row0, row0 + B)) if cache is not None else None
            plan = PrefillPlan([T] * B, dev, rows=rows, cache=cache)
            self._plans[key] = plan
        pos32 = torch.arange(T, dtype=torch.int32, device=dev).repeat(B)
        seq = torch.arange(row0, row0 + B, dtype=torch.int32, device=dev).repeat_interleave(T)
        rp = None
        if positions is not None:
            rp = positions.expand(B, T).reshape(B * T).to(torch.int32).contiguous()
        h = self.prefill(xb, pos32, seq, None, T, cache, rope_pos=rp, plan=plan)
        return h.view(B, T, d)
