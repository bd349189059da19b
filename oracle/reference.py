"""CPU restatement of the reference decoder path (test infrastructure; see oracle/__init__.py).

Numerics modes:
  "fp32"     -- viktor/decoder.py in fp32: F.rms_norm, apply_rope, SDPA, F.linear, fp32 residual stream.
  "fused"    -- the fused inference path's rounding points (viktor/triton_ops.py:1-10, 25-31, 44-49, 132-134,
                219; viktor/fast_decoder.py:33-60): every op reads bf16, computes in fp32 and stores bf16;
                weights are bf16; logits fp32 for greedy decode steps, bf16 for the prefill token and for
                sampled steps (viktor/engine.py:96, 112, 191).
  "autocast" -- the reference's scoring path: Basecaller.logits of the fp32 master model under
                torch.autocast("cuda", bf16) (scripts/gspo.py:345-347; viktor/model.py:55-60, 71-85;
                viktor/decoder.py:63-67, 82-87, 117-120, 144). Rounding points, as torch 2.10's autocast
                applies them on the GPU (ops outside autocast's lists run in their inputs' dtype):
                  * nn.Linear: input and weight (and bias) cast to bf16, fp32 accumulation, bf16 output;
                  * the residual stream is fp32: prefix rows fp32(bf16 projector output), token rows the fp32
                    embedding (nn.Embedding is not cast), and x + sublayer(x) adds a bf16 output in fp32;
                  * nn.RMSNorm of the fp32 stream runs in fp32 with the fp32 weights; the next nn.Linear rounds
                    it to bf16 (the final norm too, at the LM head);
                  * the QK-norm of a bf16 head with fp32 weights returns bf16(x / rms * w) (torch's rms_norm
                    computes in fp32 and casts back to its input's dtype when the weight dtype differs);
                    apply_rope runs in fp32 with the fp32 tables and casts back to bf16 -- the rounding points
                    of the fused path's qkv_rope_cache, with fp32 weights and tables;
                  * F.silu(gate) * up: silu of the bf16 gate rounded to bf16, the product rounded to bf16;
                  * flash_attn_func: bf16 q / k / v, fp32 scores, bf16 probabilities in the PV product
                    (attention_rows with p_bf16), bf16 output;
                  * logits bf16; log_softmax of their fp32 cast.
"""

import math

import numpy as np
import torch
import torch.nn.functional as F

PAD, BOS, EOS = 0, 1, 2


def bf(t):
    """Round an fp32 tensor to bf16 precision (round to nearest even), keep fp32 storage."""
    return t.to(torch.bfloat16).to(torch.float32)


# ---------------------------------------------------------------------------------------------
# rope (viktor/encoder.py:30-40)
def rope_tables(dim, max_len, theta):
    inv = 1.0 / theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv
    return ang.cos().float(), ang.sin().float()


def apply_rope(x, cos, sin):
    """x [..., T, H, D]; cos/sin [..., T, D/2]: rotate the first half against the second half (in fp32, or in
    fp64 for fp64 input)."""
    x1, x2 = x.to(torch.promote_types(x.dtype, torch.float32)).chunk(2, -1)
    c, s = cos.unsqueeze(-2), sin.unsqueeze(-2)
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1)


# ---------------------------------------------------------------------------------------------
# fused-path ops (bf16 in / fp32 inside / bf16 out)
def rmsnorm_fused(x, w, eps):
    """bf16(x * rsqrt(mean(x^2) + eps) * w) of bf16-valued x (viktor/triton_ops.py:28-31)."""
    r = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    return bf(x * r * w)


def add_rmsnorm_fused(x, delta, w, eps):
    """(x_new, h): x_new = bf16(x + delta), h = rmsnorm_fused(x_new) (viktor/triton_ops.py:17-31)."""
    xn = bf(x + delta) if delta is not None else x
    return xn, rmsnorm_fused(xn, w, eps)


def linear_fused(x, w, out_fp32=False):
    y = x @ w.t()
    return y if out_fp32 else bf(y)


def swiglu_fused(g, u):
    """bf16(bf16(silu(g)) * u) of bf16 g, u (viktor/triton_ops.py:132-134, 217-220)."""
    return bf(bf(g * torch.sigmoid(g)) * u)


def qk_norm_rope_fused(x, w, cos, sin, eps):
    """x [n, H, D] bf16 values; cos/sin [n, D/2] (table dtype already applied). Per-head RMSNorm over D
    rounded to bf16, then the rotation rounded to bf16 (viktor/triton_ops.py:44-49)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    r = torch.rsqrt(((x1 * x1).sum(-1, keepdim=True) + (x2 * x2).sum(-1, keepdim=True)) / x.shape[-1] + eps)
    y1 = bf(x1 * r * w[:half])
    y2 = bf(x2 * r * w[half:])
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([bf(y1 * c - y2 * s), bf(y1 * s + y2 * c)], -1)


def attention_rows(q, k, v, causal_shift=None, p_bf16=False, block=None):
    """Exact fp32 softmax attention of one sequence. q [Tq, H, D], k/v [Tk, Hkv, D]; query head h reads KV
    head h // (H / Hkv) (GQA, viktor/decoder.py:91-105 repeat_interleave); query r sits at key position
    causal_shift + r when causal_shift is not None. Returns [Tq, H, D] fp32.
    p_bf16: the flash-attention rounding point -- the unnormalised weights exp(s - max) are rounded to bf16
    for the PV product while the normaliser sums them unrounded (viktor/decode_attention.py:27-37 stores
    p.to(v.dtype) the same way): o = sum_j bf16(e_j) v_j / sum_j e_j.
    block (with p_bf16): the weights rounded the way a tiled online-softmax kernel rounds them -- key blocks of
    `block` visited from the last to the first, as flash-attention 2's forward walks them (flash_attn_func, the
    reference's scoring attention; a third-party kernel that is not here, restated from its published design), each
    block's weights exp(s - running max) rounded to bf16 for the PV product, the accumulator and the unrounded
    normaliser rescaled when the running max grows."""
    Tq, H, D = q.shape
    Tk, Hkv, _ = k.shape
    rep = H // Hkv
    qg = q.reshape(Tq, Hkv, rep, D)
    s = torch.einsum("qgrd,kgd->grqk", qg, k) / math.sqrt(D)  # [Hkv, rep, Tq, Tk]
    if causal_shift is not None:
        qp = causal_shift + torch.arange(Tq)[:, None]
        kp = torch.arange(Tk)[None, :]
        s = s.masked_fill((kp > qp)[None, None], float("-inf"))
    if not p_bf16:
        p = torch.softmax(s, -1)
        return torch.einsum("grqk,kgd->qgrd", p, v).reshape(Tq, H, D)
    if block is not None:
        m = torch.full((Hkv, rep, Tq, 1), float("-inf"))
        lsum = torch.zeros(Hkv, rep, Tq, 1)
        acc = torch.zeros(Hkv, rep, Tq, D)
        for b0 in reversed(range(0, Tk, block)):
            sb = s[..., b0:b0 + block]
            m_new = torch.maximum(m, sb.amax(-1, keepdim=True))
            live = torch.isfinite(m_new)  # rows with no unmasked key yet keep their (empty) state
            mn = torch.where(live, m_new, torch.zeros_like(m_new))
            scale = torch.where(torch.isfinite(m), torch.exp(m - mn), torch.zeros_like(m))
            e = torch.exp(sb - mn)
            lsum = lsum * scale + e.sum(-1, keepdim=True)
            acc = acc * scale + torch.einsum("grqk,kgd->grqd", bf(e), v[b0:b0 + block])
            m = torch.where(live, m_new, m)
        return (acc / lsum).permute(2, 0, 1, 3).reshape(Tq, H, D)
    e = torch.exp(s - s.amax(-1, keepdim=True))
    o = torch.einsum("grqk,kgd->grqd", bf(e), v) / e.sum(-1, keepdim=True)
    return o.permute(2, 0, 1, 3).reshape(Tq, H, D)


# ---------------------------------------------------------------------------------------------
class RefModel:
    """fp32 CPU copy of a Basecaller's projector + decoder weights, run in one numerics mode."""

    def __init__(self, model, mode="fp32", table_bf16=None, p_bf16=False, attn_block=None):
        """p_bf16 (fused mode): attention weights rounded to bf16 before the PV product, the rounding point of
        flash-attention and of the reference's decode kernel (attention_rows). Off by default: the two choices
        bracket the reference's bf16 rounding noise. Autocast mode always rounds them (flash_attn_func); attn_block
        (autocast mode): round them blockwise as a tiled kernel does (attention_rows), instead of against the row's
        final maximum -- two equally faithful restatements whose spread is the reference's own rounding noise."""
        self.attn_block = attn_block if mode == "autocast" else None
        assert mode in ("fp32", "fused", "autocast")
        self.mode = mode
        self.p_bf16 = (bool(p_bf16) and mode == "fused") or mode == "autocast"
        self.cfg = model.decoder.cfg
        self.k = model.tokenizer.k
        self.strings = list(model.tokenizer.strings)
        self.V = model.tokenizer.vocab_size
        self.tail = model.tokenizer.tail_mask.clone().bool()
        self.pos_scale = getattr(model, "pos_scale", 1)
        sd = {n: p.detach().float().cpu().clone() for n, p in model.named_parameters()}
        if mode == "fused":
            sd = {n: bf(t) for n, t in sd.items()}
        elif mode == "autocast":  # products take bf16 copies (biases too); norms and the embedding stay fp32
            sd = {n: bf(t) if (t.dim() == 2 and not n.endswith("embed.weight")) or n.endswith("bias") else t
                  for n, t in sd.items()}
        self.p = sd
        cos, sin = rope_tables(self.cfg.head_dim, self.cfg.max_seq_len, self.cfg.rope_theta)
        if table_bf16 is None:
            table_bf16 = mode == "fused"
        self.cos, self.sin = (bf(cos), bf(sin)) if table_bf16 else (cos, sin)
        self.is_homo = torch.tensor([i >= 3 and len(t) == self.k and len(set(t)) == 1
                                     for i, t in enumerate(self.strings)])

    @classmethod
    def from_decoder(cls, dec, mode="fp32"):
        """A RefModel of a bare Decoder (no projector / tokenizer): for decoder_forward and head only."""
        self = cls.__new__(cls)
        self.mode, self.cfg = mode, dec.cfg
        self.p_bf16 = False
        self.attn_block = None
        sd = {f"decoder.{n}": p.detach().float().cpu().clone() for n, p in dec.named_parameters()}
        self.p = {n: bf(t) for n, t in sd.items()} if mode == "fused" else sd
        cos, sin = rope_tables(dec.cfg.head_dim, dec.cfg.max_seq_len, dec.cfg.rope_theta)
        self.cos, self.sin = (bf(cos), bf(sin)) if mode == "fused" else (cos, sin)
        self.pos_scale = 1
        return self

    def L(self, i, name):
        return self.p[f"decoder.layers.{i}.{name}"]

    # projector: Linear -> GELU -> Linear (viktor/model.py:35), bf16 activations in fused and autocast modes
    def project(self, frames):
        p = self.p
        if self.mode == "fp32":
            h = F.gelu(frames @ p["projector.0.weight"].t() + p["projector.0.bias"])
            return h @ p["projector.2.weight"].t() + p["projector.2.bias"]
        x = bf(frames)
        h = bf(x @ p["projector.0.weight"].t() + p["projector.0.bias"])
        h = bf(F.gelu(h))
        return bf(h @ p["projector.2.weight"].t() + p["projector.2.bias"])

    def embed(self, tok):
        return self.p["decoder.embed.weight"][tok]

    # ---- one layer over T new positions of one sequence (prefix K/V in kv lists) ----------------
    def layer(self, i, x, h, rpos, kv, causal_shift):
        """x: residual [T, d]; h: its attention norm [T, d]; rpos [T] RoPE rows; kv[i] = (K, V) cache of this
        sequence for layer i (appended here). Returns (x, h_next)."""
        cfg = self.cfg
        H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        eps = cfg.norm_eps
        T = x.shape[0]
        cos, sin = self.cos[rpos], self.sin[rpos]
        if self.mode == "autocast":
            return self._layer_autocast(i, x, h, cos, sin, kv, causal_shift)
        fused = self.mode == "fused"
        qkv = linear_fused(h, self.L(i, "attn.qkv_proj.weight")) if fused else h @ self.L(i, "attn.qkv_proj.weight").t()
        qkv = qkv.view(T, H + 2 * Hkv, D)
        q, k, v = qkv[:, :H], qkv[:, H:H + Hkv], qkv[:, H + Hkv:]
        if fused:
            q = qk_norm_rope_fused(q, self.L(i, "attn.q_norm.weight"), cos, sin, eps)
            k = qk_norm_rope_fused(k, self.L(i, "attn.k_norm.weight"), cos, sin, eps)
        else:
            q = apply_rope(F.rms_norm(q, (D,), self.L(i, "attn.q_norm.weight"), eps), cos, sin)
            k = apply_rope(F.rms_norm(k, (D,), self.L(i, "attn.k_norm.weight"), eps), cos, sin)
        K0, V0 = kv[i]
        K = torch.cat([K0, k]) if K0 is not None else k
        Vv = torch.cat([V0, v]) if V0 is not None else v
        kv[i] = (K, Vv)
        o = attention_rows(q, K, Vv, causal_shift=causal_shift, p_bf16=self.p_bf16)
        if fused:
            o = bf(o)
            x, h = add_rmsnorm_fused(x, linear_fused(o.reshape(T, -1), self.L(i, "attn.o_proj.weight")),
                                     self.L(i, "mlp_norm.weight"), eps)
            gu = self.L(i, "gate_up.weight")
            Fd = gu.shape[0] // 2
            g = linear_fused(h, gu[:Fd])
            u = linear_fused(h, gu[Fd:])
            m = swiglu_fused(g, u)
            w_next = self.L(i + 1, "attn_norm.weight") if i + 1 < cfg.n_layers else self.p["decoder.norm.weight"]
            x, h = add_rmsnorm_fused(x, linear_fused(m, self.L(i, "down.weight")), w_next, eps)
            return x, h
        x = x + o.reshape(T, -1) @ self.L(i, "attn.o_proj.weight").t()
        h2 = F.rms_norm(x, (cfg.d_model,), self.L(i, "mlp_norm.weight"), eps)
        gate, up = (h2 @ self.L(i, "gate_up.weight").t()).chunk(2, -1)
        x = x + (F.silu(gate) * up) @ self.L(i, "down.weight").t()
        w_next = self.L(i + 1, "attn_norm.weight") if i + 1 < cfg.n_layers else self.p["decoder.norm.weight"]
        return x, F.rms_norm(x, (cfg.d_model,), w_next, eps)

    def _layer_autocast(self, i, x, h, cos, sin, kv, causal_shift):
        """One block under torch.autocast bf16 (viktor/decoder.py:117-120 with Attention at 63-87): x fp32,
        h = bf16 operand of qkv_proj. Returns (x, bf16 operand of the next product)."""
        cfg = self.cfg
        H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        eps = cfg.norm_eps
        T = x.shape[0]
        qkv = linear_fused(h, self.L(i, "attn.qkv_proj.weight")).view(T, H + 2 * Hkv, D)
        q, k, v = qkv[:, :H], qkv[:, H:H + Hkv], qkv[:, H + Hkv:]
        q = qk_norm_rope_fused(q, self.L(i, "attn.q_norm.weight"), cos, sin, eps)
        k = qk_norm_rope_fused(k, self.L(i, "attn.k_norm.weight"), cos, sin, eps)
        K0, V0 = kv[i]
        K = torch.cat([K0, k]) if K0 is not None else k
        Vv = torch.cat([V0, v]) if V0 is not None else v
        kv[i] = (K, Vv)
        o = bf(attention_rows(q, K, Vv, causal_shift=causal_shift, p_bf16=True, block=self.attn_block))
        x = x + linear_fused(o.reshape(T, -1), self.L(i, "attn.o_proj.weight"))
        h2 = bf(F.rms_norm(x, (cfg.d_model,), self.L(i, "mlp_norm.weight"), eps))
        gu = self.L(i, "gate_up.weight")
        Fd = gu.shape[0] // 2
        m = swiglu_fused(linear_fused(h2, gu[:Fd]), linear_fused(h2, gu[Fd:]))
        x = x + linear_fused(m, self.L(i, "down.weight"))
        w_next = self.L(i + 1, "attn_norm.weight") if i + 1 < cfg.n_layers else self.p["decoder.norm.weight"]
        return x, bf(F.rms_norm(x, (cfg.d_model,), w_next, eps))

    def first_norm(self, x):
        w = self.L(0, "attn_norm.weight")
        if self.mode == "fused":
            return rmsnorm_fused(x, w, self.cfg.norm_eps)
        if self.mode == "autocast":
            return bf(F.rms_norm(x, (self.cfg.d_model,), w, self.cfg.norm_eps))
        return F.rms_norm(x, (self.cfg.d_model,), w, self.cfg.norm_eps)

    def run(self, x, rpos, kv, start):
        """Forward T new rows x [T, d] of one sequence at positions start.. (KV cache kv appended).
        Returns the final-normed hidden [T, d] (after the last layer's add + final norm)."""
        h = self.first_norm(x)
        for i in range(self.cfg.n_layers):
            x, h = self.layer(i, x, h, rpos, kv, causal_shift=start)
        return h

    def new_kv(self):
        return [(None, None) for _ in range(self.cfg.n_layers)]

    def head(self, h, round_bf16):
        z = h @ self.p["decoder.lm_head.weight"].t()
        return bf(z) if round_bf16 else z

    # ---- Decoder.forward (full causal pass) and Basecaller.logits ---------------------------------
    @torch.no_grad()
    def decoder_forward(self, x, positions=None):
        """x [B, T, d] -> final-normed hidden [B, T, d] (reference: viktor/decoder.py:135-144)."""
        B, T, _ = x.shape
        out = []
        for b in range(B):
            if positions is None:
                rpos = torch.arange(T)
            else:
                rpos = positions if positions.dim() == 1 else positions[b]
            xb = bf(x[b]) if self.mode == "fused" else x[b].clone()
            out.append(self.run(xb, rpos.long(), self.new_kv(), 0))
        return torch.stack(out)

    @torch.no_grad()
    def logits(self, frames, tokens_in, plens=None, round_logits=True):
        """Teacher-forced logits [B, T, V] (fp32 mode) or bf16-rounded (fused and autocast modes), reference:
        viktor/model.py:55-85 with the window packed as [plens[b] frames | tokens]. round_logits False: the
        head's fp32 products before that rounding."""
        return self._logits(frames, tokens_in, plens, round_logits)

    def _logits(self, frames, tokens_in, plens=None, round_logits=True):
        B, P, _ = frames.shape
        T = tokens_in.shape[1]
        out = []
        for b in range(B):
            n = P if plens is None else int(plens[b])
            pre = self.project(frames[b, :n])
            emb = self.embed(tokens_in[b])
            x = torch.cat([pre, emb])
            s = self.pos_scale
            if s == 1:
                rpos = torch.arange(n + T)
            else:
                rpos = torch.cat([torch.arange(n) * s, s * n + torch.arange(T)])
            h = self.run(x, rpos, self.new_kv(), 0)[n:]
            out.append(self.head(h, round_bf16=round_logits and self.mode in ("fused", "autocast")))
        return torch.stack(out)


# ---------------------------------------------------------------------------------------------
# token choice (viktor/engine.py:79-89 + supplied-uniform sampling)
def sample_inverse_cdf(z, u):
    """z [V] fp32 (logits + bias, already / T); u scalar in [0, 1). Returns (token, margin): the first v with
    u < cdf_v of softmax(z) accumulated in fp32 in token order (the last positive-probability token when
    rounding leaves u above the total), and the distance from u to the nearest CDF boundary."""
    zn = z.numpy().astype(np.float32)
    zmax = np.float32(zn.max())
    e = np.exp((zn - zmax).astype(np.float32)).astype(np.float32)
    s = np.float32(0.0)
    for v in range(len(e)):
        s = np.float32(s + e[v])
    inv = np.float32(np.float32(1.0) / s)
    cdf = np.float32(0.0)
    pick, last_pos = -1, int(np.argmax(zn))
    margin = np.inf
    for v in range(len(e)):
        pv = np.float32(e[v] * inv)
        if pv > 0:
            last_pos = v
        cdf = np.float32(cdf + pv)
        if pv > 0:
            margin = min(margin, abs(float(u) - float(cdf)))
        if pick < 0 and float(u) < float(cdf):
            pick = v
    return (pick if pick >= 0 else last_pos), margin


def sample_gumbel(z, u):
    """z [V] fp32 (logits + bias, already / T); u [V] uniforms in [0, 1). The reference's Gumbel-max choice
    (viktor/engine.py:80-83): the first index of the maximum of z - log(-log(max(u, 1e-20))), computed in float32;
    returns (token, the top-1 minus top-2 gap of those perturbed scores)."""
    zn = z.numpy().astype(np.float32)
    un = np.maximum(np.asarray(u, dtype=np.float32), np.float32(1e-20))
    g = (zn - np.log(-np.log(un).astype(np.float32)).astype(np.float32)).astype(np.float32)
    v = int(np.argmax(g))  # numpy returns the first maximal index
    finite = np.sort(g[np.isfinite(g)])
    gap = float(finite[-1] - finite[-2]) if finite.size >= 2 else np.inf
    return v, gap


def greedy_choice(z):
    """First index of the maximum, and the top-1 minus top-2 gap."""
    v = int(torch.argmax(z))  # torch.argmax returns the first maximal index
    top = torch.topk(z, 2).values
    return v, float(top[0] - top[1])


def apply_grammar(nxt, prev, run, is_tail, is_homo, homo_stop):
    """Tail -> EOS, homopolymer run -> EOS, PAD after EOS/PAD (viktor/engine.py:84-89). Returns (token, run)."""
    if 0 <= prev < len(is_tail) and bool(is_tail[prev]):
        nxt = EOS
    if homo_stop:
        run = run + 1 if (nxt == prev and bool(is_homo[nxt])) else 0
        if run + 1 >= homo_stop:
            nxt = EOS
    if prev in (EOS, PAD):
        nxt = PAD
    return nxt, run


class RefEngine:
    """DecodeEngine semantics on the CPU (viktor/engine.py:31-220, torch backend; supplied-uniform
    sampling instead of device Gumbel noise). One sequence at a time; KV cache as per-layer tensors."""

    def __init__(self, ref: RefModel, max_new, temperature=0.0, max_homopolymer=64, bias=None, sampling="inverse_cdf"):
        """bias: [V] additive logit bias replacing the engine's default (-inf at PAD and BOS), e.g. one that
        also bans EOS so that every sequence runs to max_new (DecodeEngine.bias is the same tensor).
        sampling "gumbel": the reference's formula (viktor/engine.py:80-83), argmax of
        z / T - log(-log(clamp(u, 1e-20))) with uniforms [B, steps, V]; "inverse_cdf": uniforms [B, steps]."""
        assert sampling in ("inverse_cdf", "gumbel")
        self.gumbel = sampling == "gumbel"
        self.ref = ref
        self.max_new = max_new
        self.T = float(temperature)
        V = ref.V
        if bias is None:
            bias = torch.zeros(V)
            bias[[PAD, BOS]] = float("-inf")
        self.bias = bias.detach().float().cpu().clone()
        assert self.bias.shape == (V,)
        self.homo_stop = max_homopolymer // ref.k if max_homopolymer else 0

    def _choose(self, logits, prev, run, u):
        z = logits.float() + self.bias
        if self.T > 0 and self.gumbel:
            raw, margin = sample_gumbel(z / self.T, u)
        elif self.T > 0:
            raw, margin = sample_inverse_cdf(z / self.T, u)
        else:
            raw, margin = greedy_choice(z)
        nxt, run2 = apply_grammar(raw, prev, run, self.ref.tail, self.ref.is_homo, self.homo_stop)
        return raw, nxt, run2, margin

    @torch.no_grad()
    def run(self, frames_list, steps=None, uniforms=None, forced=None):
        """frames_list: per sequence [L_b, d_enc] fp32. steps: output tokens (default max_new).
        forced [B, steps]: tokens to feed back instead of the oracle's own (teacher forcing on another
        implementation's stream). Entries of frames_list that are the same tensor object are prefilled once. Returns dict(tokens, choice, margin, logits) with choice = the oracle's
        token at each position given the (forced) history, margin = top-2 gap (greedy) or distance of the
        uniform to a CDF boundary (sampled)."""
        ref = self.ref
        steps = self.max_new if steps is None else steps
        B = len(frames_list)
        tokens = torch.full((B, self.max_new), PAD, dtype=torch.long)
        choice = torch.full((B, steps), PAD, dtype=torch.long)
        margin = torch.full((B, steps), float("inf"))
        logit_rows = torch.zeros(B, steps, ref.V)
        fused = ref.mode == "fused"
        s = ref.pos_scale
        prefilled = {}  # id(frames) -> (kv after the prefix, BOS hidden): members of one group share it
        for b, fr in enumerate(frames_list):
            n = fr.shape[0]
            hit = prefilled.get(id(fr))
            if hit is None:
                kv = ref.new_kv()
                x = torch.cat([ref.project(fr), ref.embed(torch.tensor([BOS]))])
                rpos = torch.arange(n + 1) * s if s != 1 else torch.arange(n + 1)
                h = ref.run(x, rpos, kv, 0)[-1:]
                prefilled[id(fr)] = (list(kv), h)
            else:  # layer() appends by concatenation, so the shared prefix tensors are never written
                kv, h = list(hit[0]), hit[1]
            prev, run = BOS, 0
            for j in range(steps):
                # prefill token from bf16 logits; later greedy steps fp32, sampled steps bf16
                round_bf16 = fused and (j == 0 or self.T > 0)
                z = ref.head(h, round_bf16)[0]
                logit_rows[b, j] = z
                if uniforms is None:
                    u = 0.0
                else:
                    u = uniforms[b, j] if self.gumbel else float(uniforms[b, j])
                raw, nxt, run_new, m = self._choose(z, prev, run, u)
                choice[b, j] = nxt
                margin[b, j] = m
                fed = nxt if forced is None else int(forced[b, j])
                if forced is not None and fed not in (EOS, PAD):
                    run = run_new if fed == raw else (run + 1 if (fed == prev and bool(ref.is_homo[fed])) else 0)
                else:
                    run = run_new
                tokens[b, j] = fed
                prev = fed
                if j + 1 == steps:
                    break
                pos = n + 1 + j
                rp = torch.tensor([pos + n * (s - 1)])
                h = ref.run(ref.embed(torch.tensor([fed])), rp, kv, pos)
        return {"tokens": tokens, "choice": choice, "margin": margin, "logits": logit_rows}


def greedy_full_recompute(ref: RefModel, frames_list, max_new, max_homopolymer=None):
    """The reference test's brute-force decoder (tests/test_viktor.py:33-54): recompute the whole sequence
    every step without a cache (plus the homopolymer rule when max_homopolymer is given)."""
    bias = torch.zeros(ref.V)
    bias[[PAD, BOS]] = float("-inf")
    homo_stop = max_homopolymer // ref.k if max_homopolymer else 0
    out = []
    for fr in frames_list:
        prefix = ref.project(fr)
        toks, prev, run = [], BOS, 0
        for j in range(max_new):
            x = torch.cat([prefix, ref.embed(torch.tensor([BOS] + toks))])
            h = ref.run(x, torch.arange(x.shape[0]), ref.new_kv(), 0)[-1]
            z = ref.head(h[None], ref.mode == "fused" and j == 0)[0]
            raw = int(torch.argmax(z + bias))
            nxt, run = apply_grammar(raw, prev, run, ref.tail, ref.is_homo, homo_stop)
            if nxt not in (EOS, PAD):
                toks.append(nxt)
            out.append(nxt)
            prev = nxt
    return torch.tensor(out).view(len(frames_list), max_new)


# ---------------------------------------------------------------------------------------------
# GSPO (scripts/gspo.py:340-353, 446-477)
def token_logprobs_ref(logits, targets):
    """log_softmax(fp32 logits) gathered at the PAD-clamped targets."""
    return torch.log_softmax(logits.float(), -1).gather(-1, targets.clamp(min=0)[..., None])[..., 0]


def sampled_mask_ref(targets, seqs, ended, k):
    mask = targets != PAD
    for b, (s, e) in enumerate(zip(seqs, ended)):
        if not e or len(s) % k:
            mask[b, -(-len(s) // k)] = False
    return mask


def advantages_ref(reward, std_floor=0.003, eps=None):
    r = np.asarray(reward, dtype=np.float64)
    std = r.std(1)
    live = np.nonzero(std > 1e-6)[0]
    den = (std + eps) if eps is not None else np.maximum(std, std_floor)
    return (r - r.mean(1, keepdims=True)) / den[:, None], live


def gspo_loss_autograd(logits, targets, mask, old_lp, n_bases, adv, eps_lo, eps_hi, inv_n):
    """The reference's per-sequence loss with autograd (scripts/gspo.py:474-477, separate low/high clip).
    Returns (loss, s, pg, lp, dlogits)."""
    z = logits.detach().float().clone().requires_grad_(True)
    lp = torch.log_softmax(z, -1).gather(-1, targets.clamp(min=0)[..., None])[..., 0]
    B = z.shape[0]
    s = torch.stack([((lp[b][mask[b]] - old_lp[b][mask[b]]).sum() / n_bases[b]).exp() for b in range(B)])
    a = adv.float()
    pg = -torch.minimum(s * a, s.clamp(1 - eps_lo, 1 + eps_hi) * a)
    loss = pg.sum() * inv_n
    loss.backward()
    return loss.detach(), s.detach(), pg.detach(), lp.detach(), z.grad


def gspo_param_grads(ref, frames, tokens_in, plens, targets, mask, old_lp, n_bases, adv, eps_lo, eps_hi, inv_n,
                     dtype=torch.float32):
    """Gradients of the GSPO loss (scripts/gspo.py:471-477) w.r.t. every projector / decoder parameter by
    autograd through the restated teacher-forced forward (viktor/model.py:55-60, viktor/decoder.py:54-144),
    in `dtype` (fp32 mode weights; fp64 for finite-difference checks). Returns (loss, {name: grad})."""
    assert ref.mode == "fp32"
    params = {n: t.detach().to(dtype).clone().requires_grad_(True) for n, t in ref.p.items()}
    saved, saved_tables = ref.p, (ref.cos, ref.sin)
    ref.p, ref.cos, ref.sin = params, ref.cos.to(dtype), ref.sin.to(dtype)
    try:
        with torch.enable_grad():
            z = ref._logits(frames.to(dtype), tokens_in, plens)
            lp = torch.log_softmax(z, -1).gather(-1, targets.clamp(min=0)[..., None])[..., 0]
            s = torch.stack([((lp[b][mask[b]] - old_lp[b][mask[b]].to(dtype)).sum() / n_bases[b]).exp()
                             for b in range(z.shape[0])])
            a = adv.to(dtype)
            pg = -torch.minimum(s * a, s.clamp(1 - eps_lo, 1 + eps_hi) * a)
            loss = pg.sum() * inv_n
            loss.backward()
    finally:
        ref.p, (ref.cos, ref.sin) = saved, saved_tables
    return loss.detach(), {n: p.grad for n, p in params.items() if p.grad is not None}


def gspo_grad_closed_form(logits, targets, mask, old_lp, n_bases, adv, eps_lo, eps_hi, inv_n):
    """dL/dlogits by the closed form (independent of autograd), fp64."""
    z = logits.double()
    lp = torch.log_softmax(z, -1)
    y = targets.clamp(min=0)
    lpy = lp.gather(-1, y[..., None])[..., 0]
    m = mask.double()
    s = torch.exp((m * (lpy - old_lp.double())).sum(1) / n_bases.double())
    A = adv.double()
    lo, hi = 1 - eps_lo, 1 + eps_hi
    a1 = s * A
    a2 = s.clamp(lo, hi) * A
    d2 = torch.where((s >= lo) & (s <= hi), A, torch.zeros_like(A))
    dmin = torch.where(a1 < a2, A, torch.where(a2 < a1, d2, 0.5 * (A + d2)))
    g = -dmin
    coef = inv_n * g * s / n_bases.double()
    onehot = F.one_hot(y, z.shape[-1]).double()
    return coef[:, None, None] * m[..., None] * (onehot - lp.exp())


# ---------------------------------------------------------------------------------------------
# GSPO reward: strict identity (scripts/gspo.py:86-89, ref_errors at scripts/train.py:170-188, EMPTY_MAX at
# scripts/evaluate.py:30)
EMPTY_MAX = 4


def edit_distance(a, b):
    """Levenshtein distance by the textbook row DP (independent of any path choice)."""
    prev = list(range(len(b) + 1))
    for i, ca in enumerate(a, 1):
        cur = [i] + [0] * len(b)
        for j, cb in enumerate(b, 1):
            cur[j] = min(prev[j] + 1, cur[j - 1] + 1, prev[j - 1] + (ca != cb))
        prev = cur
    return prev[-1]


def strict_identity_ref(call, ref, scored, empty_max=EMPTY_MAX):
    """(reward, edit distance, scored errors) of call against ref with scored [len(ref)] bool. The errors are
    those of the global alignment path whose every cell takes the first optimal predecessor in the order
    diagonal, deletion (of a ref base), insertion (of a call base): a mismatch or deletion counts at its ref
    base, an insertion at the ref base before it (base 0 before any ref base), as ref_errors places them.
    The count is carried forward along the chosen predecessors (numpy over anti-diagonals)."""
    n, m = len(call), len(ref)
    if m == 0:
        return (1.0 if n <= empty_max else empty_max / n), n, 0
    r = np.frombuffer(ref.encode(), np.uint8).astype(np.int64)
    c = np.frombuffer(call.encode(), np.uint8).astype(np.int64)
    sc = np.asarray(scored, dtype=bool).astype(np.int64)
    D = [np.zeros(m + 1, np.int64) for _ in range(3)]
    C = [np.zeros(m + 1, np.int64) for _ in range(3)]
    for k in range(m + n + 1):
        d0, c0 = D[k % 3], C[k % 3]
        d1, c1 = D[(k - 1) % 3], C[(k - 1) % 3]
        d2, c2 = D[(k - 2) % 3], C[(k - 2) % 3]
        lo, hi = max(0, k - n), min(m, k)
        i = np.arange(lo, hi + 1)
        j = k - i
        d = np.zeros_like(i)
        e = np.zeros_like(i)
        top, left, inner = i == 0, (j == 0) & (i > 0), (i > 0) & (j > 0)
        d[top] = j[top]
        e[top] = np.where(j[top] > 0, c1[0] + sc[0], 0)
        il = i[left]
        d[left] = il
        e[left] = c1[il - 1] + sc[il - 1]
        ii, jj = i[inner], j[inner]
        mis = (r[ii - 1] != c[jj - 1]).astype(np.int64)
        dd, du, dl = d2[ii - 1] + mis, d1[ii - 1] + 1, d1[ii] + 1
        best = np.minimum(np.minimum(dd, du), dl)
        e_in = np.where(dd == best, c2[ii - 1] + mis * sc[ii - 1],
                        np.where(du == best, c1[ii - 1] + sc[ii - 1], c1[ii] + sc[ii - 1]))
        d[inner] = best
        e[inner] = e_in
        d0[i] = d
        c0[i] = e
    dist, errs = int(D[(m + n) % 3][m]), int(C[(m + n) % 3][m])
    return 1.0 - errs / max(n, m), dist, errs
