"""The GSPO update on the HIP kernels: the teacher-forced forward with saved activations, its backward, the
gradient clip and the AdamW step.

Reference: scripts/gspo.py:340-353 (token_logprobs under torch.autocast bf16), 459-493 (the update loop:
loss.backward() through Basecaller.logits, clip_grad_norm_, AdamW(fused).step()), 113-126 (bf16_copy / sync);
viktor/model.py:55-60 (Basecaller.logits), viktor/decoder.py:54-144 (the decoder blocks).

The model keeps fp32 master weights, as the reference's trainable model does, and the forward keeps the rounding
points of torch.autocast bf16 over them (the autocast token_logprobs runs under, scripts/gspo.py:345-347): the
products take the weights cast to bf16 and give bf16 outputs, and every product-weight gradient arrives in fp32
through that cast; the residual stream, the token-embedding rows and the RMSNorm weights stay fp32
(viktor/model.py:81-84, viktor/decoder.py:117-120), and each RMSNorm is rounded once, to the bf16 operand of the
next product.
Every product of the update runs on the HIP kernels:
  * the decoder stack is one autograd node (`_DecoderStack`): its forward runs the prefill kernels over the
    packed windows and keeps each layer's activations; its backward runs the HIP backward kernels (attention,
    RMSNorm, QK-norm + RoPE, SwiGLU), the input gradients dX = dY W as MFMA products against W^T (formed once
    per backward) and the weight gradients dW = dY^T X as split-K MFMA reductions (vk_wgrad: fp32 row slices
    summed in a fixed order, rounded to bf16 once as the autocast matmul output);
  * the per-frame projector (`_Projector`: linear, bias + GELU, linear, bias) and the LM head (`_LMHead`,
    V = 7 or 343 columns: the V-wide operand zero-padded to the products' tile width) likewise;
  * the token-embedding gradient is a deterministic segmented row sum (vk_embed_grad) of the fp32 residual
    gradient rows.
"""

from typing import List, Optional, Sequence

import numpy as np
import torch

from . import hip_ops as ops
from .gspo import sequence_ratio_loss

BF16 = torch.bfloat16
_LAYER_PARAMS = ("attn_norm.weight", "attn.qkv_proj.weight", "attn.q_norm.weight", "attn.k_norm.weight",
                 "attn.o_proj.weight", "mlp_norm.weight", "gate_up.weight", "down.weight")


def decoder_params(dec) -> List[torch.Tensor]:
    """The decoder-stack parameters in _DecoderStack order: 8 per layer (_LAYER_PARAMS), then the final norm."""
    sd = dict(dec.named_parameters())
    out = [sd[f"layers.{i}.{n}"] for i in range(dec.cfg.n_layers) for n in _LAYER_PARAMS]
    return out + [sd["norm.weight"]]


def _residual_norm(x, a, w, norm_w, eps):
    """x + bf16(a @ w^T) on the fp32 residual stream x, into a new buffer (x is kept for the backward), then
    bf16(RMSNorm of it * norm_w) with fp32 norm_w: `x = x + sublayer(...)` and the next nn.RMSNorm under
    autocast (viktor/decoder.py:118-120). The residual add rides in the product's epilogue, which hands the row
    sums of squares to the norm. Returns (new stream, normed bf16 rows)."""
    y = torch.empty_like(x)
    return y, ops.rmsnorm_apply(y, ops.linear_residual_big(a, w, x, out=y), norm_w, eps)


class _TokenEmbed(torch.autograd.Function):
    """emb[tokens] in fp32 (the gather of viktor/model.py:77, 81-84: nn.Embedding of fp32 weights, which autocast
    leaves in fp32) with the table's gradient as the fp32 sum of the gradient rows of each token id (vk_embed_grad:
    deterministic, no atomics)."""

    @staticmethod
    def forward(ctx, weight, tokens):
        ctx.save_for_backward(tokens)
        ctx.vocab = weight.shape[0]
        return weight.detach().float()[tokens]

    @staticmethod
    def backward(ctx, d_rows):
        (tokens,) = ctx.saved_tensors
        d = d_rows.reshape(-1, d_rows.shape[-1]).float().contiguous()
        return ops.embed_grad(d, tokens.reshape(-1).contiguous(), ctx.vocab), None


def _pad_cols(t, width):
    """t [n, c] bf16 -> [n, width] with zero columns past c."""
    out = torch.zeros(t.shape[0], width, dtype=BF16, device=t.device)
    out[:, :t.shape[1]] = t
    return out


class _Projector(torch.autograd.Function):
    """Per-frame projector nn.Linear(d_enc, d) -> nn.GELU() -> nn.Linear(d, d) under torch.autocast bf16
    (viktor/model.py:35, 74): x [n, d_enc] bf16 -> [n, d] bf16. Each linear is an MFMA product with fp32 output
    whose epilogue adds the bf16-cast bias and rounds once (vk_bias_act, GELU fused after the first). Backward:
    bias gradients as fixed-order column sums, weight gradients by vk_wgrad, the GELU backward fused with the
    first bias's column sums (vk_act_backward); no input gradient (the frames are data)."""

    @staticmethod
    def forward(ctx, x, w1, b1, w2, b2):
        w1b, w2b = w1.detach().to(BF16).contiguous(), w2.detach().to(BF16).contiguous()
        b1b, b2b = (b.detach().to(BF16).float().contiguous() for b in (b1, b2))
        pre, a = ops.bias_act(ops.linear(x, w1b, out_dtype=torch.float32), b1b, gelu=True)
        y = ops.bias_act(ops.linear(a, w2b, out_dtype=torch.float32), b2b, gelu=False)
        ctx.save_for_backward(x, pre, a, w2b)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, pre, a, w2b = ctx.saved_tensors
        dy = dy.to(BF16).contiguous()
        gb2 = ops.act_backward(dy)
        gw2 = ops.wgrad(dy, a)
        da = ops.linear(dy, w2b.t().contiguous())
        dz, gb1 = ops.act_backward(da, pre)
        gw1 = ops.wgrad(dz, x)
        # autocast rounds the bias gradients to bf16 like the weight gradients
        return None, gw1.float(), gb1.to(BF16).float(), gw2.float(), gb2.to(BF16).float()


class _LMHead(torch.autograd.Function):
    """logits = h lm_head^T in bf16 (viktor/decoder.py:130, 163-164 under autocast): h [n, d] bf16, weight
    [V, d] fp32 master. The V-wide gradient operand is zero-padded to a multiple of 128 columns so that both
    backward products run on the MFMA kernels: dh = dz W (vk_linear against W^T padded) and dW = dz^T h
    (vk_wgrad, computed as (h^T dz)^T)."""

    @staticmethod
    def forward(ctx, h, weight):
        wb = weight.detach().to(BF16).contiguous()
        ctx.save_for_backward(h, wb)
        return ops.linear(h, wb)

    @staticmethod
    def backward(ctx, dz):
        h, wb = ctx.saved_tensors
        V = wb.shape[0]
        width = -(-V // 128) * 128
        zp = _pad_cols(dz.to(BF16), width)
        dh = ops.linear(zp, _pad_cols(wb.t(), width))
        gw = ops.wgrad(h, zp)[:, :V].t().float()
        return dh, gw


class _PackRows(torch.autograd.Function):
    """The packed decoder input x [N, d] fp32: the real prefix rows of each window followed by its token rows
    (the sequence viktor/model.py:72-86 builds per window with fp32 gathers, without its padding). prefix [B P, d]
    bf16 and emb [B T, d] fp32: the projector's and the embedding's rows; pre_src / pre_dst: the real prefix rows
    and their packed rows; tok_rows: the packed rows of the tokens, in emb's order. Each source row is used once,
    so the backward is two row gathers (no accumulation), the prefix rows' gradient rounded to bf16 as the
    backward of prefix.float() rounds it; all_prefix: every prefix row is real (pre_src is 0 .. B P - 1)."""

    @staticmethod
    def forward(ctx, prefix, emb, pre_src, pre_dst, tok_rows, all_prefix):
        x = torch.empty(pre_dst.numel() + tok_rows.numel(), prefix.shape[1], dtype=torch.float32, device=prefix.device)
        x.index_copy_(0, pre_dst, (prefix if all_prefix else prefix.index_select(0, pre_src)).float())
        x.index_copy_(0, tok_rows, emb)
        ctx.save_for_backward(pre_src, pre_dst, tok_rows)
        ctx.n_prefix, ctx.all_prefix = prefix.shape[0], all_prefix
        return x

    @staticmethod
    def backward(ctx, dx):
        pre_src, pre_dst, tok_rows = ctx.saved_tensors
        g = dx.index_select(0, pre_dst).to(BF16)
        if ctx.all_prefix:
            dp = g
        else:
            dp = g.new_zeros(ctx.n_prefix, dx.shape[1])
            dp.index_copy_(0, pre_src, g)
        return dp, dx.index_select(0, tok_rows), None, None, None, None


_NORMS = ("attn_norm.weight", "attn.q_norm.weight", "attn.k_norm.weight", "mlp_norm.weight")


class _DecoderStack(torch.autograd.Function):
    """x [N, d] fp32 packed rows -> final-normed hidden of the token rows [n_tok, d] bf16, with the rounding
    points of FastDecoder.teacher_forced (torch.autocast bf16 over fp32 master weights): products on bf16 weights,
    the RMSNorms (QK-norm included) on the fp32 weights, an fp32 residual stream. The forward runs the same
    kernels as teacher_forced (so its rows equal the scoring forward's bit for bit) and keeps what the backward
    needs: each layer's input and middle stream (written out of place), the unrotated Wqkv product and the
    gate | up rows."""

    @staticmethod
    def forward(ctx, x, meta, *params):
        cfg = meta["cfg"]
        H, HKV, D, eps = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.norm_eps
        L = cfg.n_layers
        N = x.shape[0]
        norm_slot = {8 * i + _LAYER_PARAMS.index(n) for i in range(L) for n in _NORMS} | {8 * L}
        w = [p.detach().float().contiguous() if j in norm_slot else p.detach().to(BF16).contiguous()
             for j, p in enumerate(params)]
        plan, rpos, cos, sin = meta["plan"], meta["rpos"], meta["cos"], meta["sin"]
        x = x.detach().float().contiguous()  # read only: every layer writes its stream into a new buffer
        h = ops.rmsnorm_f32(x, w[0], eps)
        saved = []
        for i in range(L):
            wa, wqkv, wqn, wkn, wo, wm, wgu, wd = w[8 * i:8 * i + 8]
            x_in = x
            # the product, then QK-norm + RoPE in its epilogue (the scoring forward's kernel), keeping the unrotated
            # projection for the backward
            qkv = torch.empty(N, wqkv.shape[0], dtype=BF16, device=x.device)
            q, k, v = ops.linear_qkv_rope(h, wqkv, wqn, wkn, cos, sin, rpos, None, None, None, eps, H, HKV, D,
                                          return_kv=True, qkv_out=qkv)
            lse = torch.empty(N, H, dtype=torch.float32, device=x.device)
            o = ops.varlen_attention(q, k, v, plan.attn, lse=lse, prefix=(k, v) if plan.prefixed else None)
            x_mid, h2 = _residual_norm(x_in, o.view(N, H * D), wo, wm, eps)
            # SwiGLU in the product's epilogue (the scoring forward's kernel), keeping gate | up for the backward
            gu = torch.empty(N, wgu.shape[0], dtype=BF16, device=x.device)
            g = ops.linear(h2, wgu, swiglu=True, gu_out=gu)
            w_next = w[8 * (i + 1)] if i + 1 < L else w[8 * L]
            x, h_next = _residual_norm(x_mid, g, wd, w_next, eps)
            saved.append((x_in, h, qkv, q, k, v, o, lse, x_mid, h2, gu, g))
            h = h_next
        ctx.meta, ctx.saved_acts, ctx.w, ctx.x_final = meta, saved, w, x
        return h[meta["tok_rows"]]

    @staticmethod
    def backward(ctx, dh_tok):
        meta, saved, w = ctx.meta, ctx.saved_acts, ctx.w
        cfg = meta["cfg"]
        H, HKV, D, eps = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.norm_eps
        L = cfg.n_layers
        plan, rpos, cos, sin = meta["plan"], meta["rpos"], meta["cos"], meta["sin"]
        x_final = ctx.x_final
        N, d = x_final.shape
        grads = [None] * len(w)
        dh = torch.zeros(N, d, dtype=torch.float32, device=x_final.device)
        dh[meta["tok_rows"]] = dh_tok.float()
        # each norm backward also writes its fp32 input gradient rounded to bf16 (the next products' operand)
        dxb = torch.empty(N, d, dtype=BF16, device=x_final.device)
        dx, grads[8 * L] = ops.rmsnorm_backward(x_final, w[8 * L], dh, eps, dx_bf16=dxb)  # dx: d loss / d x_L (fp32)
        for i in reversed(range(L)):
            x_in, h, qkv, q, k, v, o, lse, x_mid, h2, gu, g = saved[i]
            wa, wqkv, wqn, wkn, wo, wm, wgu, wd = w[8 * i:8 * i + 8]
            # x_{i+1} = x_mid + g Wd^T
            dm = dxb
            gd = ops.wgrad(dm, g)
            dg = ops.linear(dm, wd.t().contiguous())
            dgu = ops.swiglu_backward(gu, dg)
            ggu = ops.wgrad(dgu, h2)
            dh2 = ops.linear(dgu, wgu.t().contiguous())
            da = torch.empty(N, d, dtype=BF16, device=dx.device)
            dx, gm = ops.rmsnorm_backward(x_mid, wm, dh2, eps, dres=dx, dx_bf16=da)  # d / d x_mid
            # x_mid = x_in + o Wo^T
            go = ops.wgrad(da, o.view(N, H * D))
            do = ops.linear(da, wo.t().contiguous()).view(N, H, D)
            dq, dk, dv = ops.attention_backward(q, k, v, o, do, lse, plan.attn, plan.keys)
            dqkv, gqn, gkn = ops.qknorm_rope_backward(qkv, wqn, wkn, cos, sin, rpos, dq, dk, dv, eps, H, HKV, D)
            gqkv = ops.wgrad(dqkv, h)
            dhh = ops.linear(dqkv, wqkv.t().contiguous())
            dxb = torch.empty(N, d, dtype=BF16, device=dx.device) if i > 0 else None
            dx, ga = ops.rmsnorm_backward(x_in, wa, dhh, eps, dres=dx, dx_bf16=dxb)  # d / d x_in
            grads[8 * i:8 * i + 8] = [ga, gqkv, gqn, gkn, go, gm, ggu, gd]
        ctx.saved_acts = None
        return (dx, None, *[gr.float() for gr in grads])


class TrainPlan:
    """Work lists of one packed batch of causal sequences: the attention's 64-query blocks (forward and dQ)
    and 64-key blocks (dK / dV). Keys of sequence i are the packed k / v rows [n, 2, 64] from cu[i]."""

    def __init__(self, seq_lens, device, kv_row=128):
        cu = [0]
        for n in seq_lens:
            cu.append(cu[-1] + int(n))
        self.attn = ops.AttentionPlan(seq_lens, seq_lens, [c * kv_row for c in cu[:-1]], device, causal=True)
        self.keys = ops.KeyBlockPlan(seq_lens, device)
        self.prefixed = False

    @classmethod
    def shared(cls, pre_lens, G, T, device, kv_row=128):
        """The shared-prefix layout of groups of G windows with one prefix each: the n_groups prefixes packed
        first (group g: pre_lens[g] rows), then every member's T token rows. A prefix is a causal sequence on its
        own; a member's token rows see its group's prefix keys, then their own keys causally (in the key order
        of the window [prefix | tokens]); each prefix key block also collects the gradients of every member's T
        token rows, which see all of its keys (one work item per member, summed in member order)."""
        pre_lens = [int(p) for p in pre_lens]
        ng = len(pre_lens)
        cu_pre = np.concatenate([[0], np.cumsum(pre_lens)]).astype(np.int64)
        n_pre = int(cu_pre[-1])
        member_pre = np.repeat(np.asarray(pre_lens, dtype=np.int64), G)
        B = ng * G
        lens = pre_lens + [T] * B
        starts = np.concatenate([cu_pre[:-1], n_pre + T * np.arange(B, dtype=np.int64)])
        self = cls.__new__(cls)
        self.attn = ops.AttentionPlan(lens, pre_lens + (member_pre + T).tolist(), (starts * kv_row).tolist(), device,
                                      causal=True, p_lens=[0] * ng + member_pre.tolist(),
                                      p_off=[0] * ng + (np.repeat(cu_pre[:-1], G) * kv_row).tolist())
        # group g's prefix key blocks: its own causal rows, then one segment per member (T token rows each)
        extra = [[(n_pre + (g * G + m) * T, T) for m in range(G)] for g in range(ng)] + [None] * B
        self.keys = ops.KeyBlockPlan(lens, device, extra=extra)
        self.prefixed = True
        return self


def train_logits(model, frames, tokens_in, plens=None, group_size=1):
    """Differentiable Basecaller.logits: bf16 logits [B, T, V] of every token position, with gradients into the
    fp32 projector and decoder parameters (reference: viktor/model.py:55-60 under torch.autocast bf16, as
    token_logprobs calls it at scripts/gspo.py:345-347). frames [B, P, d_enc]; plens [B] real prefix frames.
    group_size = G > 1: consecutive groups of G windows share their frames (a GSPO micro-batch of whole groups,
    scripts/gspo.py:444, 459-466; checked, ValueError otherwise). Each group's prefix rows then run the
    projector and the decoder once, its members' token rows attend to them, and the backward sums every
    member's gradient into them: the same logits as the unshared forward, and the same gradients up to the
    order of the fp32 sums over the members."""
    dec = model.decoder
    cfg = dec.cfg
    B, P = frames.shape[:2]
    T = tokens_in.shape[1]
    dev = frames.device
    plens_h = [P] * B if plens is None else [int(p) for p in plens.tolist()]
    assert all(0 < p <= P for p in plens_h), "plens outside 1..P"
    if int(group_size) > 1:
        return _train_logits_shared(model, frames, tokens_in, plens_h, int(group_size))
    proj = model.projector
    prefix = _Projector.apply(frames.reshape(B * P, -1).to(BF16).contiguous(), proj[0].weight, proj[0].bias,
                              proj[2].weight, proj[2].bias)                            # [B P, d] bf16
    emb = _TokenEmbed.apply(dec.embed.weight, tokens_in.to(dev).reshape(-1))          # [B T, d] fp32
    # packed layout, window b: its plens[b] real prefix rows, then its T token rows; row indices on the host
    s = model.pos_scale

    def build():
        seq_lens = [p + T for p in plens_h]
        pl = np.asarray(plens_h, dtype=np.int64)
        off = np.concatenate([[0], np.cumsum(pl + T)])
        pre_dst = np.concatenate([np.arange(off[b], off[b] + pl[b]) for b in range(B)])
        pre_src = np.concatenate([b * P + np.arange(pl[b]) for b in range(B)])
        tok_rows_h = np.concatenate([np.arange(off[b] + pl[b], off[b + 1]) for b in range(B)])
        rpos_h = np.concatenate([np.concatenate([np.arange(p) * s, s * p + np.arange(T)]) for p in plens_h])
        idx = torch.from_numpy(np.concatenate([pre_src, pre_dst, tok_rows_h, rpos_h])).to(dev)
        n_pre, n_tok = len(pre_src), len(tok_rows_h)
        return (TrainPlan(seq_lens, dev), idx[:n_pre], idx[n_pre:2 * n_pre], idx[2 * n_pre:2 * n_pre + n_tok],
                idx[2 * n_pre + n_tok:].to(torch.int32), n_pre == B * P)

    plan, pre_src_d, pre_dst_d, tok_rows, rpos, all_prefix = dec.fast().layout(("train", tuple(plens_h), P, T, s),
                                                                               build)
    x = _PackRows.apply(prefix, emb, pre_src_d, pre_dst_d, tok_rows, all_prefix)
    cos, sin = dec.cos.float().contiguous(), dec.sin.float().contiguous()
    meta = {"cfg": cfg, "plan": plan, "rpos": rpos, "cos": cos, "sin": sin, "tok_rows": tok_rows}
    h = _DecoderStack.apply(x, meta, *decoder_params(dec))
    return _LMHead.apply(h, dec.lm_head.weight).view(B, T, -1)


def _train_logits_shared(model, frames, tokens_in, plens_h, G):
    """train_logits over groups of G windows that share their prefix: packed rows [each group's prefix rows |
    every member's token rows] (TrainPlan.shared)."""
    from .model import check_groups
    dec = model.decoder
    cfg = dec.cfg
    B, P = frames.shape[:2]
    T = tokens_in.shape[1]
    dev = frames.device
    pre_lens = check_groups(frames, plens_h, G)
    ng = len(pre_lens)
    proj = model.projector
    prefix = _Projector.apply(frames[::G].reshape(ng * P, -1).to(BF16).contiguous(), proj[0].weight, proj[0].bias,
                              proj[2].weight, proj[2].bias)                            # [B / G P, d] bf16
    emb = _TokenEmbed.apply(dec.embed.weight, tokens_in.to(dev).reshape(-1))          # [B T, d] fp32
    s = model.pos_scale

    def build():
        pl = np.asarray(pre_lens, dtype=np.int64)
        cu_pre = np.concatenate([[0], np.cumsum(pl)])
        n_pre = int(cu_pre[-1])
        pre_src = np.concatenate([g * P + np.arange(pl[g]) for g in range(ng)])
        pre_dst = np.arange(n_pre, dtype=np.int64)
        tok_rows_h = n_pre + np.arange(B * T, dtype=np.int64)
        member_pre = np.repeat(pl, G)
        rpos_h = np.concatenate([np.concatenate([np.arange(p) * s for p in pre_lens]),
                                 (s * member_pre[:, None] + np.arange(T)[None, :]).reshape(-1)])
        idx = torch.from_numpy(np.concatenate([pre_src, pre_dst, tok_rows_h, rpos_h])).to(dev)
        n_tok = B * T
        return (TrainPlan.shared(pre_lens, G, T, dev), idx[:n_pre], idx[n_pre:2 * n_pre],
                idx[2 * n_pre:2 * n_pre + n_tok], idx[2 * n_pre + n_tok:].to(torch.int32), n_pre == ng * P)

    plan, pre_src_d, pre_dst_d, tok_rows, rpos, all_prefix = dec.fast().layout(
        ("train_shared", tuple(pre_lens), G, P, T, s), build)
    x = _PackRows.apply(prefix, emb, pre_src_d, pre_dst_d, tok_rows, all_prefix)
    cos, sin = dec.cos.float().contiguous(), dec.sin.float().contiguous()
    meta = {"cfg": cfg, "plan": plan, "rpos": rpos, "cos": cos, "sin": sin, "tok_rows": tok_rows}
    h = _DecoderStack.apply(x, meta, *decoder_params(dec))
    return _LMHead.apply(h, dec.lm_head.weight).view(B, T, -1)


class HipAdamW:
    """AdamW over flat fp32 buffers with the global-norm gradient clip folded into the step, all on the device
    (torch.optim.AdamW(betas=(0.9, 0.95), weight_decay=0, fused=True) + clip_grad_norm_ of scripts/gspo.py:368,
    492-493). The parameters become views of one flat buffer, so the step is one launch."""

    def __init__(self, params: Sequence[torch.Tensor], lr=1e-5, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0,
                 max_grad_norm: Optional[float] = 1.0):
        self.params = [p for p in params if p.requires_grad]
        assert self.params and all(p.dtype == torch.float32 and p.is_cuda for p in self.params), \
            "HipAdamW: fp32 device parameters"
        n = sum(p.numel() for p in self.params)
        dev = self.params[0].device
        self.flat = torch.empty(n, dtype=torch.float32, device=dev)
        self.grad = torch.zeros(n, dtype=torch.float32, device=dev)
        self.m = torch.zeros(n, dtype=torch.float32, device=dev)
        self.v = torch.zeros(n, dtype=torch.float32, device=dev)
        self.slices = []
        o = 0
        for p in self.params:
            k = p.numel()
            self.flat[o:o + k].copy_(p.data.reshape(-1))
            p.data = self.flat[o:o + k].view_as(p)
            self.slices.append((o, k))
            o += k
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.max_grad_norm = max_grad_norm
        self.step_count = 0
        self.last_norm = None
        self.zero_grad()

    def zero_grad(self):
        """Zero the flat gradient buffer and make every parameter's .grad a view of its slice, so backward
        accumulates into the buffer in place (no gather before the step)."""
        self.grad.zero_()
        for p, (o, k) in zip(self.params, self.slices):
            p.grad = self.grad[o:o + k].view_as(p)

    def step(self):
        """Clip by the global norm and AdamW-update. A gradient that is not the bound view (set by the caller,
        or left None) is copied in (None counts as zero)."""
        for p, (o, k) in zip(self.params, self.slices):
            view = self.grad[o:o + k]
            if p.grad is None:
                view.zero_()
            elif p.grad.data_ptr() != view.data_ptr():
                view.copy_(p.grad.reshape(-1))
        coef = None
        if self.max_grad_norm is not None:
            coef = ops.grad_norm_clip(self.grad, self.max_grad_norm)
            self.last_norm = coef
        self.step_count += 1
        ops.adamw(self.flat, self.grad, self.m, self.v, self.lr, self.betas, self.eps, self.weight_decay,
                  self.step_count, coef=coef)


def token_logprobs_train(model, frames, plens, seqs, ended, group_size=1):
    """Differentiable token_logprobs (scripts/gspo.py:340-353): (logits [B, T, V] bf16, targets, mask).
    group_size: as train_logits."""
    from .gspo import sampled_mask
    tokens_in, targets, _ = model.batch(seqs, pad_to=128)
    dev = frames.device
    tokens_in, targets = tokens_in.to(dev), targets.to(dev)
    logits = train_logits(model, frames, tokens_in, plens, group_size)
    mask = sampled_mask(targets, seqs, ended, model.tokenizer.k)
    return logits, targets, mask


def gspo_loss(model, frames, plens, seqs, ended, old_lp, n_bases, adv, eps_lo=4e-4, eps_hi=4e-4, inv_n=None):
    """The micro-batch's GSPO loss (scripts/gspo.py:471-477) with its autograd graph into the model:
    returns (loss, s [B], pg [B], lp [B, T]). old_lp [B, T] fp32 (masked positions ignored), n_bases [B], adv [B]."""
    logits, targets, mask = token_logprobs_train(model, frames, plens, seqs, ended)
    return sequence_ratio_loss(logits, targets, mask, old_lp, n_bases, adv, eps_lo, eps_hi, inv_n)


def frame_loss(model, frames, seqs, weights=None, plens=None):
    """Differentiable weighted-mean token cross-entropy of teacher-forced label sequences, the SFT term of the
    GSPO update (Basecaller.frame_loss / weighted_loss / token_metrics, viktor/model.py:153-177, 201-203;
    called at scripts/gspo.py:482-484): sum(ce * w) / sum(w) over the targets (PAD ignored)."""
    dev = frames.device
    tokens_in, targets, w = (t.to(dev) for t in model.batch(seqs, weights))
    logits = train_logits(model, frames, tokens_in, plens)
    ce = torch.nn.functional.cross_entropy(logits.flatten(0, 1).float(), targets.flatten(), ignore_index=0,
                                           reduction="none").view_as(targets)
    return (ce * w).sum() / w.sum()


def _old_row(vals, mask_row):
    """Scatter one sequence's per-token values (its sampled positions, in order) into a row of mask_row's shape."""
    row = torch.zeros(mask_row.shape, dtype=torch.float32, device=mask_row.device)
    row[mask_row] = vals
    return row


def gspo_update(model, opt: HipAdamW, frames, plens, calls, ended, reward, G, updates=2, micro=32, eps=4e-4,
                std_floor=0.003, labels=None, weights=None, sft_weight=0.0):
    """The GSPO policy update of one rollout (scripts/gspo.py:446-493 on one GPU, without the all-reduce):
    advantages over each window's G calls (live windows: reward std > 1e-6); pi_old of every live call before
    any update; then `updates` optimiser steps, step u over the calls of windows b % updates == u: micro-batches
    of the sequence-ratio loss summed / len(mine), plus sft_weight x the weighted cross-entropy of the windows'
    labels (when given), backward, clip + AdamW (opt). frames [windows, P, d_enc], plens [windows]; calls /
    ended: the G calls of window b at b * G .. b * G + G - 1; reward [windows, G]. Returns the step statistics
    (pg, ce, clip, ratio, n as the reference's, and each step's gradient norm)."""
    from .gspo import advantages
    import numpy as np
    B = frames.shape[0]
    adv, live = advantages(np.asarray(reward, dtype=np.float64).reshape(B, G), std_floor=std_floor)
    seqs = [(b, j) for b in live for j in range(G)]
    n_bases = {bj: max(len(calls[bj[0] * G + bj[1]]), 1) for bj in seqs}
    dev = frames.device

    def batch_of(mb):
        ix = torch.tensor([b for b, _ in mb], device=dev)
        return frames[ix], plens[ix], [calls[b * G + j] for b, j in mb], [ended[b * G + j] for b, j in mb]

    def group_of(mb):
        """G when the micro-batch is whole groups (each window's G calls in a row, as `seqs` lists them): its
        windows' prefixes then run once (train_logits(group_size=G)); 1 otherwise."""
        whole = len(mb) % G == 0 and all(mb[i][0] == mb[i - i % G][0] and mb[i][1] == i % G for i in range(len(mb)))
        return G if G > 1 and whole else 1

    old = {}
    with torch.no_grad():  # pi_old through the same forward as the update's (scripts/gspo.py:455-462)
        for i in range(0, len(seqs), micro):
            mb = seqs[i:i + micro]
            logits, targets, m = token_logprobs_train(model, *batch_of(mb), group_size=group_of(mb))
            lp = ops.gspo_score(logits.contiguous(), targets.clamp(min=0).contiguous())["lp"]
            for k, bj in enumerate(mb):
                old[bj] = lp[k][m[k]].clone()
    stats = {"pg": 0.0, "ce": 0.0, "clip": 0.0, "ratio": 0.0, "n": 0, "grad_norm": []}
    for u in range(updates):
        mine = [bj for bj in seqs if bj[0] % updates == u]
        wins = [b for b in range(B) if b % updates == u]
        opt.zero_grad()
        for i in range(0, len(mine), micro):
            mb = mine[i:i + micro]
            logits, targets, mask = token_logprobs_train(model, *batch_of(mb), group_size=group_of(mb))
            old_lp = torch.stack([_old_row(old[bj], mask[k]) for k, bj in enumerate(mb)])
            nb = torch.tensor([float(n_bases[bj]) for bj in mb], device=dev)
            a = torch.tensor([adv[b, j] for b, j in mb], device=dev, dtype=torch.float32)
            loss, s, pg, _ = sequence_ratio_loss(logits, targets, mask, old_lp, nb, a, eps, eps, 1.0 / len(mine))
            loss.backward()
            stats["pg"] += float(pg.sum())
            stats["n"] += len(mb)
            stats["clip"] += float(((s - 1).abs() > eps).sum())
            stats["ratio"] += float((s - 1).abs().sum())
        if sft_weight and labels is not None:
            for i in range(0, len(wins), micro):
                wb = wins[i:i + micro]
                ix = torch.tensor(wb, device=dev)
                ce = frame_loss(model, frames[ix], [labels[b] for b in wb],
                                None if weights is None else [weights[b] for b in wb], plens=plens[ix])
                (sft_weight * ce * len(wb) / len(wins)).backward()
                stats["ce"] += float(ce) * len(wb)
        opt.step()
        stats["grad_norm"].append(None if opt.last_norm is None else float(opt.last_norm[0]))
    return stats
