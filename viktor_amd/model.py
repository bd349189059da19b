"""Basecaller subset on the rollout-and-scoring path: per-frame projector + decoder-only LM + tokenizer.

Reference: viktor/model.py:27-131. A Basecaller takes encoder frames [B, P, d_enc] directly; `encoder` may be
None (then `d_enc` gives the frame width) or the HIP encoder (viktor_amd.encoder.DoradoEncoder), which
`encode` runs.
Teacher-forced logits run on the HIP kernels: every window is packed as [its plens[b] frames | tokens]
(the causal decoder never reads the padding the reference appends after them), the decoder runs over the
packed tokens with its last layer kept for the token rows only, and the LM head gives bf16 logits. They keep
the rounding points of the reference's scoring call, which runs under torch.autocast bf16 (an fp32 residual
stream; see FastDecoder.teacher_forced).
"""

from typing import Optional

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from ._lib import require_device
from .decoder import Decoder, DecoderConfig
from . import hip_ops as ops
from .fast_decoder import PrefillPlan, SharedPrefixPlan
from .tokenizer import PAD, KmerTokenizer, get_tokenizer

BF16 = torch.bfloat16


def check_groups(frames, plens_h, G):
    """The prefix lengths of the groups of G consecutive windows (ValueError unless B is whole groups and each
    group's windows have one prefix length and the same real frames, bit for bit)."""
    B, P = frames.shape[:2]
    if B % G:
        raise ValueError(f"group_size={G}: {B} windows are not whole groups")
    pre_lens = plens_h[::G]
    if any(plens_h[b] != pre_lens[b // G] for b in range(B)):
        raise ValueError(f"group_size={G}: the windows of a group must have the same prefix length")
    if all(p == P for p in plens_h) and frames.is_contiguous() and (frames[0].numel() * frames.element_size()) % 16 == 0:
        same = ops.group_rows_equal(frames, G)
    else:
        same = all(torch.equal(frames[b:b + G, :p], frames[b:b + 1, :p].expand(G, -1, -1))
                   for b, p in zip(range(0, B, G), pre_lens))
    if not same:
        raise ValueError(f"group_size={G}: the windows of a group must share their prefix frames")
    return pre_lens


class Basecaller(nn.Module):
    def __init__(self, encoder, tokenizer: KmerTokenizer, cfg: Optional[DecoderConfig] = None, d_enc: int = 512):
        super().__init__()
        self.encoder = encoder
        self.tokenizer = tokenizer
        self.cfg = cfg or DecoderConfig(vocab_size=tokenizer.vocab_size)
        d = self.cfg.d_model
        self.d_enc = getattr(encoder, "d_model", d_enc) if encoder is not None else d_enc
        # one prefix token per encoder frame (reference: viktor/model.py:34-35)
        self.projector = nn.Sequential(nn.Linear(self.d_enc, d), nn.GELU(), nn.Linear(d, d))
        self.decoder = Decoder(self.cfg)
        # RoPE position of prefix frame j = j * pos_scale; tokens follow at pos_scale * (real frames) + i
        self.pos_scale = 1

    @classmethod
    def from_args(cls, encoder, args: dict, d_enc: int = 512):
        """The model of a training run's args: tokenizer and decoder depth (reference: viktor/model.py:42-48)."""
        tok = get_tokenizer(args.get("tokenizer", "base"))
        m = cls(encoder, tok, DecoderConfig(vocab_size=tok.vocab_size, n_layers=args.get("layers", 8)), d_enc=d_enc)
        m.pos_scale = args.get("prefix_pos_scale", 1)
        return m

    def project(self, frames):
        """Projector in bf16 (autocast for fp32 weights, as the reference's training path runs it)."""
        with torch.autocast("cuda", dtype=BF16, enabled=self.projector[0].weight.dtype != BF16):
            return self.projector(frames.to(self.projector[0].weight.dtype)).to(BF16)

    def rope_positions(self, x, P, plens=None):
        """[B, P + T] RoPE positions of a [frames | tokens] window (None at pos_scale 1: the sequence index).
        Reference: viktor/model.py:62-69."""
        if self.pos_scale == 1:
            return None
        B, L = x.shape[:2]
        pos = torch.arange(L, device=x.device).expand(B, -1)
        n = torch.full((B, 1), P, device=x.device) if plens is None else plens[:, None]
        return torch.where(pos < n, pos * self.pos_scale, pos + (self.pos_scale - 1) * n)

    @torch.no_grad()
    def encode(self, sig, valid):
        """Decoder input as at inference (viktor/model.py:89-117): encoder frames [B, P, d_enc] (P = frames of a
        full window) and the real frames per window [B]. sig [B, 1, S]; valid: real samples per window. A full
        window is encoded whole, a short one at its repeat-padded length (a multiple of the granularity, as
        encoder.encode_chunks) keeping ceil(valid / stride) frames, the rest zero. All windows go through one
        forward_varlen call (chunks are encoded independently, so this equals encoding them apart)."""
        enc = self.encoder
        if enc is None:
            raise ValueError("Basecaller.encode needs an encoder")
        B, S = sig.shape[0], sig.shape[-1]
        st, g = enc.stride, enc.granularity
        valid = [int(v) for v in (valid.tolist() if torch.is_tensor(valid) else valid)]
        if not all(0 < v <= S for v in valid):
            raise ValueError("Basecaller.encode: every window needs 0 < valid <= its length")
        lens = [S if v == S else min(-(-v // g) * g, S) for v in valid]
        flat = torch.cat([sig[b, 0, :n] for b, n in enumerate(lens)])
        out = enc.forward_varlen(flat, lens)
        P = S // st
        plens = np.array([-(-v // st) for v in valid], dtype=np.int64)
        starts = np.concatenate([[0], np.cumsum([n // st for n in lens])[:-1]])
        src = np.concatenate([np.arange(s0, s0 + k) for s0, k in zip(starts, plens)])
        dst = np.concatenate([np.arange(b * P, b * P + k) for b, k in enumerate(plens)])
        frames = out.new_zeros(B * P, out.shape[-1])
        frames.index_copy_(0, torch.from_numpy(dst).to(out.device), out.index_select(0, torch.from_numpy(src).to(out.device)))
        return frames.view(B, P, -1), torch.from_numpy(plens).to(out.device)

    def logits(self, frames, tokens_in, plens=None, group_size=1):
        """Teacher forcing from encoder frames [B, P, d_enc]: bf16 logits [B, T, vocab] of every token
        position. plens [B]: real prefix frames per window (default P). Reference: viktor/model.py:55-60, with
        the rounding points it has where scripts/gspo.py:345-347 calls it, under torch.autocast bf16: the
        projector's bf16 output and the token embeddings gathered into an fp32 residual stream
        (viktor/model.py:81-84; fp32 embedding rows from fp32 weights), the decoder on that fp32 stream
        (FastDecoder.teacher_forced) and the LM head as a bf16 product.
        group_size = G > 1: consecutive groups of G windows carry the same prefix (a GSPO rollout's repeated
        windows, scripts/gspo.py:444; checked on the device, ValueError otherwise), which then runs once per group
        (see hidden())."""
        return self.decoder.head(self.hidden(frames, tokens_in, plens, group_size)).view(
            frames.shape[0], tokens_in.shape[1], -1)

    def hidden(self, frames, tokens_in, plens=None, group_size=1):
        """The final-normed hidden state of every token position [B T, d] bf16 (the LM head's operand) of the
        teacher-forced forward that logits() runs. group_size = G > 1: the projector and the decoder run each
        group's prefix once (FastDecoder.teacher_forced_shared) and its members' token rows attend to that
        prefix's keys; the token rows' results are those of the unshared forward (the same arithmetic per row)."""
        require_device(frames, "Basecaller.hidden")
        B, P = frames.shape[:2]
        T = tokens_in.shape[1]
        dev = frames.device
        plens_h = [P] * B if plens is None else [int(p) for p in plens.tolist()]
        assert all(0 < p <= P for p in plens_h), "plens outside 1..P"
        if int(group_size) > 1:
            return self._hidden_shared(frames, tokens_in, plens_h, int(group_size))
        prefix = self.project(frames)                                       # [B, P, d] bf16
        fast = self.decoder.fast()
        emb = fast.w32(self.decoder.embed.weight)[tokens_in.to(dev)]        # [B, T, d] fp32
        s = self.pos_scale

        def build():  # the packing plan, the window layout's row indices and each row's (rotary) position
            seq_lens = [p + T for p in plens_h]
            plan = PrefillPlan(seq_lens, dev, keep=[T] * B)
            pl = np.asarray(plens_h, dtype=np.int64)
            cu = np.asarray(plan.cu[:-1], dtype=np.int64)
            pre_dst = np.concatenate([cu[b] + np.arange(pl[b]) for b in range(B)])
            pre_src = np.concatenate([b * P + np.arange(pl[b]) for b in range(B)])
            tok_dst = (cu + pl)[:, None] + np.arange(T)[None, :]
            pos = np.concatenate([np.arange(n) for n in seq_lens])
            parts = [pre_dst, pre_src, tok_dst.reshape(-1), pos]
            if s != 1:
                parts.append(np.concatenate([np.concatenate([np.arange(p) * s, s * p + np.arange(T)])
                                             for p in plens_h]))
            idx = torch.from_numpy(np.concatenate(parts)).to(dev)  # one host-to-device copy
            o = np.cumsum([0] + [len(a) for a in parts])
            sl = [idx[o[i]:o[i + 1]] for i in range(len(parts))]
            rpos = sl[4].to(torch.int32) if s != 1 else None
            return plan, sl[0], sl[1], sl[2], sl[3].to(torch.int32), rpos

        plan, pre_dst, pre_src, tok_dst, pos, rpos = fast.layout(("tf", tuple(plens_h), P, T, s), build)
        # packed rows: window b = [prefix[b, :plens[b]] | emb[b]]
        x = torch.empty(plan.total, prefix.shape[-1], dtype=torch.float32, device=dev)
        if all(p == P for p in plens_h):  # full windows: two strided copies
            xv = x.view(B, P + T, -1)
            xv[:, :P] = prefix
            xv[:, P:] = emb
        else:
            x[pre_dst] = prefix.reshape(B * P, -1)[pre_src].float()
            x[tok_dst] = emb.reshape(B * T, -1)
        return fast.teacher_forced(x, pos, plan, rope_pos=rpos)            # [B * T, d] bf16

    def _hidden_shared(self, frames, tokens_in, plens_h, G):
        """hidden() over groups of G windows that share their prefix: each group's frames are projected and run
        through the decoder once, as its members' common prefix."""
        B, P = frames.shape[:2]
        T = tokens_in.shape[1]
        dev = frames.device
        pre_lens = check_groups(frames, plens_h, G)
        d = self.cfg.d_model
        prefix = self.project(frames[::G].contiguous())                    # [B / G, P, d] bf16, one per group
        if all(p == P for p in pre_lens):
            x_pre = prefix.reshape(-1, d).float()
        else:
            x_pre = torch.cat([prefix[g, :p] for g, p in enumerate(pre_lens)]).float()
        fast = self.decoder.fast()
        x_tok = fast.w32(self.decoder.embed.weight)[tokens_in.to(dev).reshape(-1)]  # [B T, d] fp32
        s = self.pos_scale

        def build():
            plan = SharedPrefixPlan(pre_lens, G, T, self.cfg.n_kv_heads * self.cfg.head_dim, dev)
            rope_pre = rope_tok = None
            if s != 1:
                rope_pre = torch.from_numpy(np.concatenate([np.arange(p) * s for p in pre_lens]).astype(np.int32)).to(dev)
                rope_tok = torch.from_numpy((s * np.repeat(np.asarray(pre_lens), G)[:, None] +
                                             np.arange(T)[None, :]).reshape(-1).astype(np.int32)).to(dev)
            return plan, rope_pre, rope_tok

        plan, rope_pre, rope_tok = fast.layout(("shared", tuple(pre_lens), G, T, s), build)
        return fast.teacher_forced_shared(x_pre, x_tok, plan, rope_pre, rope_tok)  # [B * T, d] bf16

    def batch(self, seqs, weights=None, pad_to=1):
        """CPU teacher-forcing tensors: tokens_in, targets [B, T] and target weights [B, T], T padded up to a
        multiple of pad_to. weights: one array per sequence, a weight per base; a k-mer token weighs its
        lowest base weight (a masked base masks its token), EOS 1; without weights every target (EOS
        included) weighs 1. Reference: viktor/model.py:119-145 (alignment centres, an SFT attention-probe
        target, are not part of this path)."""
        tokens_in, targets, _ = self.tokenizer.batch(seqs)
        T = -(-targets.shape[1] // pad_to) * pad_to
        tokens_in = F.pad(tokens_in, (0, T - tokens_in.shape[1]), value=PAD)
        targets = F.pad(targets, (0, T - targets.shape[1]), value=PAD)
        if weights is None:
            return tokens_in, targets, (targets != PAD).float()
        k = self.tokenizer.k
        w = torch.zeros(targets.shape)
        for b, wb in enumerate(weights):
            wb = np.asarray(wb, dtype=np.float32)
            pad = np.full(-(-len(wb) // k) * k, np.inf, np.float32)
            pad[:len(wb)] = wb
            wt = pad.reshape(-1, k).min(1)
            w[b, :len(wt)] = torch.from_numpy(wt)
            w[b, len(wt)] = 1.0  # EOS
        return tokens_in, targets, w
