"""GSPO rollout and scoring surface (the hot functions of scripts/gspo.py) on the HIP path.

  engine(inf, batch, temperature)                 scripts/gspo.py:129-131
  decode(engine, frames, plens, tokenizer)        scripts/gspo.py:134-139
  token_logprobs(model, frames, plens, seqs, ended)  scripts/gspo.py:340-353
  bf16_copy(model), sync(inf, model)              scripts/gspo.py:113-126
  advantages(reward, std_floor | eps)             scripts/gspo.py:446-450
  sequence_ratio_loss(...)                        scripts/gspo.py:451, 474-477 (one kernel, + dL/dlogits)

Rewards (edit distance against labels), data loading, the optimiser loop and the gradient all-reduce of
the reference driver are outside this path.
"""

import copy

import numpy as np
import torch

from . import hip_ops as ops
from .engine import DecodeEngine
from .model import Basecaller
from .tokenizer import EOS, PAD

STEP_BASES = 2048  # rollout length cap in bases (reference: scripts/gspo.py:62)


def bf16_copy(model):
    """Inference model with bf16 copies of the projector and decoder (reference: scripts/gspo.py:113-118)."""
    inf = Basecaller(model.encoder, model.tokenizer, model.cfg, d_enc=model.d_enc)
    inf.projector = copy.deepcopy(model.projector).to(torch.bfloat16).eval()
    inf.decoder = copy.deepcopy(model.decoder).to(torch.bfloat16).eval()
    inf.decoder._fast = None
    inf.pos_scale = model.pos_scale
    return inf


@torch.no_grad()
def sync(inf, model):
    """Copy trained weights into the inference copy in place, so captured graphs keep their pointers
    (reference: scripts/gspo.py:121-126)."""
    for dst, src in zip(list(inf.projector.parameters()) + list(inf.decoder.parameters()),
                        list(model.projector.parameters()) + list(model.decoder.parameters())):
        dst.copy_(src)


def engine(inf, batch, temperature=0.0, max_frames=None, max_new_tokens=None, **kw):
    """Rollout engine: STEP_BASES // k output tokens; prefix capacity from the encoder (chunksize // stride)
    when the model has one, else max_frames. Reference: scripts/gspo.py:129-131."""
    if max_frames is None:
        enc = inf.encoder
        if enc is None:
            raise ValueError("engine: the model has no encoder; pass max_frames")
        max_frames = enc.chunksize // enc.stride
    max_new = STEP_BASES // inf.tokenizer.k if max_new_tokens is None else max_new_tokens
    return DecodeEngine(inf, batch, max_new, max_frames, temperature=temperature, **kw)


@torch.no_grad()
def decode(engine, frames, plens, tokenizer, steps=None):
    """frames [N, P, d_enc] and real frames per window [N] (N = engine batch) -> (calls, ended).
    Reference: scripts/gspo.py:134-139."""
    plens = plens.tolist()
    toks = engine.generate(torch.cat([f[:n] for f, n in zip(frames, plens)]), plens, steps).cpu()
    return [tokenizer.decode(t) for t in toks], (toks == EOS).any(1).tolist()


def sampled_mask(targets, seqs, ended, k):
    """Mask of the sampled tokens: targets != PAD, minus the EOS target when the call did not end or the
    engine forced it after a tail token (len % k != 0). Reference: scripts/gspo.py:349-352."""
    mask = targets != PAD
    for b, (s, e) in enumerate(zip(seqs, ended)):
        if not e or len(s) % k:
            mask[b, -(-len(s) // k)] = False
    return mask


def token_logprobs(model, frames, plens, seqs, ended, group_size=1):
    """Teacher-forced log pi of each call's tokens [B, T] (fp32) and the mask of its sampled tokens.
    Reference: scripts/gspo.py:340-353 (T padded to a multiple of 128). group_size = G > 1: the rollout's G
    samples of each window sit in consecutive rows and share its frames (scripts/gspo.py:444), so each window's
    prefix runs once (Basecaller.logits); the log-probs are those of the unshared forward."""
    tokens_in, targets, _ = model.batch(seqs, pad_to=128)
    dev = frames.device
    tokens_in, targets = tokens_in.to(dev), targets.to(dev)
    logits = model.logits(frames, tokens_in, plens, group_size=group_size)
    lp = ops.gspo_score(logits.contiguous(), targets.clamp(min=0).contiguous())["lp"]
    mask = sampled_mask(targets, seqs, ended, model.tokenizer.k)
    return lp, mask


def advantages(reward, std_floor=0.003, eps=None):
    """Group advantages of rewards [groups, G]: (r - mean) / max(std, std_floor) with live groups
    std > 1e-6 (reference rule, scripts/gspo.py:447-450), or (r - mean) / (std + eps) when eps is given.
    Host numpy in float64 as the reference; see hip_ops.group_advantage for the device kernel."""
    r = np.asarray(reward, dtype=np.float64)
    std = r.std(1)
    live = np.nonzero(std > 1e-6)[0]
    den = (std + eps) if eps is not None else np.maximum(std, std_floor)
    return (r - r.mean(1, keepdims=True)) / den[:, None], live


class _GspoLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets, mask, old_lp, n_bases, adv, eps_lo, eps_hi, inv_n):
        res = ops.gspo_score(logits.detach().contiguous(), targets, mask, old_lp, n_bases, adv, eps_lo, eps_hi, inv_n,
                             grad=logits.requires_grad)
        ctx.save_for_backward(res.get("dlogits", torch.empty(0, device=logits.device)))
        ctx.logits_dtype = logits.dtype
        # the kernel's gradient is that of the loss only: s, pg and lp are outputs to read, not to backpropagate
        # through (a backward from them raises instead of returning zeros)
        ctx.mark_non_differentiable(res["s"], res["pg"], res["lp"])
        return res["loss"], res["s"], res["pg"], res["lp"]

    @staticmethod
    def backward(ctx, g_loss, g_s, g_pg, g_lp):
        (dl,) = ctx.saved_tensors
        return (dl * g_loss).to(ctx.logits_dtype), None, None, None, None, None, None, None, None


def sequence_ratio_loss(logits, targets, mask, old_lp, n_bases, adv, eps_lo=4e-4, eps_hi=4e-4, inv_n=None):
    """GSPO objective of B sequences in one kernel: s = exp(sum_mask(lp - old) / n_bases), pg =
    -min(s A, clamp(s, 1 - eps_lo, 1 + eps_hi) A), loss = inv_n * sum(pg) (inv_n = 1 / B by default).
    Differentiable w.r.t. logits (the gradient is produced by the same kernel). Returns (loss, s, pg, lp).
    Reference: scripts/gspo.py:474-477."""
    B = logits.shape[0]
    inv = 1.0 / B if inv_n is None else inv_n
    return _GspoLoss.apply(logits, targets.clamp(min=0).contiguous(), mask, old_lp.contiguous(), n_bases, adv,
                           eps_lo, eps_hi, inv)
