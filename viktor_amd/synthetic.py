"""Seeded synthetic models and inputs for the rollout / scoring workloads (no checkpoints or datasets).

Weights are drawn on the CPU in fp32 from torch.Generator(seed), parameter by parameter in sorted-name
order: Linear weights N(0, 1) / sqrt(fan_in), embeddings N(0, 1), RMSNorm weights 1 (+ norm_jitter *
N(0, 1) when asked, which tests use so a dropped norm weight shows), projector biases 0 (+ bias_jitter).
The same fp32 tensors are kept for CPU checks and cast to bf16 for the GPU.

Workloads (sizes as named by the benchmark configurations):
  rollout:  64 prefixes x group 8 = 512 sequences, 2048 frames of N(0, 1) 512-d features each,
            uniforms [512, 1024] U[0, 1), rewards Beta(8, 2) per sequence;
  varlen:   1024 sequences with prefix lengths uniform in [1200, 2048];
  scoring:  512 sequences x response lengths uniform in [700, 1024].
"""

import math

import numpy as np
import torch

from .decoder import DecoderConfig
from .model import Basecaller
from .tokenizer import KmerTokenizer


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(int(seed))
    return g


@torch.no_grad()
def init_params(module, seed, norm_jitter=0.0, bias_jitter=0.0):
    """Deterministic fp32 init of every parameter of `module` (see the module docstring)."""
    g = _gen(seed)
    params = dict(module.named_parameters())
    for name in sorted(params):
        p = params[name]
        shape = tuple(p.shape)
        if name.endswith("embed.weight"):
            v = torch.randn(shape, generator=g)
        elif p.dim() == 2:  # Linear weight [out, in]
            v = torch.randn(shape, generator=g) / math.sqrt(shape[1])
        elif name.endswith("bias"):
            v = torch.randn(shape, generator=g) * bias_jitter
        else:  # RMSNorm weight
            v = 1.0 + torch.randn(shape, generator=g) * norm_jitter
        p.copy_(v.to(p.dtype))


def make_model(k=1, n_layers=8, seed=0, rope_theta=1e6, d_enc=512, norm_jitter=0.0, bias_jitter=0.0,
               max_seq_len=4096, **cfg_kw):
    """fp32 CPU Basecaller (projector + decoder) of the benchmark architecture with seeded weights."""
    tok = KmerTokenizer(k)
    cfg = DecoderConfig(vocab_size=tok.vocab_size, n_layers=n_layers, rope_theta=rope_theta, max_seq_len=max_seq_len,
                        **cfg_kw)
    m = Basecaller(None, tok, cfg, d_enc=d_enc)
    init_params(m, seed, norm_jitter=norm_jitter, bias_jitter=bias_jitter)
    return m.eval()


def frames(n, P, d_enc=512, seed=0):
    """[n, P, d_enc] N(0, 1) encoder features (CPU fp32)."""
    return torch.randn(n, P, d_enc, generator=_gen(seed))


def uniforms(B, T, seed=0):
    """[B, T] U[0, 1) fp32 (CPU)."""
    return torch.rand(B, T, generator=_gen(seed))


def rollout_inputs(prefixes=64, group=8, P=2048, new_tokens=1024, d_enc=512, seed=0):
    """GSPO rollout inputs: frames [prefixes * group, P, d_enc] (each prefix repeated group times, as the
    reference repeats a window per group member), plens, uniforms, rewards Beta(8, 2) [prefixes, group]."""
    f = frames(prefixes, P, d_enc, seed).repeat_interleave(group, 0)
    B = prefixes * group
    plens = torch.full((B,), P, dtype=torch.long)
    u = uniforms(B, new_tokens, seed + 1)
    rng = np.random.default_rng(seed + 2)
    rewards = rng.beta(8.0, 2.0, size=(prefixes, group))
    return f, plens, u, rewards


def varlen_lengths(B=1024, lo=1200, hi=2048, seed=0):
    """Prefix lengths uniform in [lo, hi] (inclusive)."""
    return torch.randint(lo, hi + 1, (B,), generator=_gen(seed))


def scoring_inputs(B=512, lo=700, hi=1024, k=1, seed=0):
    """Response token sequences for teacher-forced scoring: L_b ~ U[lo, hi] tokens including the final EOS,
    bases uniform over ACGT. Returns (base strings, ended flags)."""
    g = _gen(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g)
    seqs = []
    for L in lens.tolist():
        n_bases = (L - 1) * k
        idx = torch.randint(0, 4, (n_bases,), generator=g)
        seqs.append("".join("ACGT"[i] for i in idx.tolist()))
    return seqs, [True] * B


# ---- encoder (frames producer) -----------------------------------------------------------------------
# The layer shapes of Dorado's SUP v5 transformer encoder (5 convolutions of total stride 12, 18 DeepNorm
# layers of d_model 512, 8 heads, SwiGLU 2048, attention window (127, 128)) in the config layout of
# viktor/encoder.py:115-147; 12288-sample chunks.
SUP_ENCODER_CFG = {
    "model": {"encoder": {
        "conv": {"sublayers": [
            {"type": "convolution", "insize": 1, "size": 64, "winlen": 5, "stride": 1, "padding": 2, "bias": True},
            {"type": "convolution", "insize": 64, "size": 64, "winlen": 5, "stride": 1, "padding": 2, "bias": True},
            {"type": "convolution", "insize": 64, "size": 128, "winlen": 9, "stride": 3, "padding": 4, "bias": True},
            {"type": "convolution", "insize": 128, "size": 128, "winlen": 9, "stride": 2, "padding": 4, "bias": True},
            {"type": "convolution", "insize": 128, "size": 512, "winlen": 5, "stride": 2, "padding": 2, "bias": True},
            {"type": "permute", "dims": [0, 2, 1]}]},
        "transformer_encoder": {"depth": 18, "layer": {
            "d_model": 512, "nhead": 8, "dim_feedforward": 2048, "deepnorm_alpha": 2.4494897,
            "attn_window": [127, 128]}}}},
    "basecaller": {"chunksize": 12288, "overlap": 600},
    "standardisation": {"mean": 93.6, "stdev": 23.3},
}


def encoder_state_dict(cfg=SUP_ENCODER_CFG, seed=0):
    """Seeded fp32 encoder weights under the reference module's names: conv / Linear weights
    N(0, 1) / sqrt(fan_in), biases 0.1 N(0, 1), RMSNorm weights 1 + 0.1 N(0, 1)."""
    g = _gen(seed)
    sd = {}
    convs = [l for l in cfg["model"]["encoder"]["conv"]["sublayers"] if l["type"] == "convolution"]
    for i, l in enumerate(convs):
        sd[f"conv.{i}.conv.weight"] = torch.randn(l["size"], l["insize"], l["winlen"], generator=g) / math.sqrt(
            l["insize"] * l["winlen"])
        sd[f"conv.{i}.conv.bias"] = 0.1 * torch.randn(l["size"], generator=g)
    tx = cfg["model"]["encoder"]["transformer_encoder"]
    C, F = tx["layer"]["d_model"], tx["layer"]["dim_feedforward"]
    for j in range(tx["depth"]):
        pre = f"transformer_encoder.{j}."
        sd[pre + "self_attn.Wqkv.weight"] = torch.randn(3 * C, C, generator=g) / math.sqrt(C)
        sd[pre + "self_attn.out_proj.weight"] = torch.randn(C, C, generator=g) / math.sqrt(C)
        sd[pre + "self_attn.out_proj.bias"] = 0.1 * torch.randn(C, generator=g)
        sd[pre + "ff.fc1.weight"] = torch.randn(2 * F, C, generator=g) / math.sqrt(C)
        sd[pre + "ff.fc2.weight"] = torch.randn(C, F, generator=g) / math.sqrt(F)
        sd[pre + "norm1.weight"] = 1 + 0.1 * torch.randn(C, generator=g)
        sd[pre + "norm2.weight"] = 1 + 0.1 * torch.randn(C, generator=g)
    return sd


def signal(n_samples, seed=0):
    """Standardised synthetic signal: N(0, 1) fp32 samples."""
    return torch.randn(int(n_samples), generator=_gen(seed))
