"""CPU restatement of the reference's Dorado SUP encoder -- TEST INFRASTRUCTURE, not product code.

Restates viktor/encoder.py:43-192 (conv stack + sliding-window DeepNorm transformer, forward_varlen,
encode_chunks) in PyTorch on the CPU, in two numerics modes:
  "fp32" -- the reference module's fp32 semantics (F.conv1d, banded softmax attention, nn.RMSNorm);
  "bf16" -- the rounding points of the HIP encoder: bf16 weights and activations between ops, fp32 inside
            each op (conv + bias rounded, then SiLU rounded; q/k rotated and rounded; attention output
            rounded; out_proj + bias rounded; alpha * x rounded; the residual sum rounded; RMSNorm output
            rounded; SwiGLU with bf16 gate, silu and product). The first convolution reads the fp32 signal
            with fp32 weights.

How it is pinned (tests/test_oracle.py): the convolution against a direct sum, the banded attention
against a brute-force loop and against its closed-form special cases (window (0, 0) returns v; a window
as wide as the chunk is unmasked attention), the rotation against complex multiplication, and the
reference's own encoder tests (tests/test_viktor.py:71-104: a packed batch equals each chunk alone;
encode_chunks keeps ceil(valid / stride) frames per chunk, [128, 33] for its tiny config).
"""

import math

import numpy as np
import torch
import torch.nn.functional as F

from .reference import apply_rope, bf, rope_tables

# The layer shapes of Dorado's SUP v5 transformer model (5 convolutions, total stride 12, 18 layers of
# d_model 512, 8 heads, SwiGLU 2048, window (127, 128)), in the config layout viktor/encoder.py:115-147
# reads. Weights are synthetic.
SUP_CFG = {
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

# tests/test_viktor.py:13-22 (the reference's tiny encoder config)
TINY_CFG = {
    "model": {"encoder": {
        "conv": {"sublayers": [
            {"type": "convolution", "insize": 1, "size": 16, "winlen": 5, "stride": 1, "padding": 2, "bias": True},
            {"type": "convolution", "insize": 16, "size": 32, "winlen": 9, "stride": 4, "padding": 4, "bias": True},
            {"type": "permute", "dims": [0, 2, 1]}]},
        "transformer_encoder": {"depth": 2, "layer": {
            "d_model": 32, "nhead": 4, "dim_feedforward": 64, "deepnorm_alpha": 2.0, "attn_window": [7, 8]}}}},
    "basecaller": {"chunksize": 512, "overlap": 16},
}


def with_depth(cfg, depth):
    """A copy of cfg with `depth` transformer layers."""
    import copy
    c = copy.deepcopy(cfg)
    c["model"]["encoder"]["transformer_encoder"]["depth"] = depth
    return c


def conv_layers(cfg):
    """viktor/encoder.py:116-118: the convolution sublayers in order."""
    return [l for l in cfg["model"]["encoder"]["conv"]["sublayers"] if l["type"] == "convolution"]


def encoder_params(cfg, seed=0, alpha_from_cfg=True):
    """Synthetic fp32 weights under the reference module's state-dict names (viktor/encoder.py:43-134):
    conv.{i}.conv.weight/bias, transformer_encoder.{l}.self_attn.{Wqkv.weight, out_proj.weight,
    out_proj.bias}, ff.fc1.weight, ff.fc2.weight, norm1.weight, norm2.weight. Linear / conv weights
    ~ N(0, 1) / sqrt(fan_in), biases ~ N(0, 0.1), norm weights ~ 1 + N(0, 0.1)."""
    g = torch.Generator().manual_seed(seed)
    p = {}
    for i, l in enumerate(conv_layers(cfg)):
        fan = l["insize"] * l["winlen"]
        p[f"conv.{i}.conv.weight"] = torch.randn(l["size"], l["insize"], l["winlen"], generator=g) / math.sqrt(fan)
        p[f"conv.{i}.conv.bias"] = 0.1 * torch.randn(l["size"], generator=g)
    tx = cfg["model"]["encoder"]["transformer_encoder"]
    lay = tx["layer"]
    C, Fd = lay["d_model"], lay["dim_feedforward"]
    for j in range(tx["depth"]):
        pre = f"transformer_encoder.{j}."
        p[pre + "self_attn.Wqkv.weight"] = torch.randn(3 * C, C, generator=g) / math.sqrt(C)
        p[pre + "self_attn.out_proj.weight"] = torch.randn(C, C, generator=g) / math.sqrt(C)
        p[pre + "self_attn.out_proj.bias"] = 0.1 * torch.randn(C, generator=g)
        p[pre + "ff.fc1.weight"] = torch.randn(2 * Fd, C, generator=g) / math.sqrt(C)
        p[pre + "ff.fc2.weight"] = torch.randn(C, Fd, generator=g) / math.sqrt(Fd)
        p[pre + "norm1.weight"] = 1 + 0.1 * torch.randn(C, generator=g)
        p[pre + "norm2.weight"] = 1 + 0.1 * torch.randn(C, generator=g)
        if alpha_from_cfg:
            p[pre + "deepnorm_alpha"] = torch.tensor(float(lay["deepnorm_alpha"]))
    return p


def band_attention(q, k, v, window):
    """Softmax attention of one chunk with the band mask of viktor/encoder.py:64-69 (key j visible to query i
    iff -window[0] <= j - i <= window[1]); q, k, v [T, H, D] (fp32 or fp64); scale 1/sqrt(D) (SDPA's default,
    viktor/encoder.py:80-82). Returns [T, H, D]."""
    T, H, D = q.shape
    i = torch.arange(T)
    rel = i[None, :] - i[:, None]
    allowed = (rel >= -window[0]) & (rel <= window[1])
    s = torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(D)
    s = s.masked_fill(~allowed[None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), v)


class RefEncoder:
    """viktor/encoder.py:111-192 on the CPU. params: fp32 state dict (encoder_params or a loaded one)."""

    def __init__(self, cfg, params, mode="fp32"):
        assert mode in ("fp32", "bf16")
        self.mode = mode
        enc = cfg["model"]["encoder"]
        self.convs = conv_layers(cfg)
        self.stride = 1
        for l in self.convs:
            self.stride *= l["stride"]
        tx = enc["transformer_encoder"]
        lay = tx["layer"]
        self.depth, self.d_model, self.nhead = tx["depth"], lay["d_model"], lay["nhead"]
        self.head_dim = self.d_model // self.nhead
        self.window = tuple(lay["attn_window"])
        self.alpha = float(lay["deepnorm_alpha"])
        self.cos, self.sin = rope_tables(self.head_dim, lay.get("max_seq_len", 4096), lay.get("theta", 10000.0))
        self.chunksize = cfg["basecaller"]["chunksize"]
        self.granularity = self.stride * 64
        r = bf if mode == "bf16" else (lambda t: t)
        self.r = r
        # bf16 mode: every weight bf16-valued except the first convolution's (read in fp32 with the signal)
        self.p = {k: (v.float() if (mode == "fp32" or k.startswith("conv.0.")) else bf(v.float())) for k, v in params.items()}

    # viktor/encoder.py:43-49 (Conv: Conv1d + SiLU), 149-158 (forward: conv stack then transpose)
    def conv(self, x):
        """x [N, 1, T] fp32 -> [N, T / stride, C]."""
        r = self.r
        for i, l in enumerate(self.convs):
            w, b = self.p[f"conv.{i}.conv.weight"], self.p[f"conv.{i}.conv.bias"]
            y = r(F.conv1d(x, w, b, stride=l["stride"], padding=l["padding"]))
            x = r(F.silu(y))
        return x.transpose(1, 2)

    # viktor/encoder.py:71-84
    def attention(self, j, x):
        """x [N, T, C] -> out_proj(attn) [N, T, C] (bias included; bf16 mode rounds it)."""
        r, p = self.r, self.p
        pre = f"transformer_encoder.{j}.self_attn."
        N, T, C = x.shape
        qkv = r(x @ p[pre + "Wqkv.weight"].t()).view(N, T, 3, self.nhead, self.head_dim)
        q, k, v = qkv.unbind(2)
        cos, sin = self.cos[:T], self.sin[:T]
        q, k = r(apply_rope(q, cos, sin)), r(apply_rope(k, cos, sin))
        o = torch.stack([band_attention(q[n], k[n], v[n], self.window) for n in range(N)])
        o = r(o).reshape(N, T, C)
        return r(o @ p[pre + "out_proj.weight"].t() + p[pre + "out_proj.bias"])

    def rmsnorm(self, x, w):
        return self.r(x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-5) * w)

    # viktor/encoder.py:86-108 (GatedMlp: silu(second half) * first half; TxLayer: DeepNorm post-norm)
    def layer(self, j, x):
        r, p = self.r, self.p
        pre = f"transformer_encoder.{j}."
        a = self.alpha
        x = self.rmsnorm(r(self.attention(j, x) + r(a * x)), p[pre + "norm1.weight"])
        h = x @ p[pre + "ff.fc1.weight"].t()
        y, gate = h.chunk(2, -1)
        if self.mode == "bf16":
            y, gate = bf(y), bf(gate)
            f = bf(bf(F.silu(gate)) * y)
            ff = bf(f @ p[pre + "ff.fc2.weight"].t())
        else:
            ff = (F.silu(gate) * y) @ p[pre + "ff.fc2.weight"].t()
        return self.rmsnorm(r(ff + r(a * x)), p[pre + "norm2.weight"])

    def forward(self, x):
        """x [N, 1, T] -> frames [N, T / stride, d_model] (viktor/encoder.py:149-158)."""
        x = self.conv(x.float())
        for j in range(self.depth):
            x = self.layer(j, x)
        return x

    def forward_varlen(self, signal, lens):
        """viktor/encoder.py:160-176: runs of equal-length chunks, each chunk encoded independently."""
        out, off, i = [], 0, 0
        while i < len(lens):
            j = i
            while j < len(lens) and lens[j] == lens[i]:
                j += 1
            n = int(lens[i])
            out.append(self.forward(signal[off:off + n * (j - i)].view(j - i, 1, n)).flatten(0, 1))
            off, i = off + n * (j - i), j
        return torch.cat(out)

    def encode_chunks(self, signal, lens, valid):
        """viktor/encoder.py:178-192: forward_varlen, then only the first ceil(valid / stride) frames of each
        chunk. Returns (frames, frame_lens)."""
        frames = self.forward_varlen(signal, lens)
        padded = [int(n) // self.stride for n in lens]
        frame_lens = [-(-int(v) // self.stride) for v in valid]
        assert all(0 < f <= p for f, p in zip(frame_lens, padded))
        starts = np.cumsum([0] + padded[:-1])
        idx = np.concatenate([np.arange(s, s + f) for s, f in zip(starts, frame_lens)])
        return frames[torch.from_numpy(idx)], frame_lens
