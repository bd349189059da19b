"""Small Qwen3-style decoder-only LM (RMSNorm, GQA, QK-norm, RoPE, SwiGLU) whose forward runs on the
gfx950 HIP kernels.

The module tree and parameter names are those of viktor/decoder.py:25-164 (embed, layers[i].attn_norm,
.attn.{qkv_proj, o_proj, q_norm, k_norm}, .mlp_norm, .gate_up, .down, norm, lm_head; cos/sin buffers),
so reference checkpoints load and in-place weight syncs stay visible to captured graphs. Both call
modes of the reference exist:
  * full causal pass over [prefix | tokens] (optionally writing the KV cache),
  * one token per sequence against the static KV cache (pos given).
There is no CPU fallback: the forward requires the module and inputs on a ROCm GPU.
"""

from dataclasses import dataclass

import torch
import torch.nn as nn


@dataclass
class DecoderConfig:
    """Reference: viktor/decoder.py:25-36 (same fields and defaults)."""
    vocab_size: int
    d_model: int = 512
    n_layers: int = 8
    n_heads: int = 8
    n_kv_heads: int = 2
    head_dim: int = 64
    ffn_dim: int = 1536
    rope_theta: float = 10000.0
    norm_eps: float = 1e-6
    max_seq_len: int = 4096


def rope_tables(dim: int, max_len: int, theta: float):
    """cos, sin [max_len, dim/2] fp32 of angle p / theta^(2i/dim), computed in fp64 with the reference's
    order of operations (exponent 2i/dim, reciprocal of the power, then times p) so the tables match it
    bit for bit (reference: viktor/encoder.py:30-33)."""
    exponent = torch.arange(0, dim, 2, dtype=torch.float64) / dim
    inv_freq = 1.0 / (theta ** exponent)
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv_freq[None, :]
    return ang.cos().to(torch.float32), ang.sin().to(torch.float32)


class KVCache:
    """Static cache, layout [layer, batch, position, kv_head, head_dim] (reference: viktor/decoder.py:43-51).
    In HBM each (sequence, position) row of one layer is HKV * head_dim contiguous bf16 values (256 B).
    pad_rows > 0 leaves that many unused rows after each sequence's max_len rows (k / v are views of the
    padded storage): it moves the sequences' start addresses off a power-of-two stride, where concurrent
    streams over many sequences would share HBM channels."""

    def __init__(self, cfg: DecoderConfig, batch: int, max_len: int, dtype, device, pad_rows: int = 0):
        shape = (cfg.n_layers, batch, max_len + int(pad_rows), cfg.n_kv_heads, cfg.head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=device)[:, :, :max_len]
        self.v = torch.zeros(shape, dtype=dtype, device=device)[:, :, :max_len]
        self.max_len = max_len
        self.positions = torch.arange(max_len, device=device)


class Attention(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.h, self.hkv, self.d = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        self.qkv_proj = nn.Linear(cfg.d_model, (self.h + 2 * self.hkv) * self.d, bias=False)
        self.o_proj = nn.Linear(self.h * self.d, cfg.d_model, bias=False)
        self.q_norm = nn.RMSNorm(self.d, eps=cfg.norm_eps)
        self.k_norm = nn.RMSNorm(self.d, eps=cfg.norm_eps)


class Block(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.attn_norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.attn = Attention(cfg)
        self.mlp_norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.gate_up = nn.Linear(cfg.d_model, 2 * cfg.ffn_dim, bias=False)
        self.down = nn.Linear(cfg.ffn_dim, cfg.d_model, bias=False)


class Decoder(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList([Block(cfg) for _ in range(cfg.n_layers)])
        self.norm = nn.RMSNorm(cfg.d_model, eps=cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        cos, sin = rope_tables(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)
        self._fast = None

    def fast(self):
        from .fast_decoder import FastDecoder
        if self._fast is None:
            self._fast = FastDecoder(self)
        return self._fast

    def forward(self, x, cache=None, batch_slice=slice(None), pos=None, seqlens=None, positions=None):
        """x [B, T, d] input embeddings (bf16, or fp32 cast to bf16). pos [B] selects single-token decode
        mode (T == 1; the token is written at cache position pos and attends to positions <= pos).
        positions: RoPE positions when they differ from the sequence index ([T] or [B, T]; decode [B]).
        Returns the final-normed hidden states [B, T, d] (bf16); apply `head` for logits.
        Reference: viktor/decoder.py:135-144."""
        return self.fast().forward(x, cache=cache, batch_slice=batch_slice, pos=pos, positions=positions)

    def head(self, h):
        """Logits of hidden states [..., d] in bf16 (an nn.Linear in bf16). Reference: viktor/decoder.py:163-164."""
        from .hip_ops import linear
        w = self.fast().w(self.lm_head.weight)
        shp = h.shape
        return linear(h.reshape(-1, shp[-1]).to(torch.bfloat16).contiguous(), w).view(*shp[:-1], -1)
