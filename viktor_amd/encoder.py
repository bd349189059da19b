"""The Dorado SUP encoder on the HIP kernels: the frames producer in front of the decoder.

Mirrors viktor/encoder.py:111-211 (DoradoEncoder: forward, forward_varlen, encode_chunks, standardise,
load_dorado_encoder) with the reference's config dict and state-dict names. The reference runs this encoder
on ONT's closed koi kernels (viktor/koi.py, viktor/csrc/koi_tx.cpp:120-423) or in PyTorch; here:

  * the convolution stack runs in a padded chunk layout (channels-last, zero margin rows between chunks,
    margins scaled by the strides) so that every layer is one launch over the whole batch:
    vk_encoder_conv_first for the C_in = 1 layer, vk_encoder_conv (a strided-A GEMM) for the others, the
    last one writing the transformer's packed [frames, 512] input;
  * each transformer layer is seven launches: the Wqkv product with the rotary embedding in its epilogue
    (vk_linear_qkv_rope), sliding-window attention (vk_window_attention), out_proj with the bias and the
    DeepNorm residual in its epilogue (vk_linear_residual_big, which also hands over the row sums of squares)
    then the RMSNorm (vk_rmsnorm_apply_ss), fc1 with the SwiGLU epilogue, fc2 with the second DeepNorm
    residual in its epilogue, then the second RMSNorm.

Every kernel computes a chunk's rows with the same code whatever else is in the batch (row-deterministic
GEMMs, chunk-relative attention tiles, per-row convolutions), so a mixed batch gives each chunk exactly the
frames it gets alone -- the koi VCS property the reference checks at tests/gpu_check.py:103-105.

Precision: bf16 weights and activations, fp32 accumulation and fp32 math inside each kernel; the first
convolution reads the fp32 signal with fp32 weights. Built for d_model 512 with 64-wide heads (the SUP
shape); other shapes raise.
"""

import glob
import os
import sys
from typing import Dict, List, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import HipLibraryError, call, ptr, require_device

if sys.version_info >= (3, 11):
    import tomllib
else:  # pragma: no cover - Python 3.10 image
    import tomli as tomllib

_GUARD = 32  # zero rows before and after each padded activation buffer (>= every pad and window)


def _rope_tables(dim: int, max_len: int, theta: float):
    """viktor/encoder.py:30-33: inv = theta^(-2i/dim) in fp64, cos / sin [max_len, dim / 2] fp32."""
    inv = 1.0 / theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv
    return ang.cos().float(), ang.sin().float()


def _bf16_valued(t: torch.Tensor) -> torch.Tensor:
    return t.detach().float().to(torch.bfloat16).float()


class _ConvPlan:
    """Padded layouts of one batch of chunk lengths (samples): per convolution the data starts / lengths of
    its output rows and the total rows, margins chosen so that the input row of output row g is
    stride * g - pad across the whole buffer."""

    def __init__(self, convs, lens: Sequence[int], device):
        n = len(lens)
        L = len(convs)
        # output lengths per layer
        cur = np.asarray(lens, dtype=np.int64)
        out_lens = []
        for c in convs:
            cur = cur // c["stride"]
            out_lens.append(cur)
        # margins: out margin of the last layer m; input margin of layer i = stride_i * out margin of layer i
        m = 1
        while True:
            mo = [0] * L
            mo[L - 1] = m
            for i in range(L - 1, 0, -1):
                mo[i - 1] = convs[i]["stride"] * mo[i]
            ok = all(mo[i - 1] >= convs[i]["padding"] and mo[i - 1] >= convs[i]["winlen"] - convs[i]["padding"] - convs[i]["stride"]
                     for i in range(1, L))
            if ok:
                break
            m += 1
        self.margins = mo
        self.layers = []
        for i in range(L):
            M = mo[i]
            ol = out_lens[i]
            starts = (np.arange(n, dtype=np.int64) + 1) * M + np.concatenate([[0], np.cumsum(ol)[:-1]])
            rows = int(ol.sum()) + (n + 1) * M
            if rows >= 2 ** 31:
                raise HipLibraryError("encoder: batch too large for 32-bit row indices")
            # chunk of every 256th row (the kernels walk forward from it)
            hint = np.maximum(np.searchsorted(starts, np.arange(0, rows, 256), side="right") - 1, 0)
            self.layers.append({
                "rows": rows,
                "start": torch.from_numpy(starts.astype(np.int32)).to(device),
                "hint": torch.from_numpy(hint.astype(np.int32)).to(device),
                "len": torch.from_numpy(ol.astype(np.int32)).to(device),
            })
        frames = out_lens[-1]
        self.frames = [int(f) for f in frames]
        self.total_frames = int(frames.sum())
        cu = np.concatenate([[0], np.cumsum(frames)]).astype(np.int32)
        self.cu = torch.from_numpy(cu).to(device)
        self.dst0 = torch.from_numpy(cu[:-1].copy()).to(device)
        sig_off = np.concatenate([[0], np.cumsum(np.asarray(lens, dtype=np.int64))[:-1]])
        self.sig_off = torch.from_numpy(sig_off.astype(np.int64)).to(device)
        # rotary position of every frame: its index within its chunk
        self.rope_pos = torch.from_numpy(np.concatenate([np.arange(f, dtype=np.int32) for f in self.frames])).to(device)
        # attention plan: (chunk, first query row) per 128-row block
        blocks = [(c, qs) for c, f in enumerate(self.frames) for qs in range(0, f, 128)]
        self.n_blocks = len(blocks)
        self.plan = torch.tensor(np.asarray(blocks, dtype=np.int32).reshape(-1), dtype=torch.int32).to(device)
        self.max_frames = max(self.frames) if self.frames else 0


class DoradoEncoder:
    """signal [N, 1, T] (standardised pA) -> frames [N, T / stride, d_model] on the HIP kernels.
    Reference: viktor/encoder.py:111-192 (same config dict, attributes and methods)."""

    def __init__(self, cfg: dict, device="cuda"):
        enc = cfg["model"]["encoder"]
        self.convs = [l for l in enc["conv"]["sublayers"] if l["type"] == "convolution"]
        self.stride = 1
        for l in self.convs:
            self.stride *= l["stride"]
        tx = enc["transformer_encoder"]
        lay = tx["layer"]
        self.tx_layer = lay
        self.depth = tx["depth"]
        self.d_model = lay["d_model"]
        self.nhead = lay["nhead"]
        self.head_dim = self.d_model // self.nhead
        self.dim_feedforward = lay["dim_feedforward"]
        self.window = tuple(int(w) for w in lay["attn_window"])
        self.default_alpha = float(lay["deepnorm_alpha"])
        self.theta = float(lay.get("theta", 10000.0))
        self.max_seq_len = int(lay.get("max_seq_len", 4096))
        std = cfg.get("standardisation", {})
        self.mean, self.stdev = std.get("mean", 0.0), std.get("stdev", 1.0)
        self.chunksize = cfg["basecaller"]["chunksize"]
        self.granularity = self.stride * 64  # Dorado chunk_size_granularity()
        self.overlap = cfg["basecaller"]["overlap"]
        self.device = torch.device(device)
        self._check_shapes()
        cos, sin = _rope_tables(self.head_dim, self.max_seq_len, self.theta)
        self.cos, self.sin = cos.to(self.device).contiguous(), sin.to(self.device).contiguous()
        self.weights = None
        self._plans: Dict[tuple, _ConvPlan] = {}

    def _check_shapes(self):
        c = self.convs
        msgs = []
        if (not c or c[0]["insize"] != 1 or c[0]["winlen"] > 32 or c[0]["size"] % 8 or c[0]["size"] > 512
                or c[0]["size"] * c[0]["winlen"] > 4096):
            msgs.append("the first convolution must read 1 channel with winlen <= 32 and a multiple of 8 outputs "
                        "(at most 512, size * winlen <= 4096)")
        for i, l in enumerate(c):
            if l["winlen"] != 2 * l["padding"] + 1:
                msgs.append(f"conv {i}: winlen must be 2 * padding + 1")
            if i > 0 and ((l["insize"] * l["winlen"]) % 32 or l["size"] % 64 or l["padding"] > _GUARD or l["winlen"] > _GUARD):
                msgs.append(f"conv {i}: needs insize * winlen % 32 == 0 and size % 64 == 0")
        if c and c[-1]["size"] != self.d_model:
            msgs.append("the last convolution must produce d_model channels")
        if self.d_model != 512 or self.head_dim != 64:
            msgs.append(f"built for d_model 512 with head_dim 64 (got {self.d_model} / {self.head_dim})")
        if self.dim_feedforward % 64:
            msgs.append("dim_feedforward must be a multiple of 64")
        if min(self.window) < 0:
            msgs.append("attention window sides must be >= 0")
        if msgs:
            raise HipLibraryError("DoradoEncoder (HIP): unsupported config: " + "; ".join(msgs))

    # ---- weights ----------------------------------------------------------------------------------
    def load_state_dict(self, sd: Dict[str, torch.Tensor]):
        """Weights under the reference module's names (viktor/encoder.py:43-134): conv.{i}.conv.weight/bias,
        transformer_encoder.{l}.{self_attn.Wqkv.weight, self_attn.out_proj.weight, self_attn.out_proj.bias,
        ff.fc1.weight, ff.fc2.weight, norm1.weight, norm2.weight[, deepnorm_alpha]}. Stored as bf16 (the first
        convolution fp32), fc1 reordered gate-first for the SwiGLU epilogue."""
        dev = self.device
        W = {"conv": [], "layers": []}
        for i, l in enumerate(self.convs):
            w = sd[f"conv.{i}.conv.weight"].detach().float()
            b = sd.get(f"conv.{i}.conv.bias")
            b = torch.zeros(l["size"]) if b is None else b.detach().float()
            assert tuple(w.shape) == (l["size"], l["insize"], l["winlen"]), f"conv {i} weight shape {tuple(w.shape)}"
            if i == 0:
                W["conv"].append((w.reshape(l["size"], l["winlen"]).contiguous().to(dev), b.contiguous().to(dev)))
            else:
                wk = w.permute(0, 2, 1).reshape(l["size"], l["winlen"] * l["insize"])  # k = tap * C_in + channel
                W["conv"].append((wk.to(torch.bfloat16).contiguous().to(dev), _bf16_valued(b).contiguous().to(dev)))
        C, Fd = self.d_model, self.dim_feedforward
        for j in range(self.depth):
            pre = f"transformer_encoder.{j}."
            fc1 = sd[pre + "ff.fc1.weight"].detach().float()
            assert tuple(fc1.shape) == (2 * Fd, C)
            alpha = sd.get(pre + "deepnorm_alpha")
            W["layers"].append({
                "wqkv": sd[pre + "self_attn.Wqkv.weight"].detach().to(torch.bfloat16).contiguous().to(dev),
                "wo": sd[pre + "self_attn.out_proj.weight"].detach().to(torch.bfloat16).contiguous().to(dev),
                "bo": _bf16_valued(sd[pre + "self_attn.out_proj.bias"]).contiguous().to(dev),
                # y, gate = fc1(x).chunk(2): the kernel's SwiGLU takes the gate rows first
                "w1": torch.cat([fc1[Fd:], fc1[:Fd]]).to(torch.bfloat16).contiguous().to(dev),
                "w2": sd[pre + "ff.fc2.weight"].detach().to(torch.bfloat16).contiguous().to(dev),
                "n1": sd[pre + "norm1.weight"].detach().to(torch.bfloat16).contiguous().to(dev),
                "n2": sd[pre + "norm2.weight"].detach().to(torch.bfloat16).contiguous().to(dev),
                "alpha": float(alpha) if alpha is not None else self.default_alpha,
            })
        self.weights = W
        return self

    # ---- API of the reference module ----------------------------------------------------------------
    def standardise(self, pa):
        return (pa - self.mean) / self.stdev

    def _plan(self, lens) -> _ConvPlan:
        key = tuple(int(n) for n in lens)
        p = self._plans.get(key)
        if p is None:
            if len(self._plans) > 64:
                self._plans.clear()
            p = _ConvPlan(self.convs, key, self.device)
            self._plans[key] = p
        return p

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [N, 1, T] -> frames [N, T / stride, d_model] bf16 (viktor/encoder.py:149-158)."""
        n, _, t = x.shape
        return self.forward_varlen(x.reshape(-1), [t] * n).view(n, t // self.stride, self.d_model)

    __call__ = forward

    def forward_varlen(self, signal: torch.Tensor, lens: Sequence[int]) -> torch.Tensor:
        """Variable-length chunks, each encoded independently (viktor/encoder.py:160-176): signal 1D (chunks
        concatenated), lens samples per chunk (each a multiple of the stride; Dorado's VCS chunks are
        multiples of the granularity). Returns frames [sum(lens) / stride, d_model] bf16, chunks in order."""
        if self.weights is None:
            raise HipLibraryError("DoradoEncoder: no weights loaded (load_state_dict)")
        require_device(signal, "DoradoEncoder.forward_varlen")
        lens = [int(n) for n in lens]
        if not lens:
            return torch.empty(0, self.d_model, dtype=torch.bfloat16, device=signal.device)
        if any(n <= 0 or n % self.stride for n in lens):
            raise HipLibraryError(f"DoradoEncoder: chunk lengths must be positive multiples of the stride {self.stride}")
        if sum(lens) != signal.numel():
            raise HipLibraryError(f"DoradoEncoder: lens sum to {sum(lens)} samples, signal has {signal.numel()}")
        if max(lens) // self.stride > self.max_seq_len:
            raise HipLibraryError(f"DoradoEncoder: a chunk of {max(lens)} samples exceeds the rotary table "
                                  f"({self.max_seq_len} frames)")
        plan = self._plan(lens)
        sig = signal.reshape(-1).float().contiguous()
        x = self._conv_stack(sig, plan)
        self._transformer(x, plan)
        return x

    def encode_chunks(self, signal, lens, valid):
        """viktor/encoder.py:178-192: forward_varlen on the repeat-padded chunks, then only the frames of each
        chunk's real signal (ceil(valid / stride)). Returns (frames [sum(frame_lens), d_model], frame_lens)."""
        frames = self.forward_varlen(signal, lens)
        padded = [int(n) // self.stride for n in lens]
        frame_lens = [-(-int(v) // self.stride) for v in valid]
        if not all(0 < f <= p for f, p in zip(frame_lens, padded)):
            raise HipLibraryError("encode_chunks: every chunk needs 0 < valid <= its length")
        if frame_lens == padded:
            return frames, frame_lens
        starts = np.cumsum([0] + padded[:-1])
        idx = np.concatenate([np.arange(s, s + f) for s, f in zip(starts, frame_lens)])
        return frames.index_select(0, torch.from_numpy(idx).to(frames.device)), frame_lens

    # ---- the launches -----------------------------------------------------------------------------
    def _conv_stack(self, sig: torch.Tensor, plan: _ConvPlan) -> torch.Tensor:
        dev, st = sig.device, _lib.stream_handle()
        convs, W = self.convs, self.weights["conv"]
        L = len(convs)
        n = len(plan.frames)
        x = torch.empty(plan.total_frames, self.d_model, dtype=torch.bfloat16, device=dev)
        # layer 0: signal -> padded layout of layer 1's input (or straight to frames for a 1-layer stack)
        prev = None
        for i, l in enumerate(convs):
            lay = plan.layers[i]
            last = i == L - 1
            if i == 0:
                if last:
                    raise HipLibraryError("DoradoEncoder: a stack of one convolution is not supported")
                buf = torch.empty(lay["rows"] + 2 * _GUARD, l["size"], dtype=torch.bfloat16, device=dev)
                buf[:_GUARD].zero_()
                buf[_GUARD + lay["rows"]:].zero_()
                w, b = W[0]
                call("vk_encoder_conv_first", ptr(sig), ptr(plan.sig_off), ptr(lay["start"]), ptr(lay["hint"]),
                     ptr(lay["len"]), n,
                     lay["rows"], ptr(w), ptr(b), l["size"], l["winlen"], l["stride"], l["padding"],
                     ptr(buf[_GUARD:]), st)
                prev = buf
                continue
            w, b = W[i]
            cin, s, p = l["insize"], l["stride"], l["padding"]
            a = prev[_GUARD - p:]  # row -pad of the input layout
            if last:
                call("vk_encoder_conv", ptr(a), s * cin, ptr(w), l["winlen"] * cin, l["size"], ptr(b),
                     ptr(lay["start"]), ptr(lay["hint"]), ptr(lay["len"]), ptr(plan.dst0), n, lay["rows"], 1, ptr(x),
                     l["size"], st)
            else:
                buf = torch.empty(lay["rows"] + 2 * _GUARD, l["size"], dtype=torch.bfloat16, device=dev)
                buf[:_GUARD].zero_()
                buf[_GUARD + lay["rows"]:].zero_()
                call("vk_encoder_conv", ptr(a), s * cin, ptr(w), l["winlen"] * cin, l["size"], ptr(b),
                     ptr(lay["start"]), ptr(lay["hint"]), ptr(lay["len"]), ptr(None), n, lay["rows"], 0,
                     ptr(buf[_GUARD:]),
                     l["size"], st)
                prev = buf
        return x

    def _transformer(self, x: torch.Tensor, plan: _ConvPlan):
        dev, st = x.device, _lib.stream_handle()
        M, C, Fd, H = x.shape[0], self.d_model, self.dim_feedforward, self.nhead
        qkv = torch.empty(M, 3 * C, dtype=torch.bfloat16, device=dev)
        o = torch.empty(M, C, dtype=torch.bfloat16, device=dev)
        ss = torch.empty(M, C // 64, dtype=torch.float32, device=dev)
        g = torch.empty(M, Fd, dtype=torch.bfloat16, device=dev)
        n = len(plan.frames)
        hd = self.head_dim
        BF = _lib.VK_DTYPE_BF16  # the encoder's residual stream, norm weights and activations are bf16
        for Lw in self.weights["layers"]:
            # Wqkv with the rotary embedding in its epilogue: q, k (rotated) and v back into the packed rows
            call("vk_linear_qkv_rope", ptr(x), ptr(Lw["wqkv"]), M, C, ptr(None), ptr(None), BF, 0.0, ptr(self.cos),
                 ptr(self.sin), _lib.VK_DTYPE_F32, self.cos.shape[0], ptr(plan.rope_pos), ptr(None), ptr(None),
                 ptr(qkv), 3 * C, ptr(None), ptr(None), 0, 0, 0, 0, ptr(qkv[:, C:]), ptr(qkv[:, 2 * C:]), 3 * C,
                 ptr(None), H, H, hd, st)
            call("vk_window_attention", ptr(qkv), 3 * C, ptr(plan.cu), ptr(plan.plan), plan.n_blocks, n,
                 plan.max_frames, H, hd, ptr(None), ptr(None), 0, self.window[0], self.window[1], ptr(o), C, st)
            # out_proj: bias + DeepNorm residual in the product's epilogue (x in place, row sums of squares out),
            # then the RMSNorm in place; the same for fc2 without bias
            call("vk_linear_residual_big", ptr(o), ptr(Lw["wo"]), ptr(x), BF, M, C, C, ptr(Lw["bo"]), Lw["alpha"],
                 ptr(ss), ptr(None), st)
            call("vk_rmsnorm_apply_ss", ptr(x), BF, ptr(ss), C // 64, ptr(Lw["n1"]), BF, ptr(x), M, C, 1e-5, st)
            call("vk_gemm_rows", ptr(x), ptr(Lw["w1"]), ptr(g), M, Fd, C, 2, st)
            call("vk_linear_residual_big", ptr(g), ptr(Lw["w2"]), ptr(x), BF, M, C, Fd, ptr(None), Lw["alpha"],
                 ptr(ss), ptr(None), st)
            call("vk_rmsnorm_apply_ss", ptr(x), BF, ptr(ss), C // 64, ptr(Lw["n2"]), BF, ptr(x), M, C, 1e-5, st)

    def flops_per_chunk(self, samples: int) -> float:
        """Matrix FLOPs of one chunk: convolutions, the four products per layer and the window attention's
        two products over the keys each query sees (the algorithmic count, no masked tile work)."""
        t, f = samples, 0.0
        for l in self.convs:
            t //= l["stride"]
            f += 2.0 * t * l["size"] * l["insize"] * l["winlen"]
        C, Fd = self.d_model, self.dim_feedforward
        per_tok = 2.0 * (3 * C * C + C * C + 2 * Fd * C + Fd * C)
        keys = sum(min(t - 1, i + self.window[1]) - max(0, i - self.window[0]) + 1 for i in range(t))
        f += self.depth * (per_tok * t + 4.0 * keys * C)
        return f


def load_dorado_encoder(model_dir: str, load_weights: bool = True, device="cuda") -> DoradoEncoder:
    """Build the encoder from a Dorado model directory (config.toml, *.tensor weights) as
    viktor/encoder.py:199-211 does."""
    with open(os.path.join(model_dir, "config.toml"), "rb") as f:
        cfg = tomllib.load(f)
    enc = DoradoEncoder(cfg, device)
    if load_weights:
        sd = {}
        for path in glob.glob(os.path.join(model_dir, "*.tensor")):
            name = os.path.basename(path)[:-len(".tensor")]
            if name.startswith(("conv.", "transformer_encoder.")):
                sd[name] = next(torch.jit.load(path, map_location="cpu").parameters()).detach()
        enc.load_state_dict(sd)
    return enc
