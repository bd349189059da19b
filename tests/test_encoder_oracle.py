"""Pins the encoder oracle (oracle/encoder.py) and the HIP encoder's host-side layout plan, on the CPU.

The oracle restates viktor/encoder.py:43-192; each check below is independent of its formulas: a direct
sum for the convolution, a brute-force loop and closed-form special cases for the banded attention, complex
multiplication for the rotation, and the reference's own encoder tests (tests/test_viktor.py:71-104).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import encoder as E
from oracle.reference import apply_rope, rope_tables


def test_conv_matches_direct_sum():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 40, generator=g, dtype=torch.float64)
    w = torch.randn(5, 3, 9, generator=g, dtype=torch.float64)
    b = torch.randn(5, generator=g, dtype=torch.float64)
    stride, pad = 3, 4
    y = F.conv1d(x, w, b, stride=stride, padding=pad)
    T_out = (40 + 2 * pad - 9) // stride + 1
    want = torch.zeros(2, 5, T_out, dtype=torch.float64)
    for n in range(2):
        for co in range(5):
            for t in range(T_out):
                s = b[co].item()
                for ci in range(3):
                    for k in range(9):
                        pos = t * stride - pad + k
                        if 0 <= pos < 40:
                            s += w[co, ci, k].item() * x[n, ci, pos].item()
                want[n, co, t] = s
    assert torch.allclose(y, want, atol=1e-12)
    assert T_out == 40 // stride + (1 if 40 % stride else 0)  # 'same' padding: ceil(T / stride) frames


def test_band_attention_brute_force():
    g = torch.Generator().manual_seed(1)
    T, H, D = 23, 2, 8
    q, k, v = (torch.randn(T, H, D, generator=g, dtype=torch.float64) for _ in range(3))
    for window in ((3, 5), (0, 2), (7, 0), (30, 30)):
        got = E.band_attention(q, k, v, window)
        for i in range(T):
            for h in range(H):
                keys = [j for j in range(T) if -window[0] <= j - i <= window[1]]
                s = torch.tensor([(q[i, h] * k[j, h]).sum().item() / math.sqrt(D) for j in keys], dtype=torch.float64)
                p = torch.softmax(s, 0)
                want = sum(p[n] * v[j, h] for n, j in enumerate(keys))
                assert torch.allclose(got[i, h], want, atol=1e-12), (window, i, h)


def test_band_attention_special_cases():
    g = torch.Generator().manual_seed(2)
    T, H, D = 17, 3, 8
    q, k, v = (torch.randn(T, H, D, generator=g, dtype=torch.float64) for _ in range(3))
    assert torch.allclose(E.band_attention(q, k, v, (0, 0)), v, atol=1e-12)  # each query sees itself only
    full = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)).transpose(0, 1)
    assert torch.allclose(E.band_attention(q, k, v, (T, T)), full, atol=1e-12)
    causal = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                            is_causal=True).transpose(0, 1)
    assert torch.allclose(E.band_attention(q, k, v, (T, 0)), causal, atol=1e-12)  # left side = the past


def test_rope_is_complex_rotation():
    cos, sin = rope_tables(64, 300, 10000.0)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(300, 2, 64, generator=g, dtype=torch.float64)
    got = apply_rope(x, cos.double(), sin.double())
    z = torch.complex(x[..., :32], x[..., 32:])
    ang = torch.arange(300, dtype=torch.float64)[:, None] * (10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    rot = z * torch.polar(torch.ones_like(ang), ang)[:, None, :]
    assert torch.allclose(got, torch.cat([rot.real, rot.imag], -1), atol=1e-5)  # fp32 tables


def _tiny(mode="fp32"):
    return E.RefEncoder(E.TINY_CFG, E.encoder_params(E.TINY_CFG, seed=0), mode)


def test_reference_varlen_is_per_chunk():
    """tests/test_viktor.py:71-78 on the oracle."""
    enc = _tiny()
    lens = [512, 256]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(4))
    packed = enc.forward_varlen(sig, lens)
    alone = torch.cat([enc.forward(sig[:512].view(1, 1, -1))[0], enc.forward(sig[512:].view(1, 1, -1))[0]])
    assert torch.allclose(packed, alone)
    assert packed.shape == (768 // enc.stride, 32)


def test_reference_encode_chunks_drops_padding_frames():
    """tests/test_viktor.py:81-90 on the oracle: ceil(130 / 4) = 33 frames kept of the second chunk."""
    enc = _tiny()
    lens, valid = [512, 256], [512, 130]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(5))
    packed = enc.forward_varlen(sig, lens)
    frames, flens = enc.encode_chunks(sig, lens, valid)
    assert flens == [128, 33]
    assert torch.equal(frames, torch.cat([packed[:128], packed[128:161]]))


def test_oracle_layer_matches_module_composition():
    """The oracle's DeepNorm layer against nn modules assembled from the reference's description
    (viktor/encoder.py:86-108): nn.Linear, nn.RMSNorm, SDPA with the band mask."""
    cfg = E.with_depth(E.TINY_CFG, 1)
    p = E.encoder_params(cfg, seed=6)
    enc = E.RefEncoder(cfg, p)
    x = torch.randn(2, 20, 32, generator=torch.Generator().manual_seed(7))
    pre = "transformer_encoder.0."
    N, T, C, H = 2, 20, 32, 4
    qkv = (x @ p[pre + "self_attn.Wqkv.weight"].t()).view(N, T, 3, H, C // H)
    q, k, v = qkv.unbind(2)
    cos, sin = rope_tables(C // H, 4096, 10000.0)
    q, k = apply_rope(q, cos[:T], sin[:T]), apply_rope(k, cos[:T], sin[:T])
    i = torch.arange(T)
    rel = i[None, :] - i[:, None]
    mask = (rel >= -7) & (rel <= 8)
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), attn_mask=mask)
    a = o.transpose(1, 2).reshape(N, T, C) @ p[pre + "self_attn.out_proj.weight"].t() + p[pre + "self_attn.out_proj.bias"]
    n1 = torch.nn.RMSNorm(C, eps=1e-5)
    n1.weight.data = p[pre + "norm1.weight"]
    n2 = torch.nn.RMSNorm(C, eps=1e-5)
    n2.weight.data = p[pre + "norm2.weight"]
    h = n1(a + 2.0 * x)
    y, gate = (h @ p[pre + "ff.fc1.weight"].t()).chunk(2, -1)
    want = n2((F.silu(gate) * y) @ p[pre + "ff.fc2.weight"].t() + 2.0 * h)
    with torch.no_grad():
        got = enc.layer(0, x)
    assert torch.allclose(got, want.detach(), atol=1e-5)


# ---- host-side layout plan of the HIP encoder (no GPU needed) ----------------------------------------------
def _emulate_conv_stack(convs, params, sig, lens):
    """The HIP conv stack's data flow on the CPU in fp64: the padded layout, each layer as the strided-row GEMM
    the kernel computes (input row stride * g - pad), margin rows zeroed, the last layer compacted."""
    from viktor_amd.encoder import _ConvPlan, _GUARD
    plan = _ConvPlan(convs, lens, "cpu")
    n = len(lens)
    offs = np.concatenate([[0], np.cumsum(lens)])
    prev = None
    for i, l in enumerate(convs):
        lay = plan.layers[i]
        rows, start, ln = lay["rows"], lay["start"].numpy(), lay["len"].numpy()
        w = params[f"conv.{i}.conv.weight"].double()
        b = params[f"conv.{i}.conv.bias"].double()
        out = torch.zeros(rows + 2 * _GUARD, l["size"], dtype=torch.float64)
        hint = lay["hint"].numpy()
        for g in range(rows):
            c = max(int(np.searchsorted(start, g, side="right")) - 1, 0)
            ch = int(hint[g >> 8])  # the kernels' lookup: walk forward from the 256-row hint
            while ch + 1 < n and start[ch + 1] <= g:
                ch += 1
            assert ch == c
            t = g - start[c]
            if not (0 <= t < ln[c]):
                continue
            if i == 0:
                s = sig[offs[c]:offs[c + 1]].double()
                xs = torch.tensor([s[t * l["stride"] - l["padding"] + k].item()
                                   if 0 <= t * l["stride"] - l["padding"] + k < len(s) else 0.0
                                   for k in range(l["winlen"])], dtype=torch.float64)
                out[_GUARD + g] = F.silu(w[:, 0, :] @ xs + b)
            else:
                r0 = _GUARD + l["stride"] * g - l["padding"]
                a = prev[r0:r0 + l["winlen"]]  # [winlen, C_in] rows of the padded input
                out[_GUARD + g] = F.silu(torch.einsum("okc,kc->o", w.permute(0, 2, 1), a) + b)
        prev = out
    last = plan.layers[-1]
    start, ln = last["start"].numpy(), last["len"].numpy()
    return torch.cat([prev[_GUARD + start[c]:_GUARD + start[c] + ln[c]] for c in range(n)]), plan


@pytest.mark.parametrize("cfg,lens", [(E.TINY_CFG, [512, 256, 64]),
                                      (E.SUP_CFG, [768, 1536, 768])])
def test_padded_layout_equals_per_chunk_conv(cfg, lens):
    """The padded layout's strided rows reproduce each chunk's own zero-padded Conv1d stack."""
    convs = E.conv_layers(cfg)
    if cfg is E.SUP_CFG:  # narrow the channels (the layout does not depend on them) to keep the loop quick
        convs = [dict(l, size=8, insize=(1 if i == 0 else 8)) for i, l in enumerate(convs)]
        cfg = {"model": {"encoder": {"conv": {"sublayers": convs}}}}
    params = {}
    g = torch.Generator().manual_seed(8)
    for i, l in enumerate(convs):
        params[f"conv.{i}.conv.weight"] = torch.randn(l["size"], l["insize"], l["winlen"], generator=g, dtype=torch.float64)
        params[f"conv.{i}.conv.bias"] = torch.randn(l["size"], generator=g, dtype=torch.float64)
    sig = torch.randn(sum(lens), generator=g, dtype=torch.float64)
    got, plan = _emulate_conv_stack(convs, params, sig, lens)
    want, off = [], 0
    for n in lens:
        x = sig[off:off + n].view(1, 1, n)
        for i, l in enumerate(convs):
            x = F.silu(F.conv1d(x, params[f"conv.{i}.conv.weight"], params[f"conv.{i}.conv.bias"],
                                stride=l["stride"], padding=l["padding"]))
        want.append(x[0].t())
        off += n
    want = torch.cat(want)
    assert got.shape == want.shape
    assert torch.allclose(got, want, atol=1e-10)
    stride = int(np.prod([l["stride"] for l in convs]))
    assert plan.frames == [n // stride for n in lens]
    # margins: each at least the next layer's padding, scaled by the strides
    for i in range(1, len(convs)):
        assert plan.margins[i - 1] == convs[i]["stride"] * plan.margins[i] >= convs[i]["padding"]
