"""The oracle's autocast mode against torch.autocast itself, op by op, on the GPU.

The reference scores under torch.autocast("cuda", bf16) over fp32 master weights (scripts/gspo.py:345-347). Which
ops autocast casts, and where results are rounded, is torch's policy, not the reference's code; this file pins each
rounding point the oracle's "autocast" mode assumes to what torch does on this GPU. Each check compares the same
inputs through torch's modules under autocast (nn.RMSNorm, nn.Linear, nn.Embedding, F.silu, F.gelu, the residual
add) with the oracle's function for that point; a wrong assumption (an fp32 QK-norm output, a bf16 residual stream,
an unrounded norm before a product) fails one of them.
"""

import copy
import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def gen(seed):
    return torch.Generator().manual_seed(seed)


class ulp_close:
    """a, b bf16-valued: every element within `ulps` bf16 ulps, and all but a `frac` fraction identical (products and
    norms sum in another order on the GPU than on the CPU, which moves a value sitting on a rounding boundary).
    atol: an absolute allowance first (a product near zero after cancellation, whose bf16 operand flipped on a
    rounding boundary, moves by far more of its own ulps). Truthy when both hold; repr gives the largest distance
    in ulps (beyond atol) and the fraction that differs."""

    def __init__(self, a, b, ulps=1, frac=1e-3, atol=0.0):
        a, b = a.detach().float().cpu(), b.detach().float().cpu()
        ulp = torch.pow(2.0, torch.floor(torch.log2(b.abs().clamp(min=1e-30))) - 7)
        self.max_ulps = float((((a - b).abs() - atol).clamp(min=0) / ulp).max())
        self.frac = float((a != b).float().mean())
        self.ok = self.max_ulps <= ulps and self.frac <= frac

    def __bool__(self):
        return self.ok

    def __repr__(self):
        return f"max {self.max_ulps:.2f} ulps, {self.frac:.2e} of the elements differ"


def test_qk_norm_of_bf16_head_with_fp32_weights():
    """nn.RMSNorm(64) with fp32 weights on a bf16 head returns bf16((x / rms) * w): the oracle's qk_norm_rope_fused
    at rotary position 0 (cos 1, sin 0), not an fp32 output."""
    g = gen(0)
    qn = nn.RMSNorm(64, eps=1e-6)
    with torch.no_grad():
        qn.weight.copy_(1 + 0.1 * torch.randn(64, generator=g))
    w = qn.weight.detach().clone()
    q = R.bf(torch.randn(4096, 64, generator=g) * 3)
    with torch.autocast("cuda", dtype=BF):
        y = qn.to(DEV)(q.to(BF).to(DEV))
    assert y.dtype == BF
    c, s = torch.ones(4096, 32), torch.zeros(4096, 32)
    want = R.qk_norm_rope_fused(q.view(4096, 1, 64), w, c, s, 1e-6).view(4096, 64)
    r = ulp_close(y, want)
    assert r, r
    # the weight multiplies in fp32 before the one rounding: rounding the weight first moves values
    wrong = R.qk_norm_rope_fused(q.view(4096, 1, 64), R.bf(w), c, s, 1e-6).view(4096, 64)
    assert not ulp_close(y, wrong, ulps=0, frac=0.0)


def test_rope_of_the_bf16_norm_output_in_fp32():
    """apply_rope (viktor/encoder.py:36-40) on the bf16 QK-norm output: the rotation in fp32 with fp32 tables,
    rounded back to the input's dtype -- the oracle's qk_norm_rope_fused at real positions."""
    g = gen(1)
    qn = nn.RMSNorm(64, eps=1e-6)
    with torch.no_grad():
        qn.weight.copy_(1 + 0.1 * torch.randn(64, generator=g))
    w = qn.weight.detach().clone()
    q = R.bf(torch.randn(2048, 1, 64, generator=g) * 3)
    cos, sin = R.rope_tables(64, 4096, 1e6)
    rows = torch.randint(0, 4096, (2048,), generator=g)
    with torch.autocast("cuda", dtype=BF):
        y = qn.to(DEV)(q.to(BF).to(DEV))
        y1, y2 = y.float().chunk(2, -1)
        c, s = cos[rows].to(DEV)[:, None], sin[rows].to(DEV)[:, None]
        rot = torch.cat([y1 * c - y2 * s, y1 * s + y2 * c], -1).to(y.dtype)
    assert rot.dtype == BF
    want = R.qk_norm_rope_fused(q, w, cos[rows], sin[rows], 1e-6)
    r = ulp_close(rot, want)
    assert r, r


def test_residual_norm_linear_and_add():
    """On the fp32 residual stream: nn.RMSNorm(512) returns fp32, the next nn.Linear reads it as bf16 (one
    rounding) with its weight cast to bf16 and returns bf16, and x + that output stays fp32 and exact."""
    g = gen(2)
    norm = nn.RMSNorm(512, eps=1e-6)
    lin = nn.Linear(512, 768, bias=False)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(512, generator=g))
        lin.weight.copy_(torch.randn(768, 512, generator=g) / math.sqrt(512))
    x = torch.randn(1024, 512, generator=g) * 2
    nw, lw = norm.weight.detach().clone(), lin.weight.detach().clone()
    with torch.autocast("cuda", dtype=BF):
        h = norm.to(DEV)(x.to(DEV))
        y = lin.to(DEV)(h)
        x2 = x.to(DEV)[:, :512] + y[:, :512]
    assert h.dtype == torch.float32 and y.dtype == BF and x2.dtype == torch.float32
    h_ref = F.rms_norm(x, (512,), nw, 1e-6)
    assert torch.allclose(h.cpu(), h_ref, rtol=1e-5, atol=1e-6)
    y_ref = R.linear_fused(R.bf(h_ref), R.bf(lw))
    r = ulp_close(y, y_ref, frac=2e-3, atol=2e-3)
    assert r, r
    assert torch.equal(x2.cpu(), x + y[:, :512].float().cpu())


def test_swiglu_of_bf16_products():
    """F.silu(gate) * up of the bf16 gate_up output: silu rounded to bf16, the product rounded to bf16
    (swiglu_fused)."""
    g = gen(3)
    gu = R.bf(torch.randn(4096, 2, 256, generator=g) * 3)
    with torch.autocast("cuda", dtype=BF):
        gd, ud = gu.to(BF).to(DEV).unbind(1)
        out = F.silu(gd) * ud
    assert out.dtype == BF
    r = ulp_close(out, R.swiglu_fused(gu[:, 0], gu[:, 1]))
    assert r, r


def test_embedding_and_projector():
    """nn.Embedding of fp32 weights stays fp32 under autocast (the token rows enter the residual stream unrounded);
    the projector Linear -> GELU -> Linear returns the oracle's bf16 projection (RefModel.project, autocast mode)."""
    from viktor_amd.synthetic import make_model
    m = make_model(1, n_layers=1, seed=4, bias_jitter=0.1)
    tok = torch.tensor([3, 4, 5, 6, 0])
    fr = torch.randn(300, 512, generator=gen(5))
    ref = R.RefModel(m, "autocast")
    emb = m.decoder.embed.weight.detach().clone()
    md = copy.deepcopy(m).to(DEV)
    with torch.autocast("cuda", dtype=BF):
        e = md.decoder.embed(tok.to(DEV))
        p = md.projector(fr.to(DEV))
    assert e.dtype == torch.float32 and torch.equal(e.cpu(), emb[tok])
    assert p.dtype == BF
    r = ulp_close(p, ref.project(fr), frac=5e-3, atol=4e-3)
    assert r, r
