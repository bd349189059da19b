"""The GSPO update's backward and optimizer kernels against fp32 autograd / torch.optim on the CPU, and the
whole decoder's parameter gradients against the oracle's (pinned to finite differences in test_oracle.py).

Bars: element-wise backward kernels to fp32 rounding (bf16 outputs to one bf16 rounding); the attention
backward within 2% of the largest gradient entry (its P and dS are bf16 MFMA operands, as in
flash-attention's backward); AdamW + clip to 1e-5 relative; decoder parameter gradients of the bf16 path
within 10% relative L2 and cosine > 0.99 of the fp32 oracle's.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R
from viktor_amd import hip_ops as ops
from viktor_amd import train as TR

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def gen(seed):
    return torch.Generator().manual_seed(seed)


def _attn_ref(q, k, v, do):
    """fp32 autograd of causal GQA attention of one sequence: (o, lse2 [H, T], dq, dk, dv)."""
    q, k, v = (t.float().clone().requires_grad_(True) for t in (q, k, v))
    T = q.shape[0]
    s = torch.einsum("qhd,khd->hqk", q, k.repeat_interleave(4, 1)) / 8.0
    s = s.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1)[None], float("-inf"))
    lse2 = torch.logsumexp(s, -1) / math.log(2.0)
    o = torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), v.repeat_interleave(4, 1))
    (o * do.float()).sum().backward()
    return o.detach(), lse2.detach(), q.grad, k.grad, v.grad


@pytest.mark.parametrize("lens", [(1, 37, 64, 65, 130), (300,), (64, 64)])
def test_attention_backward(lens):
    g = gen(sum(lens))
    N = sum(lens)
    q = torch.randn(N, 8, 64, generator=g).to(BF)
    k = torch.randn(N, 2, 64, generator=g).to(BF)
    v = torch.randn(N, 2, 64, generator=g).to(BF)
    do = torch.randn(N, 8, 64, generator=g).to(BF)
    plan = TR.TrainPlan(list(lens), DEV)
    lse = torch.empty(N, 8, device=DEV)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    o = ops.varlen_attention(qd, kd, vd, plan.attn, lse=lse)
    dq, dk, dv = (t.cpu() for t in ops.attention_backward(qd, kd, vd, o, dod, lse, plan.attn, plan.keys))
    lse, o = lse.cpu(), o.cpu().float()
    off = 0
    for n in lens:
        sl = slice(off, off + n)
        o_r, lse_r, dq_r, dk_r, dv_r = _attn_ref(q[sl], k[sl], v[sl], do[sl])
        assert (o[sl] - o_r).abs().max() < 1e-2
        assert torch.allclose(lse[sl].t(), lse_r, atol=1e-3, rtol=1e-4), float((lse[sl].t() - lse_r).abs().max())
        for got, ref, name in ((dq[sl], dq_r, "dq"), (dk[sl], dk_r, "dk"), (dv[sl], dv_r, "dv")):
            # (a one-row sequence has dq = 0 exactly: P = 1, so dS = 0; hence the floor on the scale)
            err = float((got - ref).abs().max() / max(float(ref.abs().max()), 0.05))
            assert err < 2e-2, (name, n, err)
        off += n


@pytest.mark.parametrize("pre_lens,G,T", [((300, 129), 3, 100), ((64,), 2, 1), ((1000, 517), 4, 256)])
def test_attention_backward_shared_prefix(pre_lens, G, T):
    """The shared-prefix layout (TrainPlan.shared: each group's prefix rows once, then every member's T token rows
    seeing that prefix) against the same attention over each member's full window [prefix | tokens]: outputs and
    log-sum-exp bit for bit, dQ of the token rows and dK / dV of the token keys to fp32 rounding, and the prefix
    rows' dQ / dK / dV against the unshared sums over the members (dQ: the prefix rows are the same in every
    window; dK / dV: the members' contributions added)."""
    g = gen(sum(pre_lens) + G + T)
    ng = len(pre_lens)
    n_pre, B = sum(pre_lens), ng * G
    N = n_pre + B * T
    q = torch.randn(N, 8, 64, generator=g).to(BF)
    k = torch.randn(N, 2, 64, generator=g).to(BF)
    v = torch.randn(N, 2, 64, generator=g).to(BF)
    do = torch.randn(N, 8, 64, generator=g).to(BF)
    plan = TR.TrainPlan.shared(list(pre_lens), G, T, DEV)
    lse = torch.empty(N, 8, device=DEV)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    o = ops.varlen_attention(qd, kd, vd, plan.attn, lse=lse, prefix=(kd, vd))
    dq, dk, dv = (t.cpu() for t in ops.attention_backward(qd, kd, vd, o, dod, lse, plan.attn, plan.keys))
    # the unshared layout: member b's window = [its group's prefix rows | its token rows]; the prefix rows' dO goes
    # to the first window of each group only (the others' copies get zero), so the windows' sums are the shared ones
    cu_pre = [0]
    for p in pre_lens:
        cu_pre.append(cu_pre[-1] + p)
    rows, share = [], []
    for b in range(B):
        gi = b // G
        rows.append(torch.arange(cu_pre[gi], cu_pre[gi + 1]))
        rows.append(n_pre + b * T + torch.arange(T))
        share.append(torch.full((pre_lens[gi],), 1.0 if b % G == 0 else 0.0))
        share.append(torch.ones(T))
    idx, share = torch.cat(rows), torch.cat(share)
    do_u = (do[idx].float() * share[:, None, None]).to(BF)
    lens_u = [pre_lens[b // G] + T for b in range(B)]
    plan_u = TR.TrainPlan(lens_u, DEV)
    lse_u = torch.empty(idx.numel(), 8, device=DEV)
    qu, ku, vu = (t[idx].contiguous().to(DEV) for t in (q, k, v))
    o_u = ops.varlen_attention(qu, ku, vu, plan_u.attn, lse=lse_u)
    dq_u, dk_u, dv_u = (t.cpu() for t in ops.attention_backward(qu, ku, vu, o_u, do_u.to(DEV), lse_u, plan_u.attn,
                                                                plan_u.keys))
    # forward: every row of the shared layout equals its rows in the windows, bit for bit
    o_c, lse_c = o.cpu(), lse.cpu()
    tok_u = torch.cat([torch.arange(sum(lens_u[:b]) + pre_lens[b // G], sum(lens_u[:b + 1])) for b in range(B)])
    pre_u = torch.cat([torch.arange(sum(lens_u[:b]), sum(lens_u[:b]) + pre_lens[b // G]) for b in range(0, B, G)])
    assert torch.equal(o_c[n_pre:], o_u.cpu()[tok_u]) and torch.equal(lse_c[n_pre:], lse_u.cpu()[tok_u])
    assert torch.equal(o_c[:n_pre], o_u.cpu()[pre_u]) and torch.equal(lse_c[:n_pre], lse_u.cpu()[pre_u])
    # backward: token rows' dQ and the token keys' dK / dV (same sums; dS rounding identical)
    scale = max(float(dq_u.abs().max()), float(dk_u.abs().max()), float(dv_u.abs().max()))
    for got, ref in ((dq[n_pre:], dq_u[tok_u]), (dk[n_pre:], dk_u[tok_u]), (dv[n_pre:], dv_u[tok_u])):
        assert (got - ref).abs().max() <= 1e-5 * scale, float((got - ref).abs().max())
    # prefix rows: dQ from the first window (the only one with their dO); dK / dV summed over the G windows
    assert (dq[:n_pre] - dq_u[pre_u]).abs().max() <= 1e-5 * scale
    for got, ref in ((dk, dk_u), (dv, dv_u)):
        want = torch.zeros(n_pre, 2, 64)
        for b in range(B):
            gi = b // G
            start = sum(lens_u[:b])
            want[cu_pre[gi]:cu_pre[gi + 1]] += ref[start:start + pre_lens[gi]]
        assert (got[:n_pre] - want).abs().max() <= 2e-5 * scale, float((got[:n_pre] - want).abs().max())


def test_rmsnorm_backward():
    g = gen(5)
    n = 77
    x = (torch.randn(n, 512, generator=g) * 2).to(BF)
    w = (torch.rand(512, generator=g) + 0.5).to(BF)
    dy = torch.randn(n, 512, generator=g)
    dres = torch.randn(n, 512, generator=g)
    xx = x.float().requires_grad_(True)
    ww = w.float().requires_grad_(True)
    (F.rms_norm(xx, (512,), ww, 1e-6) * dy).sum().backward()
    for dy_dev in (dy.to(DEV), dy.to(BF).to(DEV)):
        dx, dw = ops.rmsnorm_backward(x.to(DEV), w.to(DEV), dy_dev, 1e-6, dres=dres.to(DEV).clone())
        if dy_dev.dtype == BF:  # the reference with the same bf16-rounded dy
            xx.grad = ww.grad = None
            (F.rms_norm(xx, (512,), ww, 1e-6) * dy.to(BF).float()).sum().backward()
        assert torch.allclose(dx.cpu(), xx.grad + dres, rtol=1e-4, atol=1e-4)
        assert torch.allclose(dw.cpu(), ww.grad, rtol=1e-4, atol=1e-3)


def test_rmsnorm_backward_fp32_stream():
    """The autocast forward's norms: fp32 x (the residual stream) and fp32 weights, with bf16 and fp32 dy."""
    g = gen(15)
    n = 133
    x = torch.randn(n, 512, generator=g) * 2
    w = 1 + 0.1 * torch.randn(512, generator=g)
    dy = torch.randn(n, 512, generator=g)
    dres = torch.randn(n, 512, generator=g)
    for dy_use in (dy, dy.to(BF).float()):
        xx = x.clone().requires_grad_(True)
        ww = w.clone().requires_grad_(True)
        (F.rms_norm(xx, (512,), ww, 1e-6) * dy_use).sum().backward()
        dy_dev = dy_use.to(DEV) if dy_use is dy else dy_use.to(BF).to(DEV)
        dxb = torch.empty(n, 512, dtype=BF, device=DEV)
        dx, dw = ops.rmsnorm_backward(x.to(DEV), w.to(DEV), dy_dev, 1e-6, dres=dres.to(DEV).clone(), dx_bf16=dxb)
        assert torch.allclose(dx.cpu(), xx.grad + dres, rtol=1e-4, atol=1e-4)
        assert torch.allclose(dw.cpu(), ww.grad, rtol=1e-4, atol=1e-3)
        assert torch.equal(dxb, dx.to(BF))  # the bf16 copy is the tensor cast of dx, bit for bit


@pytest.mark.parametrize("wdtype,tdtype,n,H,HKV", [
    ("bf16", "f32", 50, 8, 2), ("f32", "f32", 50, 8, 2), ("f32", "bf16", 3001, 8, 2), ("bf16", "bf16", 1, 8, 2),
    ("f32", "f32", 77, 4, 1)])
def test_qknorm_rope_backward(wdtype, tdtype, n, H, HKV):
    """The norm + rotation backward vs fp32 autograd: both weight and table types, one row, a row count whose
    (row, head) items take several sweeps of the grid and end inside a sweep (3001 x 12), and run-time head counts."""
    g = gen(6)
    qkv = (torch.randn(n, (H + 2 * HKV) * 64, generator=g) * 2).to(BF)
    wq = (torch.rand(64, generator=g) + 0.5)
    wk = (torch.rand(64, generator=g) + 0.5)
    if wdtype == "bf16":
        wq, wk = wq.to(BF), wk.to(BF)
    cos, sin = R.rope_tables(64, 4096, 1e6)
    if tdtype == "bf16":
        cos, sin = cos.to(BF), sin.to(BF)
    rpos = torch.randint(0, 4096, (n,), generator=g).int()
    dq = torch.randn(n, H, 64, generator=g)
    dk = torch.randn(n, HKV, 64, generator=g)
    dv = torch.randn(n, HKV, 64, generator=g)
    x = qkv.float().view(n, H + 2 * HKV, 64)
    q = x[:, :H].clone().requires_grad_(True)
    k = x[:, H:H + HKV].clone().requires_grad_(True)
    wqq, wkk = wq.float().requires_grad_(True), wk.float().requires_grad_(True)
    c, s = cos[rpos.long()].float(), sin[rpos.long()].float()
    loss = (R.apply_rope(F.rms_norm(q, (64,), wqq, 1e-6), c, s) * dq).sum() + \
           (R.apply_rope(F.rms_norm(k, (64,), wkk, 1e-6), c, s) * dk).sum()
    loss.backward()
    want = torch.cat([q.grad, k.grad, dv], 1).reshape(n, -1)
    dqkv, gq, gk = ops.qknorm_rope_backward(qkv.to(DEV), wq.to(DEV), wk.to(DEV), cos.to(DEV), sin.to(DEV),
                                            rpos.to(DEV), dq.to(DEV), dk.to(DEV), dv.to(DEV), 1e-6, H, HKV, 64)
    got = dqkv.cpu().float()
    assert torch.allclose(got, want, rtol=8e-3, atol=1e-4 * want.abs().max()), float((got - want).abs().max())
    assert torch.allclose(gq.cpu(), wqq.grad, rtol=1e-3, atol=1e-3)
    assert torch.allclose(gk.cpu(), wkk.grad, rtol=1e-3, atol=1e-3)


def test_swiglu_backward():
    g = gen(7)
    n, Fd = 40, 1536
    gu = (torch.randn(n, 2 * Fd, generator=g) * 2).to(BF)
    dout = torch.randn(n, Fd, generator=g).to(BF)
    gg = gu.float().requires_grad_(True)
    gate, up = gg.chunk(2, -1)
    (F.silu(gate) * up * dout.float()).sum().backward()
    got = ops.swiglu_backward(gu.to(DEV), dout.to(DEV)).cpu().float()
    assert torch.allclose(got, gg.grad, rtol=8e-3, atol=1e-3), float((got - gg.grad).abs().max())


def test_adamw_with_clip_matches_torch():
    g = gen(8)
    n = 10007
    p0 = torch.randn(n, generator=g)
    ref = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([ref], lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    p, m, v = p0.to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
    for step in range(1, 4):
        grad = torch.randn(n, generator=g) * (3.0 if step == 2 else 0.01)  # step 2 is clipped, the others not
        ref.grad = grad.clone()
        nrm = torch.nn.utils.clip_grad_norm_([ref], 1.0)
        opt.step()
        gd = grad.to(DEV)
        coef = ops.grad_norm_clip(gd, 1.0)
        assert abs(float(coef[0]) - float(nrm)) <= 1e-5 * float(nrm)
        ops.adamw(p, gd, m, v, 3e-3, (0.9, 0.95), 1e-8, 0.01, step, coef=coef)
        assert torch.allclose(p.cpu(), ref.detach(), rtol=1e-5, atol=1e-6), step


def _param_grads_vs_oracle(n_layers, plens, T, seed, pos_scale=1):
    from viktor_amd.synthetic import frames as synth_frames, make_model
    m = make_model(1, n_layers=n_layers, seed=seed, norm_jitter=0.1, bias_jitter=0.1)
    m.pos_scale = pos_scale
    ref = R.RefModel(m, "fp32")
    gm = m.to(DEV)
    g = gen(seed + 1)
    B = len(plens)
    P = max(plens)
    fr = synth_frames(B, P, 512, seed=seed + 2)
    pl = torch.tensor(plens)
    tok = torch.randint(3, 7, (B, T), generator=g)
    targets = torch.randint(3, 7, (B, T), generator=g)
    mask = torch.ones(B, T, dtype=torch.bool)
    mask[0, T - 3:] = False
    n_bases = mask.sum(1).float()
    adv = torch.randn(B, generator=g)
    with torch.no_grad():
        z0 = TR.train_logits(gm, fr.to(DEV), tok.to(DEV), pl.to(DEV))
        old = torch.log_softmax(z0.float(), -1).gather(-1, targets.to(DEV)[..., None])[..., 0].cpu()
    gm.zero_grad(set_to_none=True)
    z = TR.train_logits(gm, fr.to(DEV), tok.to(DEV), pl.to(DEV))
    from viktor_amd.gspo import sequence_ratio_loss
    loss, s, pg, lp = sequence_ratio_loss(z, targets.to(DEV), mask.to(DEV), old.to(DEV), n_bases.to(DEV),
                                          adv.to(DEV), 0.2, 0.2, 1.0 / B)
    loss.backward()
    ref_loss, ref_g = R.gspo_param_grads(ref, fr, tok, pl, targets, mask, old, n_bases, adv, 0.2, 0.2, 1.0 / B)
    assert abs(float(loss) - float(ref_loss)) < 1e-2 * abs(float(ref_loss)) + 1e-4
    worst = []
    for name, p in gm.named_parameters():
        r = ref_g[name]
        got = p.grad.detach().float().cpu() if p.grad is not None else torch.zeros_like(r)
        rel = float((got - r).norm() / (r.norm() + 1e-30))
        cos = float(F.cosine_similarity(got.reshape(1, -1), r.reshape(1, -1)))
        worst.append((rel, cos, name))
        assert rel < 0.1 and cos > 0.99, (name, rel, cos)
    return sorted(worst)[-3:]


def test_decoder_param_grads_match_oracle():
    """Two layers, three windows of different prefix lengths: every projector / decoder parameter's GSPO
    gradient through the HIP training path against the oracle's fp32 autograd."""
    print(_param_grads_vs_oracle(2, [70, 33, 100], 24, seed=31))


def test_decoder_param_grads_pos_scale():
    print(_param_grads_vs_oracle(1, [40, 65], 17, seed=41, pos_scale=2))


@pytest.mark.parametrize("B,P,T", [(1, 200, 64), (4, 2048, 256)])
def test_train_logits_equal_scoring_logits(B, P, T):
    """The update's differentiable forward (train_logits) and the scoring forward (Basecaller.logits, the old
    policy's log-probs) are one function in the reference (scripts/gspo.py:345-347, 471-477), so a first update
    step with unchanged weights sees a sequence ratio of exactly 1. Here they run the same kernels at the same
    rounding points: bit-equal logits, below the large-product row count (small-M products) and above it."""
    from viktor_amd.synthetic import frames, make_model
    m = make_model(1, n_layers=2, seed=11, norm_jitter=0.1, bias_jitter=0.1).to(DEV)
    g = gen(12)
    fr = frames(B, P, 512, seed=13).to(DEV)
    pl = torch.full((B,), P, device=DEV)
    pl[0] = P - 37  # a ragged window
    tok = torch.randint(3, 7, (B, T), generator=g).to(DEV)
    with torch.no_grad():
        z_train = TR.train_logits(m, fr, tok, pl)
        z_score = m.logits(fr, tok, pl)
    assert z_train.shape == z_score.shape == (B, T, 7)
    assert torch.equal(z_train, z_score)


@pytest.mark.parametrize("pre_lens,pos_scale", [((1024, 1024), 1), ((1024, 900), 2)])
def test_train_logits_shared_prefix(pre_lens, pos_scale):
    """train_logits over groups of G windows that share their frames (a GSPO micro-batch of whole groups): the
    logits equal the unshared forward's bit for bit (every product over at least 4096 rows in both forwards), and
    every parameter's gradient is the unshared one's up to the order of the fp32 sums over the members (relative
    L2 < 1e-2, cosine > 0.9999 per tensor)."""
    from viktor_amd.synthetic import make_model
    G, T, P = 4, 256, 1024
    ng = len(pre_lens)
    B = ng * G
    m = make_model(1, n_layers=2, seed=61, norm_jitter=0.1, bias_jitter=0.1).to(DEV)
    m.pos_scale = pos_scale
    g = torch.Generator(device=DEV).manual_seed(62)
    fr = torch.randn(ng, P, 512, generator=g, device=DEV).repeat_interleave(G, 0).contiguous()
    pl = torch.tensor(pre_lens, device=DEV).repeat_interleave(G)
    tok = torch.randint(3, 7, (B, T), generator=torch.Generator().manual_seed(63)).to(DEV)
    w = torch.randn(B, T, 7, generator=g, device=DEV)
    params = [p for p in m.parameters()]

    def grads(group):
        for p in params:
            p.grad = None
        z = TR.train_logits(m, fr, tok, pl, group_size=group)
        (z.float() * w).sum().backward()
        return z.detach(), [p.grad.detach().clone() for p in params]

    z1, g1 = grads(1)
    zg, gg = grads(G)
    assert torch.equal(zg, z1)
    for (name, _), a, b in zip(m.named_parameters(), gg, g1):
        rel = float((a - b).norm() / b.norm().clamp_min(1e-30))
        cos = float(F.cosine_similarity(a.flatten().double(), b.flatten().double(), dim=0))
        assert rel < 1e-2 and cos > 0.9999, (name, rel, cos)


def test_hip_adamw_update_changes_params_in_place():
    """HipAdamW: parameters become views of one flat buffer, a step moves them and keeps the module's
    tensors (the inference copy syncs from them by copy_)."""
    from viktor_amd.synthetic import make_model
    m = make_model(1, n_layers=1, seed=51).to(DEV)
    params = list(m.parameters())
    before = [p.detach().clone() for p in params]
    opt = TR.HipAdamW(params, lr=1e-3)
    for p in params:
        p.grad = torch.ones_like(p)
    opt.step()
    assert float(opt.last_norm[0]) > 1.0 and float(opt.last_norm[1]) < 1.0
    for p, b in zip(params, before):
        assert torch.allclose(p.detach(), b - 1e-3, atol=2e-6)  # Adam's first step moves by lr * sign(g)
        assert p.data.data_ptr() >= opt.flat.data_ptr()


def _update_inputs(seed):
    from viktor_amd.synthetic import frames as synth_frames
    g = gen(seed)
    Bw, G, P = 3, 2, 40
    fr = synth_frames(Bw, P, 512, seed=seed + 1).to(DEV)
    plens = torch.tensor([40, 23, 31], device=DEV)
    rnd = lambda n: "".join("ACGT"[int(i)] for i in torch.randint(0, 4, (n,), generator=g))
    calls = [rnd(int(n)) for n in torch.randint(5, 30, (Bw * G,), generator=g)]
    ended = [bool(e) for e in torch.randint(0, 2, (Bw * G,), generator=g)]
    reward = [[0.5, 0.9], [0.7, 0.7], [0.2, 0.6]]  # window 1 has no learning signal
    labels = [rnd(20), rnd(12), rnd(25)]
    weights = [[1.0] * 20, [1.0] * 5 + [0.0] + [1.0] * 6, [0.5] * 25]
    return fr, plens, calls, ended, reward, labels, weights, G


def test_gspo_update_bookkeeping_matches_direct_gradient():
    from viktor_amd.synthetic import make_model
    from viktor_amd.gspo import advantages, sequence_ratio_loss
    fr, plens, calls, ended, reward, labels, weights, G = _update_inputs(61)
    m1 = make_model(1, n_layers=2, seed=62, norm_jitter=0.1).to(DEV)
    m2 = make_model(1, n_layers=2, seed=62, norm_jitter=0.1).to(DEV)
    opt = TR.HipAdamW(list(m1.parameters()), lr=0.0)
    st = TR.gspo_update(m1, opt, fr, plens, calls, ended, reward, G, updates=1, micro=2, eps=0.2, labels=labels,
                        weights=weights, sft_weight=0.5)
    assert st["n"] == 4 and st["ratio"] == 0.0  # pi_old from the same forward: s = 1 exactly before any step
    # the same update's gradient in one pass over every live call and every window
    adv, live = advantages(torch.tensor(reward, dtype=torch.float64).numpy())
    seqs = [(b, j) for b in live for j in range(G)]
    ix = torch.tensor([b for b, _ in seqs], device=DEV)
    cs = [calls[b * G + j] for b, j in seqs]
    en = [ended[b * G + j] for b, j in seqs]
    logits, targets, mask = TR.token_logprobs_train(m2, fr[ix], plens[ix], cs, en)
    old = ops.gspo_score(logits.detach().contiguous(), targets.clamp(min=0).contiguous())["lp"]
    nb = torch.tensor([float(max(len(c), 1)) for c in cs], device=DEV)
    a = torch.tensor([adv[b, j] for b, j in seqs], device=DEV, dtype=torch.float32)
    loss = sequence_ratio_loss(logits, targets, mask, old, nb, a, 0.2, 0.2, 1.0 / len(seqs))[0]
    loss.backward()
    # the SFT term as scripts/gspo.py:480-484 forms it: per micro-batch of windows, its weighted-mean CE times
    # len(micro-batch) / len(windows) (micro = 2: windows [0, 1] and [2])
    for wb in ([0, 1], [2]):
        w_ix = torch.tensor(wb, device=DEV)
        ce = TR.frame_loss(m2, fr[w_ix], [labels[b] for b in wb], [weights[b] for b in wb], plens=plens[w_ix])
        (0.5 * ce * len(wb) / 3).backward()
    want = torch.cat([p.grad.reshape(-1) for p in m2.parameters()])
    rel = float((opt.grad - want).norm() / want.norm())
    assert rel < 1e-2, rel


def test_gspo_update_steps_move_weights():
    from viktor_amd.synthetic import make_model
    fr, plens, calls, ended, reward, labels, weights, G = _update_inputs(71)
    m = make_model(1, n_layers=2, seed=72).to(DEV)
    before = [p.detach().clone() for p in m.parameters()]
    opt = TR.HipAdamW(list(m.parameters()), lr=1e-4)
    st = TR.gspo_update(m, opt, fr, plens, calls, ended, reward, G, updates=2, micro=3)
    # step 0 takes windows 0 and 2 (both live); step 1 only window 1, whose rewards are equal: no live call,
    # a zero gradient (Adam still moves the weights on its first-step moments)
    assert st["n"] == 4 and len(st["grad_norm"]) == 2 and st["grad_norm"][0] > 0 and st["grad_norm"][1] == 0
    moved = sum(int(not torch.equal(p.detach(), b)) for p, b in zip(m.parameters(), before))
    assert moved >= len(before) - 1  # (the embedding rows of unused tokens still move: Adam on zero grads
    #                                     does nothing only at step 1, so allow one untouched tensor)


@pytest.mark.parametrize("n,ka,kb", [(90112, 3072, 512), (90112, 512, 1536), (4099, 512, 512), (33, 768, 512),
                                     (1000, 256, 128), (64 * 1024 + 17, 768, 512)])
def test_wgrad_kernel_against_fp64(n, ka, kb):
    """vk_wgrad (MFMA over LDS transpose reads, row slices summed in order): a^T b against the fp64 product, fp32
    output within fp32 accumulation error, bf16 output within one rounding of it; ragged row counts (the masked
    last step), a single slice (33 rows) and the update's shapes (gate_up, down at 90112 packed rows)."""
    g = gen(n + ka)
    a = (torch.randn(n, ka, generator=g) * 0.1).to(BF)
    b = (torch.randn(n, kb, generator=g) * 0.1).to(BF)
    ad, bd = a.to(DEV), b.to(DEV)
    a64, b64 = ad.double(), bd.double()  # the fp64 reference products on the device (exact bf16 inputs)
    want = a64.t() @ b64
    scale = a64.abs().t() @ b64.abs()  # sum of |terms|: the scale of the fp32 accumulation error
    del a64, b64
    got32 = ops.wgrad(ad, bd, out_dtype=torch.float32).double()
    assert bool(((got32 - want).abs() <= scale * 2.0 ** -20 + 1e-9).all()), float((got32 - want).abs().max())
    got16 = ops.wgrad(ad, bd).double()
    assert bool(((got16 - want).abs() <= want.abs() * 2.0 ** -8 + scale * 2.0 ** -20 + 1e-9).all())
    assert torch.equal(ops.wgrad(ad, bd), ops.wgrad(ad, bd))  # deterministic
    # a strided view (rows of a wider buffer), as the backward's slices of packed activations are
    wide = torch.zeros(n, ka + 64, dtype=BF, device=DEV)
    wide[:, 32:32 + ka] = ad
    assert torch.equal(ops.wgrad(wide[:, 32:32 + ka], bd, out_dtype=torch.float32).double(), got32)


@pytest.mark.parametrize("n,d", [(3000, 512), (77, 136), (4099, 1024)])
def test_projector_bias_gelu_forward_and_backward(n, d):
    """vk_bias_act / vk_act_backward against fp64 on the CPU: pre = bf16(y + b) exactly; out = bf16(gelu(pre)) and
    din = bf16(dout gelu'(pre)) within one bf16 rounding of the fp64 values plus the fp32 cancellation of
    1 + erf(x / sqrt 2) at negative x (2^-21 |x| for gelu, 2^-19 |dout| for its derivative); the bias gradients
    (column sums) to fp32 accumulation error."""
    g = gen(n + d)
    y = torch.randn(n, d, generator=g) * 3
    b = torch.randn(d, generator=g).to(BF).float()
    pre, out = (t.cpu().float() for t in ops.bias_act(y.to(DEV), b.to(DEV), gelu=True))
    want_pre = (y + b).to(BF).float()
    assert torch.equal(pre, want_pre)
    x64 = want_pre.double()
    cdf = 0.5 * (1 + torch.special.erf(x64 / math.sqrt(2)))
    want_out = x64 * cdf
    err = (out.double() - want_out).abs()
    assert bool((err <= want_out.abs() * 2.0 ** -8 + x64.abs() * 2.0 ** -21 + 1e-30).all()), float(err.max())
    plain = ops.bias_act(y.to(DEV), b.to(DEV), gelu=False).cpu().float()
    assert torch.equal(plain, want_pre)
    dout = torch.randn(n, d, generator=g).to(BF)
    din, gb = ops.act_backward(dout.to(DEV), pre.to(BF).to(DEV))
    want_din = dout.double() * (cdf + x64 * torch.exp(-0.5 * x64 * x64) / math.sqrt(2 * math.pi))
    got_din = din.cpu().float()
    err = (got_din.double() - want_din).abs()
    assert bool((err <= want_din.abs() * 2.0 ** -8 + dout.double().abs() * 2.0 ** -19 + 1e-30).all()), float(err.max())
    ref_gb = got_din.double().sum(0)
    scale = got_din.double().abs().sum(0)
    assert bool(((gb.cpu().double() - ref_gb).abs() <= scale * 2.0 ** -20).all())
    gb2 = ops.act_backward(dout.to(DEV)).cpu().double()
    assert bool(((gb2 - dout.double().sum(0)).abs() <= dout.double().abs().sum(0) * 2.0 ** -20).all())
    assert torch.equal(ops.act_backward(dout.to(DEV)), ops.act_backward(dout.to(DEV)))  # fixed order


@pytest.mark.parametrize("n,V,d", [(32 * 1024 + 5, 7, 512), (5000, 343, 512), (999, 70, 1024), (300, 7, 136),
                                   (0, 7, 512)])
def test_embed_grad_against_fp64(n, V, d):
    """vk_embed_grad: per-token sums of the gradient rows against the fp64 index_add on the CPU: 7 ids (the base
    vocabulary), 343 and 70 (several 32-id chunks, the last ragged), two 512-column blocks, a partial block
    (d = 136), no rows at all; ids outside [0, V) add nothing; repeated calls are bit-identical."""
    g = gen(n + V + d)
    tok = torch.randint(0, V, (n,), generator=g)
    if n > 10:
        tok[3], tok[7] = V, -1  # out of range: ignored
    rows = torch.randn(n, d, generator=g).to(BF)
    got = ops.embed_grad(rows.to(DEV), tok.to(DEV), V).cpu().double()
    if n > 10:  # an id that only its low 32 bits would put in range is ignored too
        tok2 = tok.clone()
        tok2[5] = (1 << 32) + 3
        keep2 = (tok2 >= 0) & (tok2 < V)
        want2 = torch.zeros(V, d, dtype=torch.float64).index_add_(0, tok2[keep2], rows[keep2].double())
        got2 = ops.embed_grad(rows.to(DEV), tok2.to(DEV), V).cpu().double()
        assert torch.allclose(got2, want2, rtol=0, atol=1e-4)
        # fp32 gradient rows (the autocast forward's fp32 residual gradient): fp32 sums of the fp32 rows
        r32 = torch.randn(n, d, generator=g)
        g32 = ops.embed_grad(r32.to(DEV), tok.to(DEV), V).cpu().double()
        w32 = torch.zeros(V, d, dtype=torch.float64).index_add_(0, tok[(tok >= 0) & (tok < V)],
                                                              r32[(tok >= 0) & (tok < V)].double())
        s32 = torch.zeros(V, d, dtype=torch.float64).index_add_(0, tok[(tok >= 0) & (tok < V)],
                                                              r32[(tok >= 0) & (tok < V)].double().abs())
        assert bool(((g32 - w32).abs() <= s32 * 2.0 ** -20).all())
    keep = (tok >= 0) & (tok < V)
    want = torch.zeros(V, d, dtype=torch.float64).index_add_(0, tok[keep], rows[keep].double())
    scale = torch.zeros(V, d, dtype=torch.float64).index_add_(0, tok[keep], rows[keep].double().abs())
    assert bool(((got - want).abs() <= scale * 2.0 ** -20).all()), float((got - want).abs().max())
    if n:
        assert torch.equal(ops.embed_grad(rows.to(DEV), tok.to(DEV), V), ops.embed_grad(rows.to(DEV), tok.to(DEV), V))
        # a strided view (rows of a wider buffer)
        wide = torch.zeros(n, d + 16, dtype=BF, device=DEV)
        wide[:, 8:8 + d] = rows.to(DEV)
        assert torch.equal(ops.embed_grad(wide[:, 8:8 + d], tok.to(DEV), V).cpu().double(), got)


@pytest.mark.parametrize("V", [7, 343])
def test_lm_head_backward_products(V):
    """_LMHead: logits = bf16(h W^T) and its backward (dh = dz W, dW = dz^T h through the zero-padded V-wide
    operand) against fp64 products of the same bf16 operands, each within one bf16 rounding plus fp32 error."""
    g = gen(V)
    n = 4500
    h = (torch.randn(n, 512, generator=g)).to(BF)
    w = torch.randn(V, 512, generator=g) * 0.05
    dz = (torch.randn(n, V, generator=g) * 0.1).to(BF)
    hd = h.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    z = TR._LMHead.apply(hd, wd)
    z.backward(dz.to(DEV))
    wb = w.to(BF).double()
    for got, want, scale in ((z.detach(), h.double() @ wb.t(), h.double().abs() @ wb.abs().t()),
                             (hd.grad, dz.double() @ wb, dz.double().abs() @ wb.abs()),
                             (wd.grad, dz.double().t() @ h.double(), dz.double().abs().t() @ h.double().abs())):
        got = got.cpu().double()
        assert bool(((got - want).abs() <= want.abs() * 2.0 ** -8 + scale * 2.0 ** -20 + 1e-12).all()), \
            float((got - want).abs().max())
