"""The CPU oracle pinned against the reference's golden vectors, closed forms and brute force (no GPU)."""

import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R
from viktor_amd import KmerTokenizer
from viktor_amd.decoder import Decoder, DecoderConfig, rope_tables
from viktor_amd.synthetic import init_params, make_model

from .conftest import GOLDEN

TINY = dict(d_model=32, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=8, ffn_dim=64, max_seq_len=512, rope_theta=1e4)
FULL2 = dict(d_model=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=1536, max_seq_len=4096,
             rope_theta=1e6)
CFGS = {"tiny": TINY, "full2": FULL2}


def npz(name):
    return np.load(os.path.join(GOLDEN, name))


def checksum(module):
    s = sq = 0.0
    for _, p in sorted(module.named_parameters()):
        d = p.detach().double()
        s += float(d.sum())
        sq += float((d * d).sum())
    return np.array([s, sq])


# ---- golden: rope tables, tokenizer --------------------------------------------------------------
def test_rope_tables_match_reference_bitwise():
    z = npz("rope.npz")
    rows = z["rows"]
    for theta in (10000, 1000000):
        c, s = rope_tables(64, 4096, float(theta))
        assert np.array_equal(c[rows].numpy(), z[f"cos_{theta}"])
        assert np.array_equal(s[rows].numpy(), z[f"sin_{theta}"])
        c2, s2 = R.rope_tables(64, 4096, float(theta))
        assert torch.equal(c, c2) and torch.equal(s, s2)


def test_tokenizer_matches_reference():
    with open(os.path.join(GOLDEN, "tokenizer.json")) as f:
        g = json.load(f)
    for k in (1, 4):
        tk = KmerTokenizer(k)
        ref = g[str(k)]
        assert tk.strings == ref["strings"]
        assert tk.tail_mask.int().tolist() == ref["tail_mask"]
        assert tk.n_bases.tolist() == ref["n_bases"]
        assert [tk.encode(s) for s in ref["seqs"]] == ref["ids"]
        for ids, want in ref["decode_cases"]:
            assert tk.decode(ids) == want
        tin, tgt, nb = tk.batch([s for s in ref["seqs"] if s])
        assert tin.tolist() == ref["batch_in"] and tgt.tolist() == ref["batch_tgt"] and nb == ref["batch_bases"]


# ---- golden: decoder forward ---------------------------------------------------------------------
@pytest.mark.parametrize("name", ["tiny", "full2"])
def test_oracle_decoder_forward_matches_reference(name):
    z = npz("decoder.npz")
    cfg = DecoderConfig(vocab_size=7, **CFGS[name])
    dec = Decoder(cfg)
    init_params(dec, int(z[f"{name}_seed"]), norm_jitter=0.1)
    assert np.allclose(checksum(dec), z[f"{name}_checksum"], rtol=1e-12), "seeded init drifted"

    ref = R.RefModel.from_decoder(dec, "fp32")
    x = torch.from_numpy(z[f"{name}_x"])
    pos = torch.from_numpy(z[f"{name}_pos"])
    h = ref.decoder_forward(x)
    h_pos = ref.decoder_forward(x, positions=pos)
    tol = dict(rtol=1e-4, atol=2e-5)
    assert torch.allclose(h, torch.from_numpy(z[f"{name}_h"]), **tol)
    assert torch.allclose(h_pos, torch.from_numpy(z[f"{name}_h_pos"]), **tol)
    logits = ref.head(h, round_bf16=False)
    assert torch.allclose(logits, torch.from_numpy(z[f"{name}_logits"]), **tol)
    # a plausible wiring mistake must fail: swapping the k and v head groups changes the output
    ref.p = dict(ref.p)
    w = ref.p["decoder.layers.0.attn.qkv_proj.weight"].clone()
    H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    w[H * D:(H + Hkv) * D], w[(H + Hkv) * D:] = w[(H + Hkv) * D:].clone(), w[H * D:(H + Hkv) * D].clone()
    ref.p["decoder.layers.0.attn.qkv_proj.weight"] = w
    assert not torch.allclose(ref.decoder_forward(x), torch.from_numpy(z[f"{name}_h"]), **tol)


# ---- golden: engine greedy streams -----------------------------------------------------------------
ENGINE_CASES = ["tiny_k1", "tiny_k4", "full2_k1", "full2_k4", "tiny_k1_ps2"]


def _engine_model(z, name):
    k, seed, steps, mh, ps, d_enc = [int(v) for v in z[f"{name}_meta"]]
    cfg = TINY if name.startswith("tiny") else FULL2
    m = make_model(k, seed=seed, d_enc=d_enc, norm_jitter=0.1, bias_jitter=0.1, **cfg)
    m.pos_scale = ps
    assert np.allclose(checksum(m), z[f"{name}_checksum"], rtol=1e-12), "seeded init drifted"
    return m, steps, mh


@pytest.mark.parametrize("name", ENGINE_CASES)
def test_oracle_engine_matches_reference_stream(name):
    z = npz("engine.npz")
    m, steps, mh = _engine_model(z, name)
    lens = z[f"{name}_lens"].tolist()
    frames = torch.from_numpy(z[f"{name}_frames"])
    fl = list(frames.split(lens))
    eng = R.RefEngine(R.RefModel(m, "fp32"), steps, max_homopolymer=mh)
    res = eng.run(fl)
    assert torch.equal(res["tokens"], torch.from_numpy(z[f"{name}_tokens"]))


def test_oracle_engine_cached_equals_full_recompute():
    """The reference's own engine invariant (tests/test_viktor.py:71-83), incl. the homopolymer rule."""
    z = npz("engine.npz")
    for name in ("tiny_k1", "tiny_k4"):
        m, steps, mh = _engine_model(z, name)
        lens = z[f"{name}_lens"].tolist()
        fl = list(torch.from_numpy(z[f"{name}_frames"]).split(lens))
        ref = R.RefModel(m, "fp32")
        cached = R.RefEngine(ref, steps, max_homopolymer=mh).run(fl)["tokens"]
        full = R.greedy_full_recompute(ref, fl, steps, max_homopolymer=mh)
        assert torch.equal(cached, full)


def test_oracle_engine_forced_history_reproduces_own_stream():
    z = npz("engine.npz")
    m, steps, mh = _engine_model(z, "tiny_k4")
    lens = z["tiny_k4_lens"].tolist()
    fl = list(torch.from_numpy(z["tiny_k4_frames"]).split(lens))
    eng = R.RefEngine(R.RefModel(m, "fp32"), steps, max_homopolymer=mh)
    free = eng.run(fl)
    forced = eng.run(fl, forced=free["tokens"])
    assert torch.equal(forced["choice"], free["tokens"][:, :steps])


# ---- golden: teacher-forced logits ----------------------------------------------------------------
@pytest.mark.parametrize("name", ["tiny_k4", "full2_k1", "tiny_k1_ps4"])
def test_oracle_teacher_forced_logits_match_reference(name):
    z = npz("logits.npz")
    k, seed, ps, d_enc = [int(v) for v in z[f"{name}_meta"]]
    cfg = TINY if name.startswith("tiny") else FULL2
    m = make_model(k, seed=seed, d_enc=d_enc, norm_jitter=0.1, bias_jitter=0.1, **cfg)
    m.pos_scale = ps
    assert np.allclose(checksum(m), z[f"{name}_checksum"], rtol=1e-12)
    seqs = [str(s) for s in z[f"{name}_seqs"]]
    tin, tgt, w = m.batch(seqs, pad_to=8)
    assert np.array_equal(tin.numpy(), z[f"{name}_tokens_in"]) and np.array_equal(tgt.numpy(), z[f"{name}_targets"])
    assert np.array_equal(w.numpy(), z[f"{name}_w"])
    ref = R.RefModel(m, "fp32")
    lg = ref.logits(torch.from_numpy(z[f"{name}_frames"]), tin, torch.from_numpy(z[f"{name}_plens"]))
    assert torch.allclose(lg, torch.from_numpy(z[f"{name}_logits"]), rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("name", ["tiny_k4", "full2_k1", "tiny_k1_ps4"])
def test_oracle_autocast_logits_near_reference_and_closer_than_fused(name):
    """The autocast mode (the reference's scoring numerics) against the reference's fp32 golden logits: within the
    bf16 rounding of the logits themselves (one ulp is 1.6e-2 at |z| in [2, 4)), and on average closer than the
    fused mode -- whose bf16 residual stream rounds every block's sum -- so a restatement that let the residual
    fall back to bf16 fails. The two modes differ on most logits."""
    z = npz("logits.npz")
    k, seed, ps, d_enc = [int(v) for v in z[f"{name}_meta"]]
    cfg = TINY if name.startswith("tiny") else FULL2
    m = make_model(k, seed=seed, d_enc=d_enc, norm_jitter=0.1, bias_jitter=0.1, **cfg)
    m.pos_scale = ps
    tin, _, _ = m.batch([str(s) for s in z[f"{name}_seqs"]], pad_to=8)
    gold = torch.from_numpy(z[f"{name}_logits"])
    fr, pl = torch.from_numpy(z[f"{name}_frames"]), torch.from_numpy(z[f"{name}_plens"])
    ac = R.RefModel(m, "autocast").logits(fr, tin, pl)
    fu = R.RefModel(m, "fused").logits(fr, tin, pl)
    assert torch.equal(ac, R.bf(ac))  # bf16 logits
    e_ac, e_fu = (ac - gold).abs(), (fu - gold).abs()
    assert float(e_ac.max()) < 3e-2, float(e_ac.max())
    assert float(e_ac.mean()) < 0.85 * float(e_fu.mean()), (float(e_ac.mean()), float(e_fu.mean()))
    assert float((ac != fu).float().mean()) > 0.3


def test_oracle_autocast_parameters():
    """What autocast casts: every nn.Linear weight and bias of the projector and decoder is used as its bf16
    rounding; the RMSNorm weights (QK-norm included), the embedding and the rotary tables stay fp32."""
    m = make_model(4, seed=3, norm_jitter=0.1, bias_jitter=0.1, **FULL2)
    ref = R.RefModel(m, "autocast")
    for n, p in m.named_parameters():
        want = p.detach().float()
        if n.endswith("bias") or (p.dim() == 2 and not n.endswith("embed.weight")):
            want = R.bf(want)
        assert torch.equal(ref.p[n], want), n
    assert any(not torch.equal(R.bf(p), p) for n, p in m.named_parameters() if "norm" in n)
    cos, sin = rope_tables(64, 4096, 1e6)
    assert torch.equal(ref.cos, cos) and torch.equal(ref.sin, sin)


# ---- closed forms / brute force for the fused-mode ops ---------------------------------------------
def test_fused_rmsnorm_closed_form():
    g = torch.Generator().manual_seed(0)
    x = R.bf(torch.randn(5, 64, generator=g))
    d = R.bf(torch.randn(5, 64, generator=g))
    w = R.bf(torch.rand(64, generator=g) + 0.5)
    xn, h = R.add_rmsnorm_fused(x, d, w, 1e-6)
    xd = x.double() + d.double()
    assert torch.equal(xn, R.bf(xd.float()))  # the bf16 sum of two bf16 values is the rounded exact sum
    ref = xn.double() / torch.sqrt((xn.double() ** 2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(h.double(), ref, rtol=8e-3, atol=1e-6)
    assert torch.allclose(h, R.bf(F.rms_norm(xn, (64,), w, 1e-6)), atol=1e-2)


def test_fused_rope_is_a_rotation():
    g = torch.Generator().manual_seed(1)
    x = R.bf(torch.randn(3, 8, 64, generator=g))
    w = torch.ones(64)
    cos, sin = R.rope_tables(64, 100, 1e4)
    p = torch.tensor([0, 7, 99])
    y = R.qk_norm_rope_fused(x, w, cos[p], sin[p], 1e-6)
    nrm = R.qk_norm_rope_fused(x, w, cos[[0, 0, 0]], sin[[0, 0, 0]], 1e-6)  # position 0: no rotation
    # norms preserved by the rotation (up to bf16 rounding), position 0 = pure RMSNorm
    assert torch.allclose(y.norm(dim=-1), nrm.norm(dim=-1), rtol=2e-2)
    xn = x / torch.sqrt((x ** 2).mean(-1, keepdim=True) + 1e-6)
    assert torch.allclose(nrm, xn, atol=2e-2)
    # half-split pairing: element i rotates with element i + 32 at angle p * theta^(-2i/64)
    i = 5
    ang = 7 * 10000.0 ** (-2 * i / 64)
    a, b = nrm[1, 0, i], nrm[1, 0, i + 32]
    assert abs(float(y[1, 0, i] - (a * math.cos(ang) - b * math.sin(ang)))) < 2e-2
    assert abs(float(y[1, 0, i + 32] - (a * math.sin(ang) + b * math.cos(ang)))) < 2e-2


def test_attention_rows_brute_force():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(5, 8, 64, generator=g)
    k = torch.randn(9, 2, 64, generator=g)
    v = torch.randn(9, 2, 64, generator=g)
    o = R.attention_rows(q, k, v, causal_shift=4)
    for r in range(5):
        for h in range(8):
            kh = h // 4
            n = 4 + r + 1
            s = (q[r, h].double() @ k[:n, kh].double().t()) / 8.0
            ref = torch.softmax(s, 0) @ v[:n, kh].double()
            assert torch.allclose(o[r, h].double(), ref, atol=1e-5)
    # special cases: one key -> its value; equal keys -> the mean of the values
    o1 = R.attention_rows(q[:1], k[:1], v[:1])
    assert torch.allclose(o1[0], v[0].repeat_interleave(4, 0), atol=1e-6)
    ke = k[:1].expand(9, 2, 64)
    oe = R.attention_rows(q[:1], ke, v)
    assert torch.allclose(oe[0], v.mean(0).repeat_interleave(4, 0), atol=1e-5)


def test_attention_rows_bf16_weights_brute_force():
    """p_bf16: o = sum_j bf16(exp(s_j - max)) v_j / sum_j exp(s_j - max), per query row and head, in fp64 on a
    tiny case; equal keys give exactly the mean of the values (every weight is exp(0) = 1, exact in bf16); and a
    planted mistake -- normalising by the rounded weights -- is caught by the brute force."""
    g = torch.Generator().manual_seed(12)
    q = torch.randn(3, 8, 64, generator=g)
    k = torch.randn(7, 2, 64, generator=g)
    v = torch.randn(7, 2, 64, generator=g)
    o = R.attention_rows(q, k, v, causal_shift=4, p_bf16=True)

    def brute(o, rounded_norm=False):
        for r in range(3):
            for h in range(8):
                n = 4 + r + 1
                s = (q[r, h].double() @ k[:n, h // 4].double().t()) / 8.0
                e = torch.exp(s - s.max())
                eb = e.float().to(torch.bfloat16).double()
                ref = eb @ v[:n, h // 4].double() / (eb.sum() if rounded_norm else e.sum())
                if not torch.allclose(o[r, h].double(), ref, atol=2e-6):
                    return False
        return True

    assert brute(o)
    assert not brute(o, rounded_norm=True)
    exact = R.attention_rows(q, k, v, causal_shift=4)
    assert 0 < float((o - exact).abs().max()) < 2e-2  # a bf16 rounding of the weights, no more
    ke = k[:1].expand(7, 2, 64)
    oe = R.attention_rows(q[:1], ke, v, p_bf16=True)
    assert torch.allclose(oe[0], v.mean(0).repeat_interleave(4, 0), atol=1e-6)


def test_attention_rows_blockwise_bf16_weights_brute_force():
    """block: each query row's keys in blocks visited from the last to the first; a block's weights are
    bf16(exp(s - m_b)) with m_b the running max after that block, the accumulator and the fp32 normaliser rescaled
    by exp(m_old - m_b). Brute force per row in fp64 of that recurrence; one block covering every key equals the
    final-maximum rounding exactly; causal rows whose first visited blocks are fully masked."""
    g = torch.Generator().manual_seed(13)
    q = torch.randn(20, 8, 64, generator=g)
    k = torch.randn(45, 2, 64, generator=g) * 2
    v = torch.randn(45, 2, 64, generator=g)
    o = R.attention_rows(q, k, v, causal_shift=25, p_bf16=True, block=8)
    for r in (0, 7, 19):
        for h in (0, 5):
            n = 25 + r + 1
            s = (q[r, h].double() @ k[:n, h // 4].double().t()) / 8.0
            m, l, acc = -math.inf, 0.0, torch.zeros(64, dtype=torch.float64)
            for b0 in reversed(range(0, 45, 8)):
                sb = s[b0:min(b0 + 8, n)]
                if sb.numel() == 0:
                    continue
                mb = max(m, float(sb.max()))
                sc = math.exp(m - mb) if m > -math.inf else 0.0
                e = torch.exp(sb - mb)
                l = l * sc + float(e.sum())
                acc = acc * sc + e.float().to(torch.bfloat16).double() @ v[b0:b0 + sb.numel(), h // 4].double()
                m = mb
            assert torch.allclose(o[r, h].double(), acc / l, atol=2e-6)
    whole = R.attention_rows(q, k, v, causal_shift=25, p_bf16=True, block=64)
    assert torch.allclose(whole, R.attention_rows(q, k, v, causal_shift=25, p_bf16=True), atol=1e-6)
    assert 0 < float((o - whole).abs().max()) < 2e-2


def test_swiglu_fused_closed_form():
    g = R.bf(torch.linspace(-6, 6, 97))
    u = R.bf(torch.linspace(2, -3, 97))
    out = R.swiglu_fused(g, u)
    ref = (g.double() / (1 + torch.exp(-g.double()))) * u.double()
    assert torch.allclose(out.double(), ref, rtol=1.6e-2, atol=1e-3)


# ---- token choice -----------------------------------------------------------------------------------
def test_inverse_cdf_boundaries():
    z = torch.tensor([float("-inf"), float("-inf"), 0.3, -1.0, 2.0, 0.0, 0.5])
    p = torch.softmax(z.double(), 0)
    cdf = torch.cumsum(p, 0)
    assert R.sample_inverse_cdf(z, 0.0)[0] == 2  # u -> 0 picks the first non-banned token
    for v in range(2, 7):
        assert R.sample_inverse_cdf(z, float(cdf[v]) - 1e-4)[0] == v  # just below C_v picks v
        if v < 6:
            assert R.sample_inverse_cdf(z, float(cdf[v]) + 1e-4)[0] == v + 1
    assert R.sample_inverse_cdf(z, 0.9999999)[0] == 6


def test_gumbel_choice_closed_form_and_frequencies():
    """sample_gumbel: the first argmax of z - log(-log(max(u, 1e-20))) (brute force in fp64 on random draws, and
    u = 0 taking the clamp), banned entries never chosen; over 200k draws each token's frequency is softmax(z)
    within 4 binomial standard deviations (Gumbel-max samples the softmax; a sign slip in either log would not)."""
    z = torch.tensor([float("-inf"), float("-inf"), 0.3, -1.0, 2.0, 0.0, 0.5])
    rng = np.random.default_rng(5)
    for _ in range(200):
        u = rng.random(7).astype(np.float32)
        u[rng.integers(0, 7)] = 0.0 if rng.random() < 0.1 else u[0]
        v, gap = R.sample_gumbel(z, u)
        g = z.double().numpy() - np.log(-np.log(np.maximum(u.astype(np.float64), 1e-20)))
        assert v == int(np.argmax(g)) and v >= 2 and gap >= 0
    n = 200000
    U = torch.from_numpy(rng.random((n, 7)).astype(np.float32)).clamp(min=1e-20)
    G = z[None] - torch.log(-torch.log(U))
    counts = torch.bincount(G.argmax(1), minlength=7).double()
    picks = [R.sample_gumbel(z, U[i].numpy())[0] for i in range(2000)]
    assert picks == G[:2000].argmax(1).tolist()
    p = torch.softmax(z.double(), 0)
    sd = torch.sqrt(n * p * (1 - p))
    assert bool(((counts - n * p).abs() <= 4 * sd + 1e-9).all()), (counts / n, p)


def test_inverse_cdf_frequencies():
    g = torch.Generator().manual_seed(3)
    z = torch.randn(7, generator=g) * 1.5
    z[0] = z[1] = float("-inf")
    p = torch.softmax(z.double(), 0).numpy()
    u = torch.rand(20000, generator=g)
    counts = np.bincount([R.sample_inverse_cdf(z, float(x))[0] for x in u], minlength=7)
    expected = p * len(u)
    chi2 = (((counts - expected) ** 2) / np.maximum(expected, 1e-9))[2:].sum()
    assert counts[0] == counts[1] == 0 and chi2 < 25  # 4 dof: p(chi2 > 25) < 1e-4


def test_grammar_rules():
    tail = torch.tensor([False] * 5 + [True, True])
    homo = torch.tensor([False, False, False, True, True, False, False])
    assert R.apply_grammar(3, 5, 0, tail, homo, 0) == (R.EOS, 0)        # after a tail -> EOS
    assert R.apply_grammar(3, 3, 2, tail, homo, 4) == (R.EOS, 3)        # run reaches homo_stop -> EOS
    assert R.apply_grammar(3, 3, 1, tail, homo, 4) == (3, 2)
    assert R.apply_grammar(4, 3, 2, tail, homo, 4) == (4, 0)            # different token resets the run
    assert R.apply_grammar(4, R.EOS, 0, tail, homo, 4)[0] == R.PAD      # after EOS -> PAD
    assert R.apply_grammar(4, R.PAD, 0, tail, homo, 4)[0] == R.PAD


# ---- GSPO ---------------------------------------------------------------------------------------------
def _gspo_inputs(seed=0, B=6, T=11, V=7):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, T, V, generator=g) * 2
    targets = torch.randint(3, V, (B, T), generator=g)
    mask = torch.rand(B, T, generator=g) > 0.2
    lp = torch.log_softmax(logits, -1).gather(-1, targets[..., None])[..., 0]
    old = lp + torch.randn(B, T, generator=g) * 1e-3
    n_bases = torch.randint(1, T + 1, (B,), generator=g).float()
    adv = torch.randn(B, generator=g)
    adv[0] = 0.0
    return logits, targets, mask, old, n_bases, adv


def test_gspo_autograd_matches_closed_form():
    logits, targets, mask, old, nb, adv = _gspo_inputs()
    for elo, ehi in ((3e-4, 4e-4), (1.0, 1.0), (1e-9, 1e-9)):
        loss, s, pg, lp, grad = R.gspo_loss_autograd(logits, targets, mask, old, nb, adv, elo, ehi, 1 / 6)
        closed = R.gspo_grad_closed_form(logits, targets, mask, old, nb, adv, elo, ehi, 1 / 6)
        assert torch.allclose(grad.double(), closed, atol=1e-7)
        assert torch.all(grad[0] == 0)  # A = 0 -> zero gradient


def test_gspo_special_cases():
    logits, targets, mask, _, nb, adv = _gspo_inputs(1)
    lp = R.token_logprobs_ref(logits, targets)
    loss, s, pg, _, grad = R.gspo_loss_autograd(logits, targets, mask, lp, nb, adv, 3e-4, 4e-4, 1.0)
    assert torch.allclose(s, torch.ones_like(s))        # old == new -> ratio 1
    assert torch.allclose(pg, -adv)                      # -> pg = -A
    assert torch.allclose(loss, -adv.sum())
    # a clipped sequence (A > 0, s above 1 + eps_hi) has no gradient
    old = lp.clone()
    old[2] -= 0.5
    adv2 = adv.clone()
    adv2[2] = 1.0
    _, s2, _, _, g2 = R.gspo_loss_autograd(logits, targets, mask, old, nb, adv2, 3e-4, 4e-4, 1.0)
    assert s2[2] > 1 + 4e-4 and torch.all(g2[2] == 0)


def test_advantages_ref():
    r = np.array([[0.5, 0.7, 0.9, 0.9], [0.8, 0.8, 0.8, 0.8], [0.1, 0.2, 0.3, 0.9]])
    adv, live = R.advantages_ref(r)
    assert list(live) == [0, 2]
    sd = r[0].std()
    assert np.allclose(adv[0], (r[0] - r[0].mean()) / sd)
    assert np.allclose(adv[1], 0)
    adv_e, _ = R.advantages_ref(r, eps=1e-6)
    assert np.allclose(adv_e[2], (r[2] - r[2].mean()) / (r[2].std() + 1e-6))


def test_sampled_mask_rule():
    tk = KmerTokenizer(4)
    seqs = ["ACGTAC", "ACGT", "ACG"]
    tin, tgt, _ = tk.batch(seqs)
    m = R.sampled_mask_ref(tgt, seqs, [True, True, False], 4)
    # "ACGTAC": 2 tokens (last one a tail) + EOS forced after the tail -> EOS not sampled
    assert m[0].tolist() == [True, True, False]
    # "ACGT" ended by a sampled EOS -> kept
    assert m[1].tolist() == [True, True, False]
    # "ACG" did not end -> its EOS target is dropped
    assert m[2].tolist() == [True, False, False]


def test_gspo_param_grads_match_finite_differences():
    """The oracle's parameter gradients of the GSPO loss (autograd through the fp32 restatement) against
    central differences in fp64 on a one-layer model: pins the gradient oracle the update's HIP backward is
    checked against. The clip range is wide (no clamp), so the objective is smooth."""
    from viktor_amd.synthetic import frames as synth_frames, make_model
    m = make_model(1, n_layers=1, seed=21, norm_jitter=0.1, bias_jitter=0.1)
    ref = R.RefModel(m, "fp32")
    g = torch.Generator().manual_seed(22)
    fr = synth_frames(2, 9, 512, seed=23)
    plens = torch.tensor([9, 5])
    tok = torch.randint(3, 7, (2, 4), generator=g)
    targets = torch.randint(3, 7, (2, 4), generator=g)
    mask = torch.ones(2, 4, dtype=torch.bool)
    mask[1, 3] = False
    old = -1.5 + 0.1 * torch.randn(2, 4, generator=g)
    n_bases = torch.tensor([4.0, 3.0])
    adv = torch.tensor([0.7, -1.2])
    args = (fr, tok, plens, targets, mask, old, n_bases, adv, 10.0, 10.0, 0.5)
    loss, grads = R.gspo_param_grads(ref, *args, dtype=torch.float64)
    names = ["projector.0.weight", "projector.2.bias", "decoder.embed.weight", "decoder.layers.0.attn_norm.weight",
             "decoder.layers.0.attn.qkv_proj.weight", "decoder.layers.0.attn.q_norm.weight",
             "decoder.layers.0.attn.k_norm.weight", "decoder.layers.0.attn.o_proj.weight",
             "decoder.layers.0.gate_up.weight", "decoder.layers.0.down.weight", "decoder.norm.weight",
             "decoder.lm_head.weight"]
    base = ref.p
    for name in names:
        gr = grads[name]
        # the element with the largest gradient, and one more
        flat = gr.reshape(-1)
        for idx in (int(flat.abs().argmax()), int(torch.randint(0, flat.numel(), (1,), generator=g))):
            vals = []
            for sgn in (1.0, -1.0):
                p2 = {n: t.double().clone() for n, t in base.items()}
                p2[name].view(-1)[idx] += sgn * 1e-4
                ref.p = p2
                lv, _ = R.gspo_param_grads(ref, *args, dtype=torch.float64)
                vals.append(float(lv))
            ref.p = base
            fd = (vals[0] - vals[1]) / 2e-4
            an = float(flat[idx])
            assert abs(fd - an) <= 1e-5 + 1e-3 * abs(an), (name, idx, fd, an)


def test_strict_identity_oracle_pinned():
    """The reward oracle: its distance is the textbook edit distance; with every base scored the error count
    is that distance (any optimal path); hand cases with a unique optimal path place the errors as ref_errors
    does (scripts/train.py:170-188); the empty-label and empty-call rules (scripts/gspo.py:86-89)."""
    g = np.random.default_rng(3)
    for _ in range(60):
        a = "".join(g.choice(list("ACGT"), g.integers(0, 40)))
        b = "".join(g.choice(list("ACGT"), g.integers(1, 40)))
        rew, dist, errs = R.strict_identity_ref(a, b, np.ones(len(b), bool))
        assert dist == R.edit_distance(a, b) == errs
        assert abs(rew - (1 - dist / max(len(a), len(b)))) < 1e-12
    # substitution at 2, deletion of base 1, insertion after base 1: each a unique optimal path
    for call, ref, pos in (("ACTT", "ACGT", 2), ("AGT", "ACGT", 1), ("ACXGT", "ACGT", 1)):
        for p in range(len(ref)):
            scored = np.ones(len(ref), bool)
            scored[p] = False
            _, _, errs = R.strict_identity_ref(call, ref, scored)
            assert errs == (0 if p == pos else 1), (call, ref, p)
    assert R.strict_identity_ref("XACGT", "ACGT", np.array([False, True, True, True]))[2] == 0  # before base 0
    # an empty call deletes every label base; an empty label scores by length
    assert R.strict_identity_ref("", "ACGT", np.array([1, 0, 1, 1], bool)) == (0.25, 4, 3)
    assert R.strict_identity_ref("ACG", "", np.zeros(0, bool)) == (1.0, 3, 0)
    assert R.strict_identity_ref("ACGTAC", "", np.zeros(0, bool))[0] == 4 / 6
