"""Parity of the benchmarked rollout itself against the oracle, at its own shape: 64 windows x group 8 =
512 sequences, 2048-frame prefixes, 8 layers, vocab 7, sampled at T = 1 from supplied uniforms for 1024
tokens, one prefill per window with the prefix KV shared by the group (DecodeEngine(group_size=8)), the
launch layout the benchmark runs. EOS is banned on both sides and the homopolymer cap is off, so every
compared position is a live choice (the grammar's own paths are covered in test_engine_gpu.py).

The oracle teacher-forces the engine's tokens (scripts/gspo.py:444 repeats each window for its group;
viktor/engine.py:79-116 is the state machine), so every position is compared even after an exempt one:
  bar 1: tokens equal unless the uniform lies within 5e-3 of a CDF boundary of the oracle's distribution;
  bar 2: the engine's per-token log-probabilities against the oracle's at the engine's token: no wider than
         the spread of two oracles that differ in one bf16 rounding point, and >= 95% within 2e-2 (sampled
         steps choose from bf16 logits; check_logprobs states the rule), the per-sequence ratio within 5e-3;
  bar 3: integer outputs are the token ids themselves, compared exactly.

The cfg1 test runs the CPU-plumbing configuration (4 sequences, 2048-frame prefixes, 64 greedy steps,
weights and frames from seed 0) on the GPU against the same oracle (tests/test_viktor.py:71-83 is the
reference's own invariant for that engine).
"""

import pytest
import torch

from oracle import reference as R
from viktor_amd import DecodeEngine
from viktor_amd.synthetic import frames as synth_frames
from viktor_amd.synthetic import make_model, uniforms as synth_uniforms

from .test_engine_gpu import DEV, check_logprobs, check_stream, gpu_copy, no_eos_bias

pytestmark = pytest.mark.gpu

WINDOWS, GROUP, P, NEW = 64, 8, 2048, 1024


@pytest.fixture(scope="module")
def rollout():
    """One full rollout at the benchmark's shape; returns the model, frames, uniforms, tokens, logprobs."""
    m = make_model(1, n_layers=8, seed=21, norm_jitter=0.1, bias_jitter=0.1)
    fr = synth_frames(WINDOWS, P, 512, seed=22)
    u = synth_uniforms(WINDOWS * GROUP, NEW, seed=23)
    gm = gpu_copy(m)
    eng = DecodeEngine(gm, WINDOWS * GROUP, NEW, P, temperature=1.0, max_homopolymer=None, group_size=GROUP,
                       logprobs=True)
    assert eng.prefix_cache is not None
    bias = no_eos_bias(m.tokenizer.vocab_size)
    eng.bias.copy_(bias)
    eng.set_uniforms(u.to(DEV))
    frd = fr.to(DEV).repeat_interleave(GROUP, 0).reshape(-1, 512)
    out = eng.generate(frd, [P] * (WINDOWS * GROUP)).clone().cpu()
    logp = eng.logp.clone().cpu()
    del eng, frd
    torch.cuda.empty_cache()
    return dict(m=m, fr=fr, u=u, out=out, logp=logp, bias=bias)


def _oracle(rollout, members, steps, p_bf16=False):
    m, fr, bias = rollout["m"], rollout["fr"], rollout["bias"]
    windows = {b // GROUP: fr[b // GROUP] for b in members}  # one tensor per window: one oracle prefill each
    ref = R.RefEngine(R.RefModel(m, "fused", p_bf16=p_bf16), NEW, temperature=1.0, max_homopolymer=None, bias=bias)
    return ref.run([windows[b // GROUP] for b in members], steps=steps, uniforms=rollout["u"][members],
                   forced=rollout["out"][members])


def test_rollout_first_64_steps_two_groups(rollout):
    """Every member of the first and the last window's group, 64 steps."""
    members = list(range(GROUP)) + list(range((WINDOWS - 1) * GROUP, WINDOWS * GROUP))
    res = _oracle(rollout, members, 64)
    out = rollout["out"][members]
    agree, _ = check_stream(out, res, 64, 5e-3, min_live=1.0)
    assert agree > 0.97, agree
    pair = _oracle(rollout, members, 64, p_bf16=True)
    err, within = check_logprobs(rollout["logp"][members], res, out, rollout["bias"], 1.0, pair_res=pair)
    print(f"64 steps x {len(members)} members: agreement {agree:.4f}, max |logp diff| {err:.2e}, "
          f"{within:.4f} within 2e-2")
    # members of a group share the prefix but not the uniforms: their streams differ
    assert not torch.equal(out[0], out[1])


def test_rollout_all_1024_steps_two_members(rollout):
    """Two members of one group over the whole rollout: own-cache rows up to 1023, attention spans up to
    3072 positions (2049 prefix rows + the member's own tokens). The last 32 positions are reported apart."""
    members = [8, 13]
    res = _oracle(rollout, members, NEW)
    out = rollout["out"][members]
    agree, _ = check_stream(out, res, NEW, 5e-3, min_live=1.0)
    tail = {"choice": res["choice"][:, -32:], "margin": res["margin"][:, -32:]}
    agree_tail, _ = check_stream(out[:, -32:], tail, 32, 5e-3, min_live=1.0)
    pair = _oracle(rollout, members, NEW, p_bf16=True)
    err, within = check_logprobs(rollout["logp"][members], res, out, rollout["bias"], 1.0, pair_res=pair)
    print(f"1024 steps x 2 members: agreement {agree:.4f} (last 32: {agree_tail:.4f}), max |logp diff| {err:.2e}, "
          f"{within:.4f} within 2e-2")
    assert agree > 0.97


def test_rollout_invariants_all_members(rollout):
    """All 512 x 1024 tokens: in the allowed range (EOS banned: bases only), reproducible from the uniforms,
    and every logprob finite and <= 0."""
    out, logp = rollout["out"], rollout["logp"]
    assert bool(((out >= 3) & (out <= 6)).all())
    assert bool(torch.isfinite(logp).all()) and bool((logp <= 1e-6).all())


def test_cfg1_greedy_full_size():
    """The CPU-plumbing configuration on the GPU: 4 sequences x 2048-frame prefixes, 8 layers, 64 greedy
    steps, weights and frames from seed 0, EOS banned (the reference's default grammar otherwise)."""
    m = make_model(1, n_layers=8, seed=0)
    B, steps = 4, 64
    fr = synth_frames(B, P, 512, seed=0)
    gm = gpu_copy(m)
    eng = DecodeEngine(gm, B, steps, P, temperature=0.0, max_homopolymer=None, logprobs=True)
    bias = no_eos_bias(m.tokenizer.vocab_size)
    eng.bias.copy_(bias)
    out = eng.generate(fr.to(DEV).reshape(-1, 512), [P] * B, steps=steps).clone().cpu()
    logp = eng.logp.clone().cpu()
    ref = R.RefEngine(R.RefModel(m, "fused"), steps, temperature=0.0, max_homopolymer=None, bias=bias)
    res = ref.run(list(fr), forced=out)
    agree, _ = check_stream(out, res, steps, 1e-2, min_live=1.0)
    # greedy: the prefill token comes from bf16 logits, later ones from fp32 logits (viktor/engine.py:96, 191)
    err, within = check_logprobs(logp, res, out, bias, 0.0)
    print(f"cfg1: agreement {agree:.4f}, max |logp diff| {err:.2e}, {within:.4f} within 2e-2")
    assert agree > 0.95
