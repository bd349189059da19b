"""Scoring over groups that share their prefix (token_logprobs / Basecaller.logits with group_size): each group's
prefix runs once and its members' token rows attend to its keys. The reference scores every repeated window in
full (scripts/gspo.py:340-353 over the rollout of scripts/gspo.py:444), so the shared forward is checked against
the unshared one on the same inputs: the token rows' hidden states and logits bit for bit (every product of both
forwards on the same kernels: at least 4096 rows), with unequal prefix lengths across groups and with the
scaled prefix positions, and the log-probs at the rollout's scoring shape. The unshared forward itself is held
to the oracle by tests/test_engine_gpu.py."""

import copy

import pytest
import torch

from viktor_amd import gspo
from viktor_amd.synthetic import make_model, scoring_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def master(n_layers, seed, pos_scale=1):
    m = make_model(1, n_layers=n_layers, seed=seed, norm_jitter=0.1, bias_jitter=0.1)
    m.pos_scale = pos_scale
    g = copy.deepcopy(m).to(DEV)
    g.decoder._fast = None
    return g.eval()


def grouped_frames(n_groups, G, P, seed):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    base = torch.randn(n_groups, P, 512, generator=gen, device=DEV)
    return base.repeat_interleave(G, 0).contiguous()


@pytest.mark.parametrize("pre_lens,pos_scale", [(None, 1), ([1280, 1100, 1000, 1217], 1), (None, 2)])
def test_shared_prefix_hidden_equals_unshared(pre_lens, pos_scale):
    n_groups, G, P, T = 4, 4, 1280, 384
    gm = master(4, 21, pos_scale)
    fr = grouped_frames(n_groups, G, P, 22)
    B = n_groups * G
    plens = None if pre_lens is None else torch.tensor(pre_lens, device=DEV).repeat_interleave(G)
    gen = torch.Generator().manual_seed(23)
    tin = torch.randint(0, gm.tokenizer.vocab_size, (B, T), generator=gen).to(DEV)
    with torch.no_grad():
        h1 = gm.hidden(fr, tin, plens)
        hg = gm.hidden(fr, tin, plens, group_size=G)
        z1 = gm.logits(fr, tin, plens)
        zg = gm.logits(fr, tin, plens, group_size=G)
    assert hg.shape == h1.shape == (B * T, 512)
    assert torch.equal(hg, h1), float((hg.float() - h1.float()).abs().max())
    assert torch.equal(zg, z1)


def test_shared_prefix_logprobs_at_scoring_shape():
    """64 windows x 8 samples (the rollout's groups), 2048-frame prefixes, 700..1024-token calls (T = 1024 after
    padding to 128): the log-probs and masks of token_logprobs equal the unshared call's."""
    n_groups, G, P = 64, 8, 2048
    gm = master(8, 24)
    fr = grouped_frames(n_groups, G, P, 25)
    B = n_groups * G
    seqs, ended = scoring_inputs(B, 700, 1024, k=1, seed=26)
    plens = torch.full((B,), P, device=DEV)
    with torch.no_grad():
        lp1, m1 = gspo.token_logprobs(gm, fr, plens, seqs, ended)
        lpg, mg = gspo.token_logprobs(gm, fr, plens, seqs, ended, group_size=G)
    assert torch.equal(mg, m1)
    assert torch.equal(lpg, lp1), float((lpg - lp1).abs().max())


def test_shared_prefix_rejects_groups_that_differ():
    gm = master(2, 27)
    G, P, T = 4, 256, 128
    fr = grouped_frames(2, G, P, 28)
    tin = torch.zeros(2 * G, T, dtype=torch.long, device=DEV)
    fr_bad = fr.clone()
    fr_bad[5, 100, 7] += 1.0  # one value of one member of the second group
    with torch.no_grad():
        with pytest.raises(ValueError, match="share their prefix frames"):
            gm.hidden(fr_bad, tin, None, group_size=G)
        plens = torch.full((2 * G,), P, device=DEV)
        plens[6] = P - 1
        with pytest.raises(ValueError, match="same prefix length"):
            gm.hidden(fr, tin, plens, group_size=G)
        with pytest.raises(ValueError, match="whole groups"):
            gm.hidden(fr[:7], tin[:7], None, group_size=G)
        # shorter prefixes compare only their real frames: a difference past them is padding
        fr_pad = fr.clone()
        fr_pad[5, P - 1] += 1.0
        plens = torch.full((2 * G,), P - 1, device=DEV)
        assert torch.equal(gm.hidden(fr_pad, tin, plens, group_size=G), gm.hidden(fr, tin, plens, group_size=G))
