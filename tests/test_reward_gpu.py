"""The GSPO reward on the device (vk_strict_identity) against the oracle's restatement of strict_identity
(pinned in test_oracle.py): exact integer distances and error counts, rewards to fp32 rounding. The masked
error count follows the stated path preference; edlib's own traceback is not available (parity unpinned
where masked bases and tied optimal paths meet)."""

import numpy as np
import pytest
import torch

from oracle import reference as R
from viktor_amd import reward as RW
from viktor_amd.tokenizer import KmerTokenizer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _mutate(rng, s, rate):
    out = []
    for ch in s:
        u = rng.random()
        if u < rate / 3:
            continue  # deletion
        if u < 2 * rate / 3:
            out.append(rng.choice(list("ACGT")))  # substitution (maybe the same base)
        else:
            out.append(ch)
        if rng.random() < rate / 3:
            out.append(rng.choice(list("ACGT")))  # insertion
    return "".join(out)


def _check(calls, labels, scored, roc):
    res = RW.strict_identity(calls, labels, scored, roc, device=DEV)
    rew, dist, errs = (res[k].cpu().numpy() for k in ("reward", "edit_distance", "scored_errors"))
    for c, (call, r) in enumerate(zip(calls, roc)):
        w_rew, w_dist, w_err = R.strict_identity_ref(call, labels[r], scored[r])
        assert (dist[c], errs[c]) == (w_dist, w_err), (c, len(call), len(labels[r]))
        assert abs(float(rew[c]) - w_rew) <= 1e-6, (c, float(rew[c]), w_rew)


def test_strict_identity_random_pairs():
    rng = np.random.default_rng(1)
    labels = ["".join(rng.choice(list("ACGT"), rng.integers(1, 200))) for _ in range(12)] + ["", "A"]
    scored = [rng.random(len(l)) > 0.2 for l in labels]
    calls, roc = [], []
    for r, lab in enumerate(labels):
        for _ in range(3):
            calls.append(_mutate(rng, lab, 0.15) if rng.random() < 0.8 else "".join(rng.choice(list("ACGT"), rng.integers(0, 60))))
            roc.append(r)
    calls += ["", "ACGTACGT"]
    roc += [0, 12]
    _check(calls, labels, scored, roc)


def test_strict_identity_rollout_sizes_and_limits():
    """Label-sized pairs (0.8-1.5 kb, 5% errors), fully scored and masked, and a 4096-base label (more than
    64 KB of LDS for the diagonals)."""
    rng = np.random.default_rng(2)
    labels = ["".join(rng.choice(list("ACGT"), n)) for n in (800, 1500, 4096)]
    scored = [np.ones(800, bool), rng.random(1500) > 0.1, rng.random(4096) > 0.05]
    calls = [_mutate(rng, labels[0], 0.05), _mutate(rng, labels[1], 0.05), _mutate(rng, labels[2], 0.02),
             labels[0], ""]
    _check(calls, labels, scored, [0, 1, 2, 0, 1])


def test_calls_from_tokens_match_host_decode():
    rng = np.random.default_rng(3)
    for k in (1, 4):
        tok = KmerTokenizer(k)
        V = tok.vocab_size
        rows = torch.tensor(rng.integers(3, V, (9, 40)), dtype=torch.long)
        rows[1, 5] = 2          # EOS: the call stops
        rows[2, 0] = 2          # empty call
        rows[3, 7:] = 0         # PAD after the call
        rows[4, 3] = 1          # BOS inside is skipped
        data, off, lens, mx = RW.calls_from_tokens(rows.to(DEV), tok)
        data, off, lens = data.cpu().numpy(), off.cpu().numpy(), lens.cpu().numpy()
        for b in range(rows.shape[0]):
            want = tok.decode(rows[b].tolist())
            got = bytes(data[off[b]:off[b] + lens[b]]).decode()
            assert got == want, (k, b)
        assert mx == max(len(tok.decode(r.tolist())) for r in rows)


def test_rewards_from_tokens_equal_rewards_from_strings():
    rng = np.random.default_rng(4)
    tok = KmerTokenizer(1)
    G = 4
    labels = ["".join(rng.choice(list("ACGT"), n)) for n in (50, 80, 0)]
    weights = [rng.random(len(l)) for l in labels]
    rows = torch.tensor(rng.integers(3, 7, (3 * G, 90)), dtype=torch.long)
    rows[0, 60] = 2
    rows[5, 2] = 2
    dev_res = RW.gspo_rewards_from_tokens(rows.to(DEV), tok, labels, weights, G)
    calls = [tok.decode(r.tolist()) for r in rows]
    host = RW.gspo_rewards(calls, labels, weights, G, device=DEV)
    assert np.array_equal(dev_res["reward"].double().cpu().numpy().reshape(-1, G), host)
    for i, c in enumerate(calls):
        assert abs(host.reshape(-1)[i] - R.strict_identity_ref(c, labels[i // G], weights[i // G] > 0)[0]) < 1e-6
