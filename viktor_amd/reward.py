"""The GSPO reward on the device: strict identity of every call against its window's label.

Reference: scripts/gspo.py:86-89 (strict_identity), 446 (the reward of a rollout), scripts/train.py:170-188
(ref_errors, the edlib NW path's error positions), scripts/evaluate.py:30 (EMPTY_MAX). The reference runs
edlib on the host, one call after another; here one kernel scores every call of a rollout at once
(vk_strict_identity: one wavefront per call, anti-diagonal edit-distance DP in LDS).

The alignment path behind the error positions: at every cell the first optimal predecessor in the order
diagonal, deletion, insertion. edlib's own traceback order is not available here; the edit distance, and
the reward whenever every label base is scored, do not depend on the path.
"""

from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import call, ptr, require_device
from .tokenizer import EOS, N_SPECIAL

EMPTY_MAX = 4  # scripts/evaluate.py:30: a window without DNA scores 1 for a call of at most this many bases


def _pack(strings: Sequence[bytes], device):
    lens = [len(s) for s in strings]
    off = np.zeros(len(strings), dtype=np.int64)
    if len(strings) > 1:
        off[1:] = np.cumsum(lens[:-1])
    data = np.frombuffer(b"".join(strings), dtype=np.uint8) if sum(lens) else np.zeros(1, np.uint8)
    return (torch.from_numpy(data.copy()).to(device), torch.from_numpy(off).to(device),
            torch.tensor(lens, dtype=torch.int32).to(device), max(lens) if lens else 0)


def _run(call_data, call_off, call_len, max_call, refs: Sequence[str], scored: Sequence[np.ndarray], ref_of_call,
         device, empty_max):
    ref_b = [r.encode() for r in refs]
    ref_data, ref_off, ref_len, max_ref = _pack(ref_b, device)
    sc = [np.asarray(s, dtype=bool).astype(np.uint8) for s in scored]
    assert all(len(s) == len(r) for s, r in zip(sc, ref_b)), "strict_identity: a scored mask per label base"
    sc_data = torch.from_numpy(np.concatenate(sc) if sum(len(s) for s in sc) else np.zeros(1, np.uint8)).to(device)
    n = call_len.shape[0]
    roc = torch.as_tensor(ref_of_call, dtype=torch.int32).to(device)
    reward = torch.empty(n, dtype=torch.float32, device=device)
    dist = torch.empty(n, dtype=torch.int32, device=device)
    errs = torch.empty(n, dtype=torch.int32, device=device)
    call("vk_strict_identity", ptr(call_data), ptr(call_off), ptr(call_len), ptr(ref_data), ptr(ref_off),
         ptr(ref_len), ptr(sc_data), ptr(roc), n, len(refs), max_ref, max_call, float(empty_max), ptr(reward),
         ptr(dist), ptr(errs), _lib.stream_handle())
    return {"reward": reward, "edit_distance": dist, "scored_errors": errs}


def strict_identity(calls: Sequence[str], labels: Sequence[str], scored: Sequence[np.ndarray],
                    ref_of_call: Optional[Sequence[int]] = None, device="cuda", empty_max=EMPTY_MAX):
    """Strict identity of calls[c] against labels[ref_of_call[c]] (default: labels[c]) with scored[r] the bool
    mask of label r's counted bases; returns device tensors {reward fp32, edit_distance, scored_errors} [len(calls)].
    Reference: scripts/gspo.py:86-89."""
    require_device(torch.empty(0, device=device), "strict_identity")
    ref_of_call = list(range(len(calls))) if ref_of_call is None else list(ref_of_call)
    data, off, lens, max_call = _pack([c.encode() for c in calls], device)
    return _run(data, off, lens, max_call, labels, scored, ref_of_call, device, empty_max)


def gspo_rewards(calls: List[str], labels: List[str], weights: List[np.ndarray], G: int, device="cuda"):
    """The rollout's reward [windows, G] (scripts/gspo.py:446): call i against label i // G, scored where the
    label's weight is positive. float64 host array, as the reference's."""
    res = strict_identity(calls, labels, [np.asarray(w) > 0 for w in weights], [i // G for i in range(len(calls))],
                          device)
    return res["reward"].double().cpu().numpy().reshape(-1, G)


def calls_from_tokens(tokens: torch.Tensor, tokenizer):
    """Device base strings of the engine's output tokens [N, T] (int64): the tokenizer's decode on the device
    (stops at the first EOS, skips PAD and BOS; a token writes its k-mer or tail). Returns (bytes [total] uint8,
    offsets [N] int64, lengths [N] int32, max length)."""
    dev = tokens.device
    V, k = tokenizer.vocab_size, tokenizer.k
    table = torch.zeros(V, k, dtype=torch.uint8)
    tlen = torch.zeros(V, dtype=torch.int64)
    for t in range(N_SPECIAL, V):
        s = tokenizer.strings[t].encode()
        table[t, :len(s)] = torch.tensor(list(s), dtype=torch.uint8)
        tlen[t] = len(s)
    table, tlen = table.to(dev), tlen.to(dev)
    tok = tokens.clamp(0, V - 1)
    before_eos = torch.cumsum((tok == EOS).to(torch.int32), 1) == 0
    n_bases = tlen[tok] * before_eos                      # [N, T] bases each token writes
    lengths = n_bases.sum(1)
    offsets = torch.cumsum(lengths, 0) - lengths
    pos = offsets[:, None] + torch.cumsum(n_bases, 1) - n_bases  # first byte of each token
    total = int(lengths.sum())
    out = torch.zeros(max(total, 1), dtype=torch.uint8, device=dev)
    for i in range(k):  # byte i of every token that has one
        keep = n_bases > i
        out[(pos + i)[keep]] = table[tok, i][keep]
    return out, offsets, lengths.to(torch.int32), int(lengths.max()) if lengths.numel() else 0


def gspo_rewards_from_tokens(tokens: torch.Tensor, tokenizer, labels: List[str], weights: List[np.ndarray], G: int,
                             empty_max=EMPTY_MAX):
    """The rollout's rewards straight from the engine's device output (no host decode): tokens [windows * G, T];
    returns the device dict of strict_identity (reward [windows * G] fp32)."""
    data, off, lens, max_call = calls_from_tokens(tokens, tokenizer)
    return _run(data, off, lens, max_call, labels, [np.asarray(w) > 0 for w in weights],
                [i // G for i in range(tokens.shape[0])], tokens.device, empty_max)
