"""Output vocabularies of the decoder: single bases (k=1, 7 tokens) and fixed k-mers (k=4, 343 tokens).

Behaviour follows viktor/tokenizer.py:1-57 of the reference:
  ids 0, 1, 2 are PAD, BOS, EOS;
  then every full k-mer over ACGT in lexicographic (itertools.product) order;
  then the short "tail" k-mers of length 1..k-1, shortest first, each length in product order.
A tail token may only be the last token before EOS (the decode grammar enforces it).
"""

from itertools import product

import torch

PAD, BOS, EOS = 0, 1, 2
N_SPECIAL = 3
BASES = "ACGT"


class KmerTokenizer:
    """Vocabulary of one k (reference: viktor/tokenizer.py:11-53)."""

    def __init__(self, k: int):
        if k < 1:
            raise ValueError(f"k must be >= 1, got {k}")
        self.k = k
        full = ["".join(t) for t in product(BASES, repeat=k)]
        tails = [s for n in range(1, k) for s in ("".join(t) for t in product(BASES, repeat=n))]
        self.strings = ["<pad>", "<bos>", "<eos>", *full, *tails]
        self.vocab_size = len(self.strings)
        self.n_full = len(full)
        self.ids = {s: i for i, s in enumerate(self.strings) if i >= N_SPECIAL}
        first_tail = N_SPECIAL + self.n_full
        self.tail_mask = torch.arange(self.vocab_size) >= first_tail
        self.n_bases = torch.tensor([0] * N_SPECIAL + [len(s) for s in self.strings[N_SPECIAL:]])

    def encode(self, seq: str) -> list:
        """Bases -> token ids: consecutive k-base pieces, the last one shorter when len(seq) % k != 0."""
        return [self.ids[seq[i:i + self.k]] for i in range(0, len(seq), self.k)]

    def decode(self, ids) -> str:
        """Token ids -> bases: stops at the first EOS, skips PAD and BOS."""
        parts = []
        for t in ids:
            t = int(t)
            if t == EOS:
                break
            if t >= N_SPECIAL:
                parts.append(self.strings[t])
        return "".join(parts)

    def batch(self, seqs):
        """Teacher-forcing tensors for a list of base strings.

        Returns (tokens_in [B, T], targets [B, T], total bases) with T = longest token count + 1:
        tokens_in row b = [BOS, t1..tn, PAD...], targets row b = [t1..tn, EOS, PAD...]."""
        enc = [self.encode(s) for s in seqs]
        T = max(len(t) for t in enc) + 1
        tokens_in = torch.full((len(seqs), T), PAD, dtype=torch.long)
        targets = torch.full((len(seqs), T), PAD, dtype=torch.long)
        for b, t in enumerate(enc):
            n = len(t)
            tokens_in[b, 0] = BOS
            if n:
                tokens_in[b, 1:n + 1] = torch.tensor(t)
                targets[b, :n] = torch.tensor(t)
            targets[b, n] = EOS
        return tokens_in, targets, sum(len(s) for s in seqs)


def get_tokenizer(name: str) -> KmerTokenizer:
    """'base' -> k=1, '4mer' -> k=4 (reference: viktor/tokenizer.py:56-57)."""
    table = {"base": 1, "4mer": 4}
    if name not in table:
        raise KeyError(name)
    return KmerTokenizer(table[name])
