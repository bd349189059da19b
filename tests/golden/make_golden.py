"""Write the golden vectors of the reference's CPU path into tests/golden/*.npz / *.json.

Run in the build container only (it imports the reference package from /root/reference, which does not
exist where the tests run):  python tests/golden/make_golden.py

What is recorded (all fp32 CPU, reference code paths only):
  rope.npz       rope_tables rows at theta 1e4 and 1e6              (viktor/encoder.py:30-33)
  tokenizer.json vocab strings, tail mask, n_bases, encode/decode/batch examples  (viktor/tokenizer.py)
  decoder.npz    Decoder.forward hidden states + head logits, tiny and full-width configs, with and
                 without explicit RoPE positions                     (viktor/decoder.py:135-164)
  engine.npz     DecodeEngine(backend="torch") greedy token streams, k = 1 and k = 4, variable prefix
                 lengths, settings chosen so tail->EOS, homopolymer->EOS and PAD-after-EOS all occur,
                 one case with pos_scale 2                           (viktor/engine.py)
  logits.npz     Basecaller.batch + Basecaller.logits teacher-forced logits with per-window plens
                                                                     (viktor/model.py:55-85, 119-131)
Weights come from viktor_amd.synthetic.init_params (seeded, sorted parameter order), applied to the
reference modules; the tests rebuild the same weights and check a checksum recorded here.
Inputs are seeded torch.randn draws, stored in the fixtures.
"""

import json
import os
import sys

sys.dont_write_bytecode = True
HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, REPO)
sys.path.insert(0, REF)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from viktor import Basecaller, DecodeEngine, DecoderConfig, KmerTokenizer  # noqa: E402  (the reference)
from viktor.decoder import Decoder  # noqa: E402
from viktor.encoder import rope_tables  # noqa: E402
from viktor_amd.synthetic import init_params  # noqa: E402

PAD, BOS, EOS = 0, 1, 2

TINY = dict(d_model=32, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=8, ffn_dim=64, max_seq_len=512)
FULL2 = dict(d_model=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=1536, max_seq_len=4096,
             rope_theta=1e6)


class FrameSource:
    """Stand-in for the encoder: the reference Basecaller only reads encoder.d_model (and it must not add
    parameters, so the seeded init order matches the encoder-less models of the tests)."""

    def __init__(self, d_model):
        self.d_model = d_model


def checksum(module):
    """(sum, sum of squares) over all parameters in float64: detects a drift of the seeded init."""
    s = sq = 0.0
    for _, p in sorted(module.named_parameters()):
        d = p.detach().double()
        s += float(d.sum())
        sq += float((d * d).sum())
    return [s, sq]


def make_model(k, cfg_kw, seed, d_enc, norm_jitter, pos_scale=1):
    tok = KmerTokenizer(k)
    cfg = DecoderConfig(vocab_size=tok.vocab_size, **cfg_kw)
    m = Basecaller(FrameSource(d_enc), tok, cfg)
    init_params(m, seed, norm_jitter=norm_jitter, bias_jitter=0.1)
    m.pos_scale = pos_scale
    return m.eval()


def rope():
    rows = np.array([0, 1, 2, 3, 100, 1000, 2048, 3072, 4095])
    out = {"rows": rows}
    for theta in (1e4, 1e6):
        c, s = rope_tables(64, 4096, theta)
        out[f"cos_{int(theta)}"] = c[rows].numpy()
        out[f"sin_{int(theta)}"] = s[rows].numpy()
    np.savez(os.path.join(HERE, "rope.npz"), **out)


def tokenizer():
    out = {}
    for k in (1, 4):
        tk = KmerTokenizer(k)
        rng = np.random.default_rng(k)
        seqs = ["".join(rng.choice(list("ACGT"), n)) for n in (0, 1, 3, 4, 5, 9, 17)]
        ids = [tk.encode(s) for s in seqs]
        tin, tgt, nb = tk.batch([s for s in seqs if s] or ["A"])
        out[str(k)] = {
            "strings": tk.strings, "tail_mask": tk.tail_mask.int().tolist(), "n_bases": tk.n_bases.tolist(),
            "seqs": seqs, "ids": ids,
            "decode_cases": [[ids[-1] + [EOS, 5], tk.decode(ids[-1] + [EOS, 5])], [[PAD, BOS] + ids[3], tk.decode([PAD, BOS] + ids[3])]],
            "batch_in": tin.tolist(), "batch_tgt": tgt.tolist(), "batch_bases": nb,
        }
    with open(os.path.join(HERE, "tokenizer.json"), "w") as f:
        json.dump(out, f)


@torch.no_grad()
def decoder():
    out = {}
    for name, kw, seed, B, T in (("tiny", TINY, 11, 2, 12), ("full2", FULL2, 12, 2, 40)):
        tok = KmerTokenizer(1)
        cfg = DecoderConfig(vocab_size=tok.vocab_size, **kw)
        dec = Decoder(cfg).eval()
        init_params(dec, seed, norm_jitter=0.1)
        g = torch.Generator().manual_seed(seed + 100)
        x = torch.randn(B, T, cfg.d_model, generator=g)
        pos = torch.randint(0, cfg.max_seq_len - 1, (B, T), generator=g)
        h = dec(x)
        h_pos = dec(x, positions=pos)
        out.update({f"{name}_x": x.numpy(), f"{name}_pos": pos.numpy(), f"{name}_h": h.numpy(),
                    f"{name}_h_pos": h_pos.numpy(), f"{name}_logits": dec.head(h).numpy(),
                    f"{name}_seed": np.array(seed), f"{name}_checksum": np.array(checksum(dec))})
    np.savez(os.path.join(HERE, "decoder.npz"), **out)


def rules_fired(out, k, tail, homo_stop, is_homo):
    """Which grammar rules show in the output streams: tail->EOS, homopolymer->EOS, PAD after EOS."""
    fired = {"tail": False, "homo": False, "pad": False}
    for row in out.tolist():
        for j, t in enumerate(row):
            if t == EOS:
                if j > 0 and tail[row[j - 1]]:
                    fired["tail"] = True
                if homo_stop and j >= homo_stop - 1:
                    prev = row[j - homo_stop + 1:j]
                    if len(set(prev)) == 1 and is_homo[prev[0]]:
                        fired["homo"] = True
                if j + 1 < len(row) and row[j + 1] == PAD:
                    fired["pad"] = True
    return fired


@torch.no_grad()
def engine():
    out = {}
    cases = [
        # name, k, cfg, lens, steps, max_homopolymer, pos_scale, wanted rules
        ("tiny_k1", 1, TINY, [5, 17, 9, 23], 24, 4, 1, ("homo", "pad")),
        ("tiny_k4", 4, TINY, [7, 12, 30], 20, 8, 1, ("tail", "pad")),
        ("full2_k1", 1, FULL2, [20, 33, 8], 16, 4, 1, ("homo",)),
        ("full2_k4", 4, FULL2, [11, 26], 14, 8, 1, ("tail",)),
        ("tiny_k1_ps2", 1, TINY, [6, 15], 12, 64, 2, ()),
    ]
    d_enc = 24
    for name, k, kw, lens, steps, mh, ps, want in cases:
        for seed in range(100, 400):
            m = make_model(k, kw, seed, d_enc, norm_jitter=0.1, pos_scale=ps)
            g = torch.Generator().manual_seed(seed + 1)
            frames = torch.randn(sum(lens), d_enc, generator=g)
            eng = DecodeEngine(m, len(lens), steps, max(lens), backend="torch", cuda_graph=False, prefill_batch=2,
                               max_homopolymer=mh)
            toks = eng.generate(frames, lens).clone()
            fired = rules_fired(toks, k, m.tokenizer.tail_mask.tolist(), eng.homo_stop, eng.is_homo.tolist())
            if all(fired[r] for r in want):
                break
        else:
            raise RuntimeError(f"no seed fires {want} for {name}")
        print(name, "seed", seed, fired)
        out.update({f"{name}_frames": frames.numpy(), f"{name}_lens": np.array(lens), f"{name}_tokens": toks.numpy(),
                    f"{name}_meta": np.array([k, seed, steps, mh, ps, d_enc]),
                    f"{name}_checksum": np.array(checksum(m))})
    np.savez(os.path.join(HERE, "engine.npz"), **out)


@torch.no_grad()
def logits():
    out = {}
    d_enc = 24
    for name, k, kw, seed, ps in (("tiny_k4", 4, TINY, 21, 1), ("full2_k1", 1, FULL2, 22, 1), ("tiny_k1_ps4", 1, TINY, 23, 4)):
        m = make_model(k, kw, seed, d_enc, norm_jitter=0.1, pos_scale=ps)
        rng = np.random.default_rng(seed)
        seqs = ["".join(rng.choice(list("ACGT"), n)) for n in (9, 3, 14)]
        tin, tgt, w = m.batch(seqs, pad_to=8)
        g = torch.Generator().manual_seed(seed + 1)
        P = 19
        frames = torch.randn(len(seqs), P, d_enc, generator=g)
        plens = torch.tensor([19, 11, 16])
        lg = m.logits(frames, tin, plens)
        out.update({f"{name}_frames": frames.numpy(), f"{name}_plens": plens.numpy(), f"{name}_tokens_in": tin.numpy(),
                    f"{name}_targets": tgt.numpy(), f"{name}_w": w.numpy(), f"{name}_logits": lg.numpy(),
                    f"{name}_seqs": np.array(seqs), f"{name}_meta": np.array([k, seed, ps, d_enc]),
                    f"{name}_checksum": np.array(checksum(m))})
    np.savez(os.path.join(HERE, "logits.npz"), **out)


if __name__ == "__main__":
    torch.set_num_threads(8)
    rope()
    tokenizer()
    decoder()
    engine()
    logits()
    print("golden vectors written to", HERE)
