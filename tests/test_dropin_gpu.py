"""The reference entry points a drop-in user calls directly, each against the oracle on the GPU:

  Decoder.forward (viktor/decoder.py:135-144): causal pass writing the KV cache through batch_slice
      (Attention.forward, viktor/decoder.py:69-79), then decode mode with pos (viktor/decoder.py:93-105);
  FastDecoder.decode (viktor/fast_decoder.py:76-90): one token per sequence, cache rows chosen by seq
      (flash_attn_with_kvcache's cache_batch_idx), from embeddings or from token ids;
  FastDecoder.prefill with the reference signature (viktor/fast_decoder.py:62-74): packed sequences with
      cu_seqlens, the KV cache rows given by seq, and last_indices / cu_queries -- the last layer finishing
      one row per sequence that attends to the whole sequence;
  gspo.engine / gspo.decode (scripts/gspo.py:129-139): engine sizing from the encoder, calls + ended.

The oracle for a cached step is the reference's own invariant (tests/test_viktor.py:33-54): the hidden
state of a decode step equals the last row of a full causal pass over the sequence so far. Hidden states
are compared as the decoder-forward test does (bf16 path against the fused-rounding oracle: max abs < 0.1,
relative L2 < 1e-2).
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import reference as R
from viktor_amd import gspo as G
from viktor_amd.decoder import KVCache
from viktor_amd.synthetic import frames as synth_frames
from viktor_amd.synthetic import make_model

from .test_engine_gpu import DEV, BF, check_stream, gpu_copy

pytestmark = pytest.mark.gpu


def close_hidden(got, want, what):
    """bf16 hidden states against the fused-rounding oracle: max abs < 0.1 and relative L2 < 1e-2 overall, and
    every row's relative L2 < 1.5e-2 (bf16 rounding noise spreads a row by about 0.6% here; a wrong head or a few
    wrong elements of one row show in its own norm, not only in the batch's)."""
    got = got.float().cpu().reshape(want.shape)
    d = (got - want).abs()
    err = float(d.max())
    rel = float((got - want).norm() / want.norm())
    rows = (got - want).reshape(-1, want.shape[-1]).norm(dim=-1) / want.reshape(-1, want.shape[-1]).norm(dim=-1)
    print(f"  {what}: max {err:.2e} rel {rel:.2e} worst row {float(rows.max()):.2e}")
    assert err < 0.1 and rel < 1e-2 and float(rows.max()) < 1.5e-2, (what, err, rel, float(rows.max()))


def test_decoder_forward_cache_prefill_then_decode_mode():
    m = make_model(1, n_layers=2, seed=50, norm_jitter=0.1)
    gm = gpu_copy(m)
    dec = gm.decoder
    ref = R.RefModel(m, "fused")
    B, T0, extra = 4, 150, 3
    x = R.bf(torch.randn(B, T0 + extra, 512, generator=torch.Generator().manual_seed(51)))
    xd = x.to(DEV).to(BF)
    cache = KVCache(dec.cfg, B, 200, BF, DEV)
    # prefill in two halves: each call writes its batch_slice rows of the cache at positions 0..T0-1
    h_lo = dec(xd[:2, :T0], cache=cache, batch_slice=slice(0, 2))
    h_hi = dec(xd[2:, :T0], cache=cache, batch_slice=slice(2, 4))
    full = ref.decoder_forward(x[:, :T0])
    close_hidden(torch.cat([h_lo, h_hi]), full, "prefill")
    assert bool((cache.k[:, :, :T0].abs().sum(-1) > 0).all()) and bool((cache.k[:, :, T0:] == 0).all())
    for j in range(extra):
        pos = torch.full((B,), T0 + j, dtype=torch.long, device=DEV)
        h = dec(xd[:, T0 + j:T0 + j + 1], cache=cache, pos=pos)
        assert h.shape == (B, 1, 512)
        close_hidden(h[:, 0], ref.decoder_forward(x[:, :T0 + j + 1])[:, -1], f"decode step {j}")
    # decode mode writes rows 0..B-1 of the cache: a cache with another row count is refused
    with pytest.raises(AssertionError, match="one cache row per sequence"):
        dec(xd[:2, T0:T0 + 1], cache=cache, pos=torch.full((2,), T0, dtype=torch.long, device=DEV))
    with pytest.raises(AssertionError, match="batch_slice"):
        dec(xd[:2, :T0], cache=cache, batch_slice=slice(3, 5))


@pytest.mark.parametrize("from_tokens", [False, True])
def test_fast_decoder_decode_with_row_map(from_tokens):
    """Three sequences decoded against cache rows 4, 1 and 5 of a 6-row cache, at their own positions."""
    m = make_model(1, n_layers=2, seed=52, norm_jitter=0.1)
    gm = gpu_copy(m)
    dec = gm.decoder
    fast = dec.fast()
    ref = R.RefModel(m, "fused")
    Bc, S = 6, 300
    lens = [120, 37, 200, 64, 150, 90]
    g = torch.Generator().manual_seed(53)
    xs = [R.bf(torch.randn(n, 512, generator=g)) for n in lens]
    cache = KVCache(dec.cfg, Bc, S, BF, DEV)
    for r, xr in enumerate(xs):
        dec(xr[None].to(DEV).to(BF), cache=cache, batch_slice=slice(r, r + 1))
    seq = torch.tensor([4, 1, 5], dtype=torch.int32)
    tok = torch.tensor([3, 6, 4])
    emb = ref.embed(tok)  # the bf16 embedding rows
    pos = torch.tensor([lens[r] for r in seq.tolist()], dtype=torch.int32)
    fast.decode_workspace = None
    if from_tokens:
        h = fast.decode(None, pos.to(DEV), seq.to(DEV), (pos + 1).to(DEV), cache, tok=tok.to(DEV))
    else:
        h = fast.decode(emb.to(DEV).to(BF), pos.to(DEV), seq.to(DEV), (pos + 1).to(DEV), cache)
    for b, r in enumerate(seq.tolist()):
        want = ref.decoder_forward(torch.cat([xs[r], emb[b:b + 1]])[None])[0, -1]
        close_hidden(h[b:b + 1], want[None], f"sequence {b} on row {r}")
    # the new k/v rows went to (seq[b], pos[b]); the other rows' positions are untouched
    for b, r in enumerate(seq.tolist()):
        assert float(cache.k[0, r, lens[r]].abs().sum()) > 0
    for r in (0, 2, 3):
        assert float(cache.k[0, r, lens[r]:].abs().sum()) == 0


def test_gspo_engine_and_decode():
    """scripts/gspo.py:129-139 on a 4-mer model: the engine is sized from the encoder (chunksize // stride
    prefix frames, STEP_BASES // k new tokens), decode samples (T = 1, uniforms drawn by the engine) until
    every call has ended -- a k-mer tail forces EOS -- and returns the decoded calls with their ended flags;
    the tokens match the oracle driven by the engine's uniforms (bar 1)."""
    m = make_model(4, n_layers=2, seed=54, norm_jitter=0.1, bias_jitter=0.1)
    m.encoder = SimpleNamespace(chunksize=12 * 256, stride=12)
    inf = G.bf16_copy(gpu_copy(m))
    eng = G.engine(inf, 4, temperature=1.0)
    torch.manual_seed(56)
    assert eng.max_new == G.STEP_BASES // 4 and eng.max_frames == 256
    P = 256
    plens = torch.tensor([256, 100, 31, 180])
    fr = synth_frames(4, P, 512, seed=55)
    calls, ended = G.decode(eng, fr.to(DEV), plens.to(DEV), inf.tokenizer)
    out = eng.out.cpu()
    assert calls == [inf.tokenizer.decode(t) for t in out]
    assert ended == (out == R.EOS).any(1).tolist()
    steps = int((out != R.PAD).sum(1).max())
    assert steps < eng.max_new  # every call ended, so decoding stopped early
    res = R.RefEngine(R.RefModel(m, "fused"), steps, temperature=1.0).run(
        [fr[b, :int(plens[b])] for b in range(4)], uniforms=eng.uniforms.cpu(), forced=out[:, :steps])
    check_stream(out, res, steps, 5e-3)
    assert all(ended)


def _oracle_prefill(ref, xs, last_noncausal):
    """Final-normed hidden of every row of each packed sequence (fused rounding points), the last layer
    non-causal when asked (so any row's result is that of a query attending to the whole sequence); and the
    per-layer K / V rows."""
    out, kvs = [], []
    L = ref.cfg.n_layers
    for xb in xs:
        kv = ref.new_kv()
        h = ref.first_norm(xb)
        x = xb
        rpos = torch.arange(xb.shape[0])
        for i in range(L):
            x, h = ref.layer(i, x, h, rpos, kv, causal_shift=None if (last_noncausal and i == L - 1) else 0)
        out.append(h)
        kvs.append(kv)
    return out, kvs


@pytest.mark.parametrize("which", ["last_rows", "inner_rows", "all_rows"])
def test_fast_decoder_prefill_reference_signature(which):
    """FastDecoder.prefill(x, pos, seq, cu_seqlens, max_seqlen, cache, last_indices, cu_queries): three packed
    sequences written to permuted cache rows; last_indices at each sequence's last row (the engine's BOS rows),
    at inner rows (whose last-layer query attends to the whole sequence, as the reference's non-causal call), or
    absent (every row). Hidden states and cache rows against the oracle; malformed last_indices / cu_queries
    raise ValueError."""
    m = make_model(1, n_layers=2, seed=60, norm_jitter=0.1)
    gm = gpu_copy(m)
    fast = gm.decoder.fast()
    ref = R.RefModel(m, "fused")
    lens, cache_rows = [37, 130, 64], [2, 0, 1]
    cu = [0, 37, 167, 231]
    g = torch.Generator().manual_seed(61)
    xs = [R.bf(torch.randn(n, 512, generator=g)) for n in lens]
    xd = torch.cat(xs).to(DEV).to(BF)
    pos = torch.cat([torch.arange(n) for n in lens]).to(torch.int32).to(DEV)
    seq = torch.cat([torch.full((n,), r) for n, r in zip(lens, cache_rows)]).to(torch.int32).to(DEV)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=DEV)
    cache = KVCache(gm.decoder.cfg, 3, 160, BF, DEV)
    if which == "all_rows":
        h = fast.prefill(xd, pos, seq, cu_d, max(lens), cache)
        want, kvs = _oracle_prefill(ref, xs, False)
        close_hidden(h, torch.cat(want), which)
    else:
        rows = [c1 - 1 for c1 in cu[1:]] if which == "last_rows" else [5, 37 + 100, 167 + 31]
        last = torch.tensor(rows, dtype=torch.int64, device=DEV)
        cuq = torch.arange(4, dtype=torch.int32, device=DEV)
        h = fast.prefill(xd, pos, seq, cu_d, max(lens), cache, last_indices=last, cu_queries=cuq)
        assert h.shape == (3, 512)
        want, kvs = _oracle_prefill(ref, xs, True)
        close_hidden(h, torch.stack([w[r - c0] for w, r, c0 in zip(want, rows, cu[:-1])]), which)
        with pytest.raises(ValueError, match="one query per sequence"):
            fast.prefill(xd, pos, seq, cu_d, max(lens), cache, last_indices=last,
                         cu_queries=torch.tensor([0, 2, 3, 4], dtype=torch.int32, device=DEV))
        with pytest.raises(ValueError, match="inside each sequence"):
            fast.prefill(xd, pos, seq, cu_d, max(lens), cache, last_indices=torch.tensor([5, 20, 200], device=DEV),
                         cu_queries=cuq)
    # every layer's K / V rows of each sequence at its cache row
    for i in range(gm.decoder.cfg.n_layers):
        for b, (n, r) in enumerate(zip(lens, cache_rows)):
            kw, vw = kvs[b][i]
            close_hidden(cache.k[i, r, :n].reshape(n, -1), kw.reshape(n, -1), f"k layer {i} seq {b}")
            close_hidden(cache.v[i, r, :n].reshape(n, -1), vw.reshape(n, -1), f"v layer {i} seq {b}")
