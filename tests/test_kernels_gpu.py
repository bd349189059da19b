"""Per-kernel parity on the GPU: every HIP op (through the C ABI) against the CPU oracle's op on the same
seeded inputs. Bars: bit-exact for integer outputs and for values that the reference defines by a
single rounding of an exact quantity (residual sums, copies, cache rows); otherwise within the stated
tolerances (bf16 outputs: 1-2 ulp of bf16; attention: 1e-2 absolute as the reference's own check)."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R
from viktor_amd import hip_ops as ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
DEV = "cuda"


def gen(seed):
    return torch.Generator().manual_seed(seed)


def to_dev(t, dtype=None):
    return t.to(dtype).to(DEV) if dtype else t.to(DEV)


def bf_close(a, b, ulps=1.0, atol=1e-6):
    """|a - b| <= ulps bf16 ulps of b (an ulp = 2^(exponent(b) - 7)) + atol."""
    a, b = a.float().cpu(), b.float().cpu()
    ulp = torch.pow(2.0, torch.floor(torch.log2(b.abs().clamp(min=1e-30))) - 7)
    tol = ulps * ulp + atol
    bad = (a - b).abs() > tol
    return not bool(bad.any()), float((a - b).abs().max())


@pytest.mark.parametrize("n,d", [(1, 512), (37, 512), (1000, 512), (5, 1536), (3, 64)])
def test_add_rmsnorm(n, d):
    g = gen(n + d)
    x = R.bf(torch.randn(n, d, generator=g) * 3)
    delta = R.bf(torch.randn(n, d, generator=g))
    w = R.bf(torch.rand(d, generator=g) + 0.5)
    xd, dd, wd = to_dev(x, BF), to_dev(delta, BF), to_dev(w, BF)
    h = ops.add_rmsnorm(xd, wd, 1e-6, delta=dd)
    xr, hr = R.add_rmsnorm_fused(x, delta, w, 1e-6)
    assert torch.equal(xd.float().cpu(), xr)  # residual: exact
    ok, err = bf_close(h, hr, ulps=1)
    assert ok, err
    h2 = ops.add_rmsnorm(xd, wd, 1e-6)  # no delta: x unchanged
    assert torch.equal(xd.float().cpu(), xr)
    assert bf_close(h2, R.rmsnorm_fused(xr, w, 1e-6), ulps=1)[0]


def test_embed_rmsnorm():
    g = gen(5)
    emb = R.bf(torch.randn(343, 512, generator=g))
    w = R.bf(torch.rand(512, generator=g) + 0.5)
    tok = torch.tensor([0, 5, 342, 7, 7, 100])
    x, h = ops.embed_rmsnorm(to_dev(tok), to_dev(emb, BF), to_dev(w, BF), 1e-6)
    assert torch.equal(x.float().cpu(), emb[tok])
    assert bf_close(h, R.rmsnorm_fused(emb[tok], w, 1e-6), ulps=1)[0]


@pytest.mark.parametrize("table", ["f32", "bf16"])
@pytest.mark.parametrize("with_rope_pos", [False, True])
def test_qkv_rope_cache(table, with_rope_pos):
    g = gen(7)
    n, H, HKV, D, S, Bc = 300, 8, 2, 64, 700, 4
    qkv = R.bf(torch.randn(n, (H + 2 * HKV) * D, generator=g) * 2)
    qw = R.bf(torch.rand(D, generator=g) + 0.5)
    kw = R.bf(torch.rand(D, generator=g) + 0.5)
    cos, sin = R.rope_tables(D, 4096, 1e6)
    if table == "bf16":
        cos, sin = R.bf(cos), R.bf(sin)
    pos = torch.randperm(S, generator=g)[:n].int()   # distinct slots: every cache write is checkable
    seq = torch.randint(0, Bc, (n,), generator=g).int()
    rpos = (pos * 3 + 5).int() if with_rope_pos else None
    kc = torch.zeros(Bc, S, HKV, D, dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    tdt = torch.float32 if table == "f32" else BF
    q, k, v = ops.qkv_rope_cache(to_dev(qkv, BF), to_dev(qw, BF), to_dev(kw, BF), to_dev(cos, tdt), to_dev(sin, tdt),
                                 to_dev(pos), to_dev(seq), kc, vc, 1e-6, H, HKV, D, return_kv=True,
                                 rope_pos=None if rpos is None else to_dev(rpos))
    rp = (pos if rpos is None else rpos).long()
    x = qkv.view(n, H + 2 * HKV, D)
    qr = R.qk_norm_rope_fused(x[:, :H], qw, cos[rp], sin[rp], 1e-6)
    kr = R.qk_norm_rope_fused(x[:, H:H + HKV], kw, cos[rp], sin[rp], 1e-6)
    vr = x[:, H + HKV:]
    # one-ulp flips of the rounded norm output move the rotation by up to ~1 ulp of the head's scale
    assert bf_close(q, qr, ulps=2, atol=2e-2)[0]
    assert bf_close(k, kr, ulps=2, atol=2e-2)[0]
    assert torch.equal(v.float().cpu(), vr)
    kcc, vcc = kc.cpu(), vc.cpu()
    assert torch.equal(kcc[seq.long(), pos.long()], k.cpu()) and torch.equal(vcc[seq.long(), pos.long()], v.cpu())
    # nothing else written
    written = torch.zeros(Bc, S, dtype=torch.bool)
    written[seq.long(), pos.long()] = True
    assert not kcc[~written].any() and not vcc[~written].any()


def test_qkv_rope_cache_skips_out_of_range_rows():
    n, H, HKV, D = 4, 8, 2, 64
    qkv = torch.randn(n, 768, device=DEV).to(BF)
    cos, sin = R.rope_tables(D, 64, 1e4)
    kc = torch.zeros(2, 16, HKV, D, dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    pos = torch.tensor([0, 16, 3, 99], dtype=torch.int32, device=DEV)  # 16, 99 >= cache length
    seq = torch.tensor([0, 1, 5, 1], dtype=torch.int32, device=DEV)    # row 5 >= cache rows
    w = torch.ones(D, dtype=BF, device=DEV)
    ops.qkv_rope_cache(qkv, w, w, cos.to(DEV), sin.to(DEV), pos, seq, kc, vc, 1e-6, H, HKV, D)
    torch.cuda.synchronize()
    assert kc[0, 0].abs().sum() > 0 and int((kc.abs().sum((-1, -2)) > 0).sum()) == 1


@pytest.mark.parametrize("M,N,K", [(1, 768, 512), (17, 512, 512), (512, 3072, 512), (512, 512, 1536),
                                   (5000, 768, 512), (4099, 512, 1536), (64, 7, 512), (33, 343, 512),
                                   (130, 96, 96)])
def test_linear(M, N, K):
    g = gen(M + N + K)
    x = R.bf(torch.randn(M, K, generator=g))
    w = R.bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    y = ops.linear(to_dev(x, BF), to_dev(w, BF))
    ref = x.double() @ w.double().t()
    assert bf_close(y, ref.float(), ulps=1, atol=1e-5)[0]
    y32 = ops.linear(to_dev(x, BF), to_dev(w, BF), out_dtype=torch.float32)
    assert torch.allclose(y32.cpu().double(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,N,K", [(4099, 1536, 512), (8192, 520, 512), (4608, 512, 1536), (5000, 3072, 1024)])
def test_linear_large_m_tile_shapes_same_bits(M, N, K):
    """Large M: bf16 outputs run 256 x 256 tiles, fp32 outputs at K < 1024 the 256 x 128 tiles; both accumulate
    every output in the same K order, so the bf16 result is the fp32 result rounded, bit for bit (partial row
    and column tiles included)."""
    g = gen(M + 3 * N + K)
    x = to_dev(R.bf(torch.randn(M, K, generator=g)), BF)
    w = to_dev(R.bf(torch.randn(N, K, generator=g) / math.sqrt(K)), BF)
    y = ops.linear(x, w)
    y32 = ops.linear(x, w, out_dtype=torch.float32)
    assert torch.equal(y, y32.to(BF))
    ref = x.double() @ w.double().t()
    assert torch.allclose(y32.double(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M", [1, 100, 512, 4500])
def test_linear_swiglu(M):
    g = gen(M)
    Fd, K = 1536, 512
    x = R.bf(torch.randn(M, K, generator=g))
    w = R.bf(torch.randn(2 * Fd, K, generator=g) / math.sqrt(K))
    y = ops.linear(to_dev(x, BF), to_dev(w, BF), swiglu=True)
    gate = R.bf((x.double() @ w[:Fd].double().t()).float())
    up = R.bf((x.double() @ w[Fd:].double().t()).float())
    ref = R.swiglu_fused(gate, up)
    # three rounding points (gate, silu, product): a one-ulp flip upstream can reach ~3 ulps of the output
    ok, err = bf_close(y, ref, ulps=4, atol=1e-4)
    assert ok, err
    # the standalone SwiGLU op on the unfused GEMM output agrees (8 columns per thread: F % 8 == 0)
    gu = ops.linear(to_dev(x, BF), to_dev(w, BF))
    assert bf_close(ops.swiglu(gu), ref, ulps=4, atol=1e-4)[0]
    # gu_out: the same SwiGLU rows, and the gate | up rows of the plain product, bit for bit
    keep = torch.empty(M, 2 * Fd, dtype=BF, device=DEV)
    y2 = ops.linear(to_dev(x, BF), to_dev(w, BF), swiglu=True, gu_out=keep)
    assert torch.equal(y2, y) and torch.equal(keep, gu)


def test_swiglu_op_widths():
    """The standalone SwiGLU op, vectorised (F % 8 == 0) and per element (other F), equals the formula on
    the same bf16 inputs bit for bit."""
    g = gen(7)
    for Fd in (8, 1536, 12, 5):
        gu = R.bf(3 * torch.randn(37, 2 * Fd, generator=g))
        ref = R.swiglu_fused(gu[:, :Fd], gu[:, Fd:])
        got = ops.swiglu(to_dev(gu, BF)).float().cpu()
        assert bf_close(got, ref, ulps=1, atol=1e-6)[0], Fd


def _sdpa_ref(q, k, v, lens):
    B, H, D = q.shape
    S = k.shape[1]
    mask = (torch.arange(S)[None] < lens[:, None].long())[:, None, None]
    kk = k.transpose(1, 2).float().repeat_interleave(H // k.shape[2], 1)
    vv = v.transpose(1, 2).float().repeat_interleave(H // k.shape[2], 1)
    return F.scaled_dot_product_attention(q[:, :, None].float(), kk, vv, attn_mask=mask)[:, :, 0]


@pytest.mark.parametrize("B,S", [(64, 1300), (4, 3073), (512, 700), (3, 33)])
def test_decode_attention(B, S):
    torch.manual_seed(B + S)
    H, HKV, D = 8, 2, 64
    edge = torch.tensor([1, 63, 64, 65, S, 31, 32, 33]).clamp(max=S)[:B]
    lens = torch.cat([edge, torch.randint(1, S + 1, (B - len(edge),))]).int()
    q = torch.randn(B, H, D).to(BF)
    k = torch.randn(B, S, HKV, D).to(BF)
    v = torch.randn(B, S, HKV, D).to(BF)
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), lens.to(DEV))
    ref = _sdpa_ref(q, k, v, lens)
    err = (out.float().cpu() - ref).abs().max()
    assert err < 1e-2, float(err)
    # length 1 -> the first value row of each KV head
    i1 = int((lens == 1).nonzero()[0]) if (lens == 1).any() else None
    if i1 is not None:
        want = v[i1, 0].repeat_interleave(H // HKV, 0)
        assert torch.equal(out[i1].cpu(), want)


def test_decode_attention_cache_view_and_graph():
    """A layer view of a [L, B, S, 2, 64] cache, inside a captured graph replayed several times."""
    torch.manual_seed(3)
    L, B, S = 3, 16, 500
    kc = torch.randn(L, B, S, 2, 64, device=DEV).to(BF)
    vc = torch.randn(L, B, S, 2, 64, device=DEV).to(BF)
    q = torch.randn(B, 8, 64, device=DEV).to(BF)
    lens = torch.randint(1, S + 1, (B,), device=DEV).int()
    ws = ops.decode_attention_workspace(B, 8, S, DEV)
    eager = ops.decode_attention(q, kc[1], vc[1], lens, workspace=ws)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.decode_attention(q, kc[1], vc[1], lens, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.decode_attention(q, kc[1], vc[1], lens, workspace=ws)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    ref = _sdpa_ref(q.cpu(), kc[1].cpu(), vc[1].cpu(), lens.cpu())
    assert (eager.float().cpu() - ref).abs().max() < 1e-2


@pytest.mark.parametrize("B,S", [(6, 300), (700, 97)])
def test_decode_attention_row_map(B, S):
    """rows[b] picks sequence b's cache row (flash_attn_with_kvcache's cache_batch_idx at
    viktor/fast_decoder.py:86-89): a permutation over a larger cache, a repeated row, and a row outside the
    cache (zero output). Small B splits the key range (combine kernel), large B does not."""
    torch.manual_seed(B)
    Bc = B + 3
    q = torch.randn(B, 8, 64).to(BF)
    k = torch.randn(Bc, S, 2, 64).to(BF)
    v = torch.randn(Bc, S, 2, 64).to(BF)
    rows = torch.randperm(Bc)[:B].int()
    rows[1] = rows[0]
    rows[2] = Bc + 5  # outside the cache
    lens = torch.randint(1, S + 1, (B,)).int()
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), lens.to(DEV), rows=rows.to(DEV)).float().cpu()
    valid = (rows >= 0) & (rows < Bc)
    r = rows.clamp(0, Bc - 1).long()
    ref = _sdpa_ref(q, k[r], v[r], lens)
    assert (out[valid] - ref[valid]).abs().max() < 1e-2
    assert torch.equal(out[2], torch.zeros(8, 64))
    # without a row map the cache must hold one row per query: checked before any launch
    with pytest.raises(AssertionError, match="cache holds"):
        ops.decode_attention(q.to(DEV), k[:B - 1].to(DEV), v[:B - 1].to(DEV), lens.to(DEV))


@pytest.mark.parametrize("G,pre_max,suf_max", [(8, 2049, 1024), (4, 700, 33), (2, 65, 300), (16, 513, 64)])
def test_decode_attention_grouped(G, pre_max, suf_max):
    """Groups of G sequences share prefix rows [0, prefix_len) and own suffix rows [0, suffix_len): equal to
    attention over the concatenated rows."""
    torch.manual_seed(G * 1000 + pre_max)
    P = 6
    B, H, HKV, D = P * G, 8, 2, 64
    pre_edge = torch.tensor([1, 31, 32, 33, 512, 513, pre_max])
    plen = torch.cat([pre_edge, torch.randint(1, pre_max + 1, (P,))])[:P].clamp(max=pre_max).int()
    suf_edge = torch.tensor([1, 2, 31, 32, 33, suf_max])
    slen = torch.cat([suf_edge, torch.randint(1, suf_max + 1, (B,))])[:B].clamp(max=suf_max).int()
    q = torch.randn(B, H, D).to(BF)
    kp = torch.randn(P, pre_max, HKV, D).to(BF)
    vp = torch.randn(P, pre_max, HKV, D).to(BF)
    ks = torch.randn(B, suf_max, HKV, D).to(BF)
    vs = torch.randn(B, suf_max, HKV, D).to(BF)
    out = ops.decode_attention_grouped(q.to(DEV), kp.to(DEV), vp.to(DEV), plen.to(DEV), ks.to(DEV), vs.to(DEV),
                                       slen.to(DEV), G).cpu()
    for b in range(B):
        p, lp, ls = b // G, int(plen[b // G]), int(slen[b])
        k = torch.cat([kp[p, :lp], ks[b, :ls]])[None]
        v = torch.cat([vp[p, :lp], vs[b, :ls]])[None]
        ref = _sdpa_ref(q[b:b + 1], k, v, torch.tensor([lp + ls]))
        err = (out[b:b + 1].float() - ref).abs().max()
        assert err < 1e-2, (b, lp, ls, float(err))


@pytest.mark.parametrize("G,P,pre_max,suf_max", [(8, 64, 200, 70), (16, 64, 90, 33)])
def test_decode_attention_grouped_member_split(G, P, pre_max, suf_max):
    """Enough groups for each to be split into two halves of G / 2 members (one part each, output written by
    the attention kernel itself, no merge launch): equal to attention over the concatenated rows, and the
    same bits on a second call."""
    g = gen(G * 31 + P)
    B, H, HKV, D = P * G, 8, 2, 64
    plen = torch.randint(1, pre_max + 1, (P,), generator=g).int()
    plen[:4] = torch.tensor([1, 31, 32, pre_max])
    slen = torch.randint(1, suf_max + 1, (B,), generator=g).int()
    slen[:5] = torch.tensor([1, 2, 32, 33, suf_max])
    q = torch.randn(B, H, D, generator=g).to(BF)
    kp, vp = (torch.randn(P, pre_max, HKV, D, generator=g).to(BF) for _ in range(2))
    ks, vs = (torch.randn(B, suf_max, HKV, D, generator=g).to(BF) for _ in range(2))
    args = [t.to(DEV) for t in (q, kp, vp, plen, ks, vs, slen)]
    out = ops.decode_attention_grouped(*args, G)
    again = ops.decode_attention_grouped(*args, G)
    assert torch.equal(out, again)
    out = out.cpu()
    for b in list(range(0, B, 5)) + [G // 2 - 1, G // 2, B - 1]:
        p, lp, ls = b // G, int(plen[b // G]), int(slen[b])
        k = torch.cat([kp[p, :lp], ks[b, :ls]])[None]
        v = torch.cat([vp[p, :lp], vs[b, :ls]])[None]
        ref = _sdpa_ref(q[b:b + 1], k, v, torch.tensor([lp + ls]))
        err = (out[b:b + 1].float() - ref).abs().max()
        assert err < 1e-2, (b, lp, ls, float(err))


def test_decode_attention_grouped_cache_view_and_graph():
    """Layer views of [L, P, S, 2, 64] / [L, B, S, 2, 64] caches inside a graph replayed several times; the
    ungrouped kernel over the concatenated rows agrees to bf16 rounding."""
    torch.manual_seed(5)
    L, G, P, Sp, Ss = 2, 8, 4, 300, 40
    B = G * P
    kp = torch.randn(L, P, Sp, 2, 64, device=DEV).to(BF)
    vp = torch.randn(L, P, Sp, 2, 64, device=DEV).to(BF)
    ks = torch.randn(L, B, Ss, 2, 64, device=DEV).to(BF)
    vs = torch.randn(L, B, Ss, 2, 64, device=DEV).to(BF)
    q = torch.randn(B, 8, 64, device=DEV).to(BF)
    plen = torch.randint(1, Sp + 1, (P,), device=DEV).int()
    slen = torch.randint(1, Ss + 1, (B,), device=DEV).int()
    ws = ops.decode_attention_grouped_workspace(B, G, Sp, Ss, DEV)
    run = lambda: ops.decode_attention_grouped(q, kp[1], vp[1], plen, ks[1], vs[1], slen, G, workspace=ws)
    eager = run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    # ungrouped: concatenate prefix + suffix rows per sequence
    kc = torch.zeros(B, Sp + Ss, 2, 64, device=DEV, dtype=BF)
    vc = torch.zeros_like(kc)
    for b in range(B):
        lp, ls = int(plen[b // G]), int(slen[b])
        kc[b, :lp], vc[b, :lp] = kp[1, b // G, :lp], vp[1, b // G, :lp]
        kc[b, lp:lp + ls], vc[b, lp:lp + ls] = ks[1, b, :ls], vs[1, b, :ls]
    flat = ops.decode_attention(q, kc, vc, plen.repeat_interleave(G) + slen)
    assert (eager.float() - flat.float()).abs().max() < 1e-2


def test_decode_attention_grouped_rejects_bad_group():
    q = torch.zeros(12, 8, 64, device=DEV, dtype=BF)
    kp = torch.zeros(2, 8, 2, 64, device=DEV, dtype=BF)
    ks = torch.zeros(12, 8, 2, 64, device=DEV, dtype=BF)
    with pytest.raises(Exception, match="group size"):
        ops.decode_attention_grouped(q, kp, kp, torch.ones(2, dtype=torch.int32, device=DEV), ks, ks,
                                     torch.ones(12, dtype=torch.int32, device=DEV), 6,
                                     workspace=torch.empty(1 << 20, dtype=torch.uint8, device=DEV))


def _varlen_ref(q, k, v, q_lens, k_lens, causal=True):
    outs = []
    qo = ko = 0
    for ql, kl in zip(q_lens, k_lens):
        outs.append(R.attention_rows(q[qo:qo + ql].float(), k[ko:ko + kl].float(), v[ko:ko + kl].float(),
                                     causal_shift=(kl - ql) if causal else None))
        qo += ql
        ko += kl
    return torch.cat(outs)


@pytest.mark.parametrize("q_lens,k_lens", [([1, 63, 64, 65, 200], [1, 63, 64, 65, 200]),
                                            ([2049, 700], [2049, 700]),
                                            ([1, 1, 1], [2049, 5, 1300]),
                                            ([40, 130], [100, 130])])
def test_varlen_attention_packed(q_lens, k_lens):
    torch.manual_seed(sum(q_lens))
    H, HKV, D = 8, 2, 64
    q = torch.randn(sum(q_lens), H, D).to(BF)
    k = torch.randn(sum(k_lens), HKV, D).to(BF)
    v = torch.randn(sum(k_lens), HKV, D).to(BF)
    k_off, o = [], 0
    for kl in k_lens:
        k_off.append(o * HKV * D)
        o += kl
    plan = ops.AttentionPlan(q_lens, k_lens, k_off, DEV, causal=True)
    out = ops.varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), plan, stride_tok=HKV * D)
    ref = _varlen_ref(q, k, v, q_lens, k_lens)
    err = (out.float().cpu() - ref).abs().max()
    assert err < 1e-2, float(err)


def test_varlen_attention_reads_cache_rows():
    torch.manual_seed(11)
    H, HKV, D, Bc, S = 8, 2, 64, 5, 400
    kc = torch.randn(Bc, S, HKV, D).to(BF)
    vc = torch.randn(Bc, S, HKV, D).to(BF)
    rows, lens = [3, 0, 4], [120, 377, 64]
    q = torch.randn(sum(lens), H, D).to(BF)
    plan = ops.AttentionPlan(lens, lens, [r * S * HKV * D for r in rows], DEV, causal=True)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    out = ops.varlen_attention(q.to(DEV), kcd, vcd, plan, stride_tok=kcd.stride(1))
    ks = torch.cat([kc[r, :n] for r, n in zip(rows, lens)])
    vs = torch.cat([vc[r, :n] for r, n in zip(rows, lens)])
    ref = _varlen_ref(q, ks, vs, lens, lens)
    assert (out.float().cpu() - ref).abs().max() < 1e-2


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_attention_prefixed_equals_concatenated_keys(causal):
    """Each sequence's first p_lens keys from a shared prefix buffer, the rest its own rows: the same bits (out and
    log-sum-exp) as vk_varlen_attention over the concatenated keys -- prefix lengths off and on the 64-key tiles
    (tiles straddling the two buffers), two sequences on one prefix, an empty own part, a sequence with no prefix."""
    torch.manual_seed(31)
    H, HKV, D = 8, 2, 64
    pre = [(0, 100), (100, 128), (228, 77)]  # (first row, length) of three prefixes in one packed buffer
    kp = torch.randn(305, HKV, D).to(BF)
    vp = torch.randn(305, HKV, D).to(BF)
    # sequences: (prefix index or None, own keys, queries)
    seqs = [(0, 150, 150), (0, 40, 40), (1, 0, 0), (2, 300, 200), (None, 90, 90), (1, 64, 1)]
    if not causal:
        seqs[2] = (1, 0, 5)  # queries over the prefix keys alone
    q_lens = [nq for _, _, nq in seqs]
    own = [no for _, no, _ in seqs]
    p_lens = [0 if p is None else pre[p][1] for p, _, _ in seqs]
    p_off = [0 if p is None else pre[p][0] * HKV * D for p, _, _ in seqs]
    k_lens = [a + b for a, b in zip(p_lens, own)]
    ko = torch.randn(max(sum(own), 1), HKV, D).to(BF)
    vo = torch.randn(max(sum(own), 1), HKV, D).to(BF)
    k_off = list(np.concatenate([[0], np.cumsum(own)[:-1]]) * HKV * D)
    q = torch.randn(sum(q_lens), H, D).to(BF)
    dq, dkp, dvp, dko, dvo = (t.to(DEV) for t in (q, kp, vp, ko, vo))
    plan = ops.AttentionPlan(q_lens, k_lens, k_off, DEV, causal=causal, p_lens=p_lens, p_off=p_off)
    lse = torch.empty(sum(q_lens), H, dtype=torch.float32, device=DEV)
    out = ops.varlen_attention(dq, dko, dvo, plan, stride_tok=HKV * D, lse=lse, prefix=(dkp, dvp))
    # the same keys concatenated per sequence, one buffer
    kc, vc, c_off, o = [], [], [], 0
    oo = np.concatenate([[0], np.cumsum(own)])
    for i, (p, no, _) in enumerate(seqs):
        parts_k = ([kp[pre[p][0]:pre[p][0] + pre[p][1]]] if p is not None else []) + [ko[oo[i]:oo[i] + no]]
        parts_v = ([vp[pre[p][0]:pre[p][0] + pre[p][1]]] if p is not None else []) + [vo[oo[i]:oo[i] + no]]
        kc.append(torch.cat(parts_k))
        vc.append(torch.cat(parts_v))
        c_off.append(o * HKV * D)
        o += k_lens[i]
    kc, vc = torch.cat(kc).to(DEV), torch.cat(vc).to(DEV)
    plan_c = ops.AttentionPlan(q_lens, k_lens, c_off, DEV, causal=causal)
    lse_c = torch.empty_like(lse)
    out_c = ops.varlen_attention(dq, kc, vc, plan_c, stride_tok=HKV * D, lse=lse_c)
    assert torch.equal(out, out_c)
    assert torch.equal(lse, lse_c)
    ref = _varlen_ref(q, kc.cpu(), vc.cpu(), q_lens, k_lens, causal=causal)
    assert (out.float().cpu() - ref).abs().max() < 1e-2
    with pytest.raises(AssertionError, match="prefix tensors go with a prefixed plan"):
        ops.varlen_attention(dq, kc, vc, plan_c, stride_tok=HKV * D, prefix=(dkp, dvp))


def _select_ref(logits, prev, run, bias, tail, homo, homo_stop, T, u, gumbel=False):
    toks, runs, margins = [], [], []
    for b in range(logits.shape[0]):
        z = logits[b] + bias
        if T > 0 and gumbel:
            raw, m = R.sample_gumbel(z / T, u[b].numpy())
        elif T > 0:
            raw, m = R.sample_inverse_cdf(z / T, float(u[b]))
        else:
            raw, m = R.greedy_choice(z)
        nxt, r = R.apply_grammar(raw, int(prev[b]), int(run[b]), tail, homo, homo_stop)
        toks.append(nxt)
        runs.append(r)
        margins.append(m)
    return torch.tensor(toks), torch.tensor(runs), torch.tensor(margins)


def _state(B, V, g, P=50):
    tok = torch.randint(0, V, (B,), generator=g)
    tok[:4] = torch.tensor([R.EOS, R.PAD, 5, 3]) if V > 6 else tok[:4]
    run = torch.randint(0, 5, (B,), generator=g)
    plen = torch.randint(10, P, (B,), generator=g)
    pos = plen + torch.randint(0, 20, (B,), generator=g)
    rope_off = plen * 2
    return tok, run, pos, plen, rope_off


@pytest.mark.parametrize("V,T,fused_head,gumbel", [(7, 0.0, False, False), (7, 1.0, False, False),
                                                    (343, 0.0, False, False), (343, 0.7, False, False),
                                                    (7, 0.0, True, False), (343, 1.0, True, False),
                                                    (7, 1.0, False, True), (343, 0.7, False, True),
                                                    (343, 1.0, True, True)])
def test_select_update(V, T, fused_head, gumbel):
    """The choice + grammar + bookkeeping against the oracle's: greedy, inverse-CDF sampling and the reference's
    Gumbel-max formula (uniforms [B, T, V]), from fp32 logits (exactly, ties to the first index) or from the fused
    LM head (exempt where the oracle's margin is under the bf16 logits' rounding)."""
    g = gen(V + int(T * 10) + int(fused_head) + 5 * int(gumbel))
    B, d, max_new = 300, 512, 64
    bias = torch.zeros(V)
    bias[[R.PAD, R.BOS]] = float("-inf")
    tail = torch.zeros(V, dtype=torch.bool)
    if V > 7:
        tail[259:] = True
    else:
        tail[5] = True  # make the tail rule reachable in the small vocabulary too
    homo = torch.zeros(V, dtype=torch.bool)
    homo[3:7] = True
    homo_stop = 4
    tok, run, pos, plen, rope_off = _state(B, V, g)
    u = torch.rand(B, max_new, V, generator=g) if gumbel else torch.rand(B, max_new, generator=g)
    if fused_head:
        h = R.bf(torch.randn(B, d, generator=g))
        w = R.bf(torch.randn(V, d, generator=g) / math.sqrt(d) * 3)
        logits = h.double() @ w.double().t()
        logits = R.bf(logits.float()) if T > 0 else logits.float()
    else:
        logits = torch.randn(B, V, generator=g) * 2
        logits[10, 3] = logits[10, 4] = 50.0  # exact tie -> first index
        tok[10], run[10] = 6, 0  # a previous token that triggers no grammar rule for 3 / 4
    col = (pos - plen).clamp(0, max_new - 1)
    ub = u[torch.arange(B), col]
    want_tok, want_run, margin = _select_ref(logits, tok, run, bias, tail, homo, homo_stop, T, ub, gumbel)
    out = torch.full((B, max_new), R.PAD, dtype=torch.long)
    d_tok, d_run, d_pos = to_dev(tok), to_dev(run), to_dev(pos)
    d_out = to_dev(out)
    pos32 = torch.zeros(B, dtype=torch.int32, device=DEV)
    seql = torch.zeros_like(pos32)
    rpos = torch.zeros_like(pos32)
    kw = dict(logits=to_dev(logits.float())) if not fused_head else dict(h=to_dev(h, BF), w_head=to_dev(w, BF),
                                                                          round_bf16=T > 0)
    ops.select_update(to_dev(bias), to_dev(tail), to_dev(homo), homo_stop, d_tok, d_run, d_pos, to_dev(plen),
                      to_dev(rope_off), d_out, pos32, seql, rpos, R.EOS, R.PAD, temperature=T, uniforms=to_dev(u),
                      gumbel=gumbel, **kw)
    got = d_tok.cpu()
    thr = 1e-2 if T == 0 else (3e-2 if gumbel else 5e-3)
    exempt = margin < thr if fused_head else torch.zeros(B, dtype=torch.bool)
    assert bool(((got == want_tok) | exempt).all()), (got != want_tok).nonzero()[:5]
    if not fused_head:
        assert int(got[10]) in (3, 4) and (T > 0 or int(got[10]) == 3)
    same = got == want_tok
    assert torch.equal(d_run.cpu()[same], want_run[same])
    assert torch.equal(d_pos.cpu(), pos + 1)
    assert torch.equal(pos32.cpu(), (pos + 1).int()) and torch.equal(seql.cpu(), (pos + 2).int())
    assert torch.equal(rpos.cpu(), (pos + 1 + rope_off).int())
    oc = d_out.cpu()
    c = pos - plen
    for b in range(B):
        if 0 <= int(c[b]) < max_new:
            assert int(oc[b, c[b]]) == int(got[b])


@pytest.mark.parametrize("T", [0.0, 0.8])
def test_select_update_logprob_rows(T):
    """logp_out [B, T]: the chosen token's log-probability goes to the column the token is written to,
    log softmax((z + bias) / T)[token] (greedy: of z + bias), computed here in fp64."""
    g = gen(31)
    B, V, max_new = 50, 343, 16
    bias = torch.zeros(V)
    bias[[R.PAD, R.BOS, R.EOS]] = float("-inf")
    logits = torch.randn(B, V, generator=g) * 2
    plen = torch.randint(10, 40, (B,), generator=g)
    pos = plen + torch.randint(0, max_new, (B,), generator=g)
    tok = torch.full((B,), 5, dtype=torch.long)
    u = torch.rand(B, max_new, generator=g)
    d_tok, d_pos = to_dev(tok), to_dev(pos)
    lp = torch.full((B, max_new), 7.0, device=DEV)
    out = torch.full((B, max_new), R.PAD, dtype=torch.long, device=DEV)
    ops.select_update(to_dev(bias), torch.zeros(V, dtype=torch.bool, device=DEV), torch.zeros(V, dtype=torch.bool,
                      device=DEV), 0, d_tok, torch.zeros(B, dtype=torch.long, device=DEV), d_pos, to_dev(plen),
                      torch.zeros(B, dtype=torch.long, device=DEV), out, None, None, None, R.EOS, R.PAD,
                      logits=to_dev(logits), temperature=T, uniforms=to_dev(u), logp_out=lp)
    z = (logits.double() + bias.double()) / (T if T > 0 else 1.0)
    want = torch.log_softmax(z, -1).gather(1, d_tok.cpu()[:, None])[:, 0]
    col = (pos - plen).long()
    got = lp.cpu()
    assert (got[torch.arange(B), col].double() - want).abs().max() < 1e-5
    untouched = torch.ones(B, max_new, dtype=torch.bool)
    untouched[torch.arange(B), col] = False
    assert bool((got[untouched] == 7.0).all())


def test_greedy_update_reference_signature():
    """hip_ops.greedy_update with viktor/triton_ops.py:200-209's argument list: first-index argmax of
    logits + bias, tail -> EOS, homopolymer run -> EOS, PAD after EOS / PAD, out[b, pos - plen] and the
    pos / pos32 / seqlens / rpos32 advance."""
    g = gen(77)
    B, V, max_new = 64, 7, 32
    bias = torch.zeros(V)
    bias[[R.PAD, R.BOS]] = float("-inf")
    tail = torch.zeros(V, dtype=torch.bool)
    tail[6] = True
    homo = torch.zeros(V, dtype=torch.bool)
    homo[3:7] = True
    homo_stop = 3
    tok, run, pos, plen, rope_off = _state(B, V, g)
    logits = torch.randn(B, V, generator=g) * 2
    logits[7, 3] = logits[7, 5] = 40.0  # tie: the first index wins
    tok[7], run[7] = 4, 0
    want_tok, want_run, _ = _select_ref(logits, tok, run, bias, tail, homo, homo_stop, 0.0, torch.zeros(B))
    d = {n: to_dev(t) for n, t in dict(tok=tok, run=run, pos=pos, plen=plen, rope_off=rope_off).items()}
    out = torch.full((B, max_new), R.PAD, dtype=torch.long, device=DEV)
    pos32 = torch.zeros(B, dtype=torch.int32, device=DEV)
    seql, rpos = torch.zeros_like(pos32), torch.zeros_like(pos32)
    ops.greedy_update(to_dev(logits), to_dev(bias), to_dev(tail), to_dev(homo), homo_stop, d["tok"], d["run"],
                      d["pos"], d["plen"], d["rope_off"], out, pos32, seql, rpos, R.EOS, R.PAD)
    assert torch.equal(d["tok"].cpu(), want_tok) and torch.equal(d["run"].cpu(), want_run)
    assert int(want_tok[7]) == 3
    assert torch.equal(d["pos"].cpu(), pos + 1) and torch.equal(pos32.cpu(), (pos + 1).int())
    assert torch.equal(seql.cpu(), (pos + 2).int()) and torch.equal(rpos.cpu(), (pos + 1 + rope_off).int())
    oc = out.cpu()
    for b in range(B):
        c = int(pos[b] - plen[b])
        if 0 <= c < max_new:
            assert int(oc[b, c]) == int(want_tok[b])


@pytest.mark.parametrize("V,dtype", [(7, torch.float32), (7, BF), (343, BF)])
def test_gspo_score(V, dtype):
    g = gen(V)
    B, T = 40, 300
    logits = torch.randn(B, T, V, generator=g) * 2
    if dtype == BF:
        logits = R.bf(logits)
    targets = torch.randint(3, V, (B, T), generator=g)
    targets[:, -5:] = R.PAD
    mask = torch.rand(B, T, generator=g) > 0.1
    mask[:, -5:] = False
    lp_true = R.token_logprobs_ref(logits, targets)
    old = lp_true + torch.randn(B, T, generator=g) * 0.05
    old[3] = lp_true[3]  # ratio exactly 1 on one sequence
    n_bases = mask.sum(1).float().clamp(min=1)
    adv = torch.randn(B, generator=g)
    adv[0] = 0.0
    eps_lo, eps_hi = 3e-4, 4e-4
    res = ops.gspo_score(to_dev(logits, dtype), to_dev(targets), to_dev(mask), to_dev(old), to_dev(n_bases), to_dev(adv),
                         eps_lo, eps_hi, inv_n=1.0 / B)
    loss, s, pg, lp, grad = R.gspo_loss_autograd(logits, targets, mask, old, n_bases, adv, eps_lo, eps_hi, 1.0 / B)
    assert torch.allclose(res["lp"].cpu(), lp, rtol=1e-5, atol=1e-5)
    assert torch.allclose(res["s"].cpu(), s, rtol=1e-4)
    assert torch.allclose(res["pg"].cpu(), pg, rtol=1e-4, atol=1e-6)
    assert abs(float(res["loss"]) - float(loss)) <= 1e-4 * abs(float(loss)) + 1e-7
    assert torch.allclose(res["dlogits"].cpu(), grad, rtol=1e-4, atol=1e-8)
    assert float(res["s"][3]) == pytest.approx(1.0, abs=1e-6)
    assert torch.all(res["dlogits"][0] == 0)


def test_group_advantage():
    r = torch.tensor([[0.5, 0.7, 0.9, 0.9], [0.8, 0.8, 0.8, 0.8], [0.1, 0.2, 0.3, 0.9]])
    for kw in (dict(std_floor=0.003), dict(eps=1e-6)):
        adv, live = ops.group_advantage(r.to(DEV), **kw)
        want, want_live = R.advantages_ref(r.numpy(), **kw)
        assert np.allclose(adv.cpu().numpy(), want, rtol=1e-4, atol=1e-5)
        assert live.cpu().nonzero()[:, 0].tolist() == list(want_live)


# ---- decode-step fusions: against the oracle's composition of the unfused ops ------------------------
def _row_ss(x, block=32):
    """[M, K / block] fp32 partial sums of squares of the rows of x, one per block of columns (32: the
    decode-step products' hand-over)."""
    M, K = x.shape
    return (x.double() ** 2).view(M, K // block, block).sum(-1).float()


@pytest.mark.parametrize("M", [1, 45, 512, 1100])
@pytest.mark.parametrize("embed", [False, True, "ss"])
def test_norm_qkv_rope_cache(M, embed):
    use_ss = embed == "ss"
    embed = embed is True
    g = gen(M + int(embed))
    H, HKV, D, K, S, Bc = 8, 2, 64, 512, 300, max(M, 2)
    emb = R.bf(torch.randn(7, K, generator=g))
    tok = torch.randint(0, 7, (M,), generator=g)
    x = emb[tok] if embed else R.bf(torch.randn(M, K, generator=g) * 2)
    nw = R.bf(torch.rand(K, generator=g) + 0.5)
    wq = R.bf(torch.randn((H + 2 * HKV) * D, K, generator=g) / math.sqrt(K))
    qw = R.bf(torch.rand(D, generator=g) + 0.5)
    kw = R.bf(torch.rand(D, generator=g) + 0.5)
    cos, sin = R.rope_tables(D, 4096, 1e6)
    cos, sin = R.bf(cos), R.bf(sin)
    pos = torch.randint(0, S, (M,), generator=g).int()
    seq = torch.randperm(Bc, generator=g)[:M].int()
    kc = torch.zeros(Bc, S, HKV, D, dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    xs = torch.zeros(M, K, dtype=BF, device=DEV)
    if embed:
        q = ops.norm_qkv_rope_cache(to_dev(emb, BF), to_dev(nw, BF), 1e-6, to_dev(wq, BF), to_dev(qw, BF), to_dev(kw, BF),
                                    to_dev(cos, BF), to_dev(sin, BF), to_dev(pos), to_dev(seq), kc, vc, H, HKV, D,
                                    tok=to_dev(tok), x_store=xs)
        assert torch.equal(xs.float().cpu(), x)
    else:
        # ss: 1 / rms from handed-over row sums of squares instead of the kernel's own pre-pass
        q = ops.norm_qkv_rope_cache(to_dev(x, BF), to_dev(nw, BF), 1e-6, to_dev(wq, BF), to_dev(qw, BF), to_dev(kw, BF),
                                    to_dev(cos, BF), to_dev(sin, BF), to_dev(pos), to_dev(seq), kc, vc, H, HKV, D,
                                    ss=to_dev(_row_ss(x)) if use_ss else None)
    h = R.rmsnorm_fused(x, nw, 1e-6)
    qkv = R.linear_fused(h, wq).view(M, H + 2 * HKV, D)
    rp = pos.long()
    qr = R.qk_norm_rope_fused(qkv[:, :H], qw, cos[rp], sin[rp], 1e-6)
    kr = R.qk_norm_rope_fused(qkv[:, H:H + HKV], kw, cos[rp], sin[rp], 1e-6)
    # the fused norm sums squares in another order: a one-ulp flip of an h element moves qkv by ~|w| ulp(h),
    # then two more bf16 roundings (QK-norm, RoPE) follow
    ok, err = bf_close(q, qr, ulps=4, atol=4e-2)
    assert ok, err
    kcc, vcc = kc.cpu().float(), vc.cpu().float()
    ok, err = bf_close(kcc[seq.long(), pos.long()], kr, ulps=4, atol=4e-2)
    assert ok, err
    ok, err = bf_close(vcc[seq.long(), pos.long()], qkv[:, H + HKV:], ulps=1, atol=4e-3)
    assert ok, err


@pytest.mark.parametrize("M,tables", [(300, "bf16"), (4500, "f32")])
def test_linear_qkv_rope(M, tables):
    """The Wqkv product with QK-norm + RoPE + cache write in its epilogue against the oracle's composition of the
    fused path's rounding points, and against the unfused pair (linear, then qkv_rope_cache); the kept unrotated
    product (qkv_out) against linear."""
    g = gen(M + 5)
    H, HKV, D, K, S, Bc = 8, 2, 64, 512, 300, M
    x = R.bf(torch.randn(M, K, generator=g) * 2)
    wq = R.bf(torch.randn((H + 2 * HKV) * D, K, generator=g) / math.sqrt(K))
    qw = R.bf(torch.rand(D, generator=g) + 0.5)
    kw = R.bf(torch.rand(D, generator=g) + 0.5)
    cos, sin = R.rope_tables(D, 4096, 1e6)
    if tables == "bf16":
        cos, sin = R.bf(cos), R.bf(sin)
    tdt = BF if tables == "bf16" else torch.float32
    pos = torch.randint(0, S, (M,), generator=g).int()
    rpos = torch.randint(0, 4096, (M,), generator=g).int()
    seq = torch.randperm(Bc, generator=g)[:M].int()
    kc = torch.zeros(Bc, S, HKV, D, dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    dev = [to_dev(t, BF) for t in (x, wq, qw, kw)] + [to_dev(cos, tdt), to_dev(sin, tdt)]
    raw = torch.empty(M, (H + 2 * HKV) * D, dtype=BF, device=DEV)
    q, k, v = ops.linear_qkv_rope(dev[0], dev[1], dev[2], dev[3], dev[4], dev[5], to_dev(pos), to_dev(seq), kc, vc,
                                  1e-6, H, HKV, D, return_kv=True, rope_pos=to_dev(rpos), qkv_out=raw)
    qkv = R.linear_fused(x, wq).view(M, H + 2 * HKV, D)
    rp = rpos.long()
    qr = R.qk_norm_rope_fused(qkv[:, :H], qw, cos[rp], sin[rp], 1e-6)
    kr = R.qk_norm_rope_fused(qkv[:, H:H + HKV], kw, cos[rp], sin[rp], 1e-6)
    # the GEMM output can sit on a bf16 rounding boundary; the norm's sum of squares runs in another order
    for got, want in ((q, qr), (k, kr)):
        ok, err = bf_close(got, want, ulps=4, atol=4e-2)
        assert ok, err
    ok, err = bf_close(v, qkv[:, H + HKV:], ulps=1, atol=4e-3)
    assert ok, err
    assert torch.equal(kc.cpu()[seq.long(), pos.long()], k.cpu()) and torch.equal(vc.cpu()[seq.long(), pos.long()], v.cpu())
    # the unfused pair on the same device: the same values up to the norm's summation order
    qkv_d = ops.linear(dev[0], dev[1])
    assert torch.equal(raw, qkv_d)  # the kept unrotated projection is the plain product, bit for bit
    q2, k2, v2 = ops.qkv_rope_cache(qkv_d, dev[2], dev[3], dev[4], dev[5], to_dev(pos), None, None, None, 1e-6, H, HKV,
                                    D, return_kv=True, rope_pos=to_dev(rpos))
    assert torch.equal(v2, v)
    for a, b in ((q, q2), (k, k2)):
        d = (a.float() - b.float()).abs()
        assert (d > 0).float().mean() < 1e-3 and bf_close(a, b.float().cpu(), ulps=2, atol=2e-2)[0]


@pytest.mark.parametrize("M,N,K,alpha,bias", [(4500, 512, 512, 1.0, False), (700, 512, 2048, 2.4494897, True)])
def test_linear_residual_big_and_rmsnorm_apply(M, N, K, alpha, bias):
    """x = bf16(bf16(a w^T + b) + bf16(alpha x)) in place with per-64-column sums of squares (out of place: the same
    bits, x untouched), then the RMSNorm from those sums, against the formulas (and, for alpha 1 without bias,
    against add_rmsnorm of the unfused product)."""
    g = gen(M + K)
    a = R.bf(torch.randn(M, K, generator=g))
    w = R.bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    x = R.bf(torch.randn(M, N, generator=g) * 2)
    b = R.bf(0.1 * torch.randn(N, generator=g)) if bias else None
    nw = R.bf(torch.rand(N, generator=g) + 0.5)
    xd = to_dev(x, BF)
    # out of place first (the old stream read from x, the new one written to out, x untouched): the same bits
    x_keep, out = to_dev(x, BF), torch.empty(M, N, dtype=BF, device=DEV)
    ss_o = ops.linear_residual_big(to_dev(a, BF), to_dev(w, BF), x_keep, bias=None if b is None else to_dev(b),
                                   alpha=alpha, out=out)
    ss = ops.linear_residual_big(to_dev(a, BF), to_dev(w, BF), xd, bias=None if b is None else to_dev(b), alpha=alpha)
    assert torch.equal(out, xd) and torch.equal(ss_o, ss) and torch.equal(x_keep.cpu(), x)
    acc = (a.double() @ w.double().t()).float() + (0 if b is None else b)
    want = R.bf(R.bf(acc) + R.bf(alpha * x))
    ok, err = bf_close(xd, want, ulps=1, atol=2e-2)  # an accumulation-order flip of bf16(acc) moves the sum one ulp
    assert ok, err
    xn = xd.float().cpu().double()
    ss_ref = (xn * xn).view(M, N // 64, 64).sum(-1)
    assert torch.allclose(ss.cpu().double(), ss_ref, rtol=1e-5, atol=1e-6)
    h = ops.rmsnorm_apply(xd, ss, to_dev(nw, BF), 1e-6)
    ok, err = bf_close(h, R.rmsnorm_fused(xd.float().cpu(), nw, 1e-6), ulps=1, atol=1e-5)
    assert ok, err
    if alpha == 1.0 and b is None:
        xu = to_dev(x, BF)
        hu = ops.add_rmsnorm(xu, to_dev(nw, BF), 1e-6, delta=ops.linear(to_dev(a, BF), to_dev(w, BF)))
        assert torch.equal(xu, xd)  # the same residual (the product is the same kernel)
        assert bf_close(h, hu.float().cpu(), ulps=1, atol=1e-5)[0]


@pytest.mark.parametrize("n,d,nb", [(4099, 512, 8), (1, 512, 16), (6, 512, 2), (37, 256, 4), (9, 1024, 16)])
def test_rmsnorm_apply_paths(n, d, nb):
    """The norm from handed-over block sums on each path: d = 512 with four rows per wavefront (partials as vector
    loads when nb % 4 == 0, one by one otherwise; row counts that leave a wavefront's group partly empty) and
    one row per wavefront for other d; bit-equal in place and out of place, against the formula in fp64."""
    g = gen(n + d + nb)
    x = R.bf(torch.randn(n, d, generator=g) * 2)
    nw = R.bf(torch.rand(d, generator=g) + 0.5)
    xd = x.double()
    ss = (xd * xd).view(n, nb, d // nb).sum(-1).float()
    h = ops.rmsnorm_apply(to_dev(x, BF), to_dev(ss), to_dev(nw, BF), 1e-6)
    xi = to_dev(x, BF)
    ops.rmsnorm_apply(xi, to_dev(ss), to_dev(nw, BF), 1e-6, out=xi)
    assert torch.equal(h, xi)
    tot = torch.zeros(n)
    for b in range(nb):  # the kernel's order: block 0 first
        tot = tot + ss[:, b]
    r = torch.rsqrt(tot / d + 1e-6)
    want = R.bf((x.float() * r[:, None]) * nw.float())
    ok, err = bf_close(h, want, ulps=1, atol=1e-5)
    assert ok, err


@pytest.mark.parametrize("M,K,alpha,bias", [(4500, 512, 1.0, False), (300, 1536, 1.0, False), (700, 512, 0.5, True)])
def test_linear_residual_big_fp32_stream(M, K, alpha, bias):
    """The autocast residual add on an fp32 stream: x = alpha x + bf16(a w^T + b) in place (fp32), bit for bit
    against the same product's fp32 accumulator (and that against fp64), the per-64-column sums of squares of the
    new fp32 values, then the norm from those sums with fp32 weights (rmsnorm_apply) and the norm that takes its own
    sums (rmsnorm_f32), each against fp64 with one bf16 rounding."""
    g = gen(M + K + 1)
    N = 512
    a = R.bf(torch.randn(M, K, generator=g))
    w = R.bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    x = torch.randn(M, N, generator=g) * 2  # fp32 values, not bf16
    b = R.bf(0.1 * torch.randn(N, generator=g)) if bias else None
    nw = torch.rand(N, generator=g) + 0.5  # fp32 master weights
    xd = to_dev(x)
    x_keep, out = to_dev(x), torch.empty(M, N, dtype=torch.float32, device=DEV)
    ss_o = ops.linear_residual_big(to_dev(a, BF), to_dev(w, BF), x_keep, bias=None if b is None else to_dev(b),
                                   alpha=alpha, out=out)
    ss = ops.linear_residual_big(to_dev(a, BF), to_dev(w, BF), xd, bias=None if b is None else to_dev(b), alpha=alpha)
    assert torch.equal(out, xd) and torch.equal(ss_o, ss) and torch.equal(x_keep.cpu(), x)  # out of place: same bits
    # the same kernel's fp32 accumulator (its fp32-output epilogue): the residual is then exact --
    # alpha x + bf16(acc + b) with one fp32 rounding (alpha is a power of two here, so alpha x is exact)
    from viktor_amd._lib import call, ptr, stream_handle
    ad, wd = to_dev(a, BF), to_dev(w, BF)
    acc32 = torch.empty(M, N, dtype=torch.float32, device=DEV)
    call("vk_gemm_rows", ptr(ad), ptr(wd), ptr(acc32), M, N, K, 1, stream_handle())  # the large-M kernel, fp32 out
    acc32 = acc32.cpu()
    prod = R.bf(acc32 + (0 if b is None else b))
    got = xd.cpu().double()
    assert torch.equal(xd.cpu(), alpha * x + prod)
    acc = a.double() @ w.double().t()
    assert torch.allclose(acc32.double(), acc, rtol=1e-5, atol=1e-5)
    ss_ref = (got * got).view(M, N // 64, 64).sum(-1)
    assert torch.allclose(ss.cpu().double(), ss_ref, rtol=1e-5, atol=1e-6)
    ref_h = R.bf(F.rms_norm(xd.cpu(), (N,), nw, 1e-6))
    for h in (ops.rmsnorm_apply(xd, ss, to_dev(nw), 1e-6), ops.rmsnorm_f32(xd, to_dev(nw), 1e-6)):
        assert h.dtype == BF
        ok, err = bf_close(h, ref_h, ulps=1, atol=1e-5)
        assert ok, err


@pytest.mark.parametrize("n,d", [(1, 512), (333, 512), (40, 256), (17, 1536), (5, 64)])
def test_rmsnorm_f32(n, d):
    """bf16(x rsqrt(mean x^2 + eps) w) of fp32 x and w: one rounding of the fp64 value (1 ulp)."""
    g = gen(n * d)
    x = torch.randn(n, d, generator=g) * 3
    w = torch.rand(d, generator=g) + 0.5
    h = ops.rmsnorm_f32(to_dev(x), to_dev(w), 1e-6)
    xd = x.double()
    want = xd * torch.rsqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    ok, err = bf_close(h, want.float(), ulps=1, atol=1e-6)
    assert ok, err


@pytest.mark.parametrize("M", [300, 4500])
def test_linear_qkv_rope_fp32_norm_weights(M):
    """The autocast Wqkv stage: fp32 QK-norm weights that bf16 cannot hold and fp32 tables -- bf16(x / rms * w) with
    the fp32 weight, then the rotation rounded to bf16 -- against the oracle's composition, and against the unfused
    pair (linear, then qkv_rope_cache with the same fp32 weights)."""
    g = gen(M + 77)
    H, HKV, D, K = 8, 2, 64, 512
    x = R.bf(torch.randn(M, K, generator=g) * 2)
    wq = R.bf(torch.randn((H + 2 * HKV) * D, K, generator=g) / math.sqrt(K))
    qw = 1 + 0.1 * torch.randn(D, generator=g)
    kw = 1 + 0.1 * torch.randn(D, generator=g)
    assert not torch.equal(R.bf(qw), qw)
    cos, sin = R.rope_tables(D, 4096, 1e6)
    rpos = torch.randint(0, 4096, (M,), generator=g).int()
    pos = torch.arange(M).int()
    q, k, v = ops.linear_qkv_rope(to_dev(x, BF), to_dev(wq, BF), to_dev(qw), to_dev(kw), to_dev(cos), to_dev(sin),
                                  to_dev(pos), None, None, None, 1e-6, H, HKV, D, return_kv=True, rope_pos=to_dev(rpos))
    qkv = R.linear_fused(x, wq).view(M, H + 2 * HKV, D)
    rp = rpos.long()
    for got, part, nw in ((q, qkv[:, :H], qw), (k, qkv[:, H:H + HKV], kw)):
        ok, err = bf_close(got, R.qk_norm_rope_fused(part, nw, cos[rp], sin[rp], 1e-6), ulps=4, atol=4e-2)
        assert ok, err
    # with the weights rounded to bf16 instead, some values move: the fp32 weights are used as given
    qb = ops.linear_qkv_rope(to_dev(x, BF), to_dev(wq, BF), to_dev(qw, BF), to_dev(kw, BF), to_dev(cos), to_dev(sin),
                             to_dev(pos), None, None, None, 1e-6, H, HKV, D, return_kv=True, rope_pos=to_dev(rpos))[0]
    assert not torch.equal(qb, q)
    qkv_d = ops.linear(to_dev(x, BF), to_dev(wq, BF))
    q2, k2, v2 = ops.qkv_rope_cache(qkv_d, to_dev(qw), to_dev(kw), to_dev(cos), to_dev(sin), to_dev(pos), None, None,
                                    None, 1e-6, H, HKV, D, return_kv=True, rope_pos=to_dev(rpos))
    assert torch.equal(v2, v)
    for a, b in ((q, q2), (k, k2)):
        d = (a.float() - b.float()).abs()
        assert (d > 0).float().mean() < 1e-3 and bf_close(a, b.float().cpu(), ulps=2, atol=2e-2)[0]


def test_linear_qkv_rope_no_norm_in_place():
    """The encoder's use: no QK-norm, rotary positions per row, q / k / v written back into the packed qkv rows."""
    g = gen(11)
    H, D, K, M = 8, 64, 512, 700
    x = R.bf(torch.randn(M, K, generator=g))
    wq = R.bf(torch.randn(3 * H * D, K, generator=g) / math.sqrt(K))
    cos, sin = R.rope_tables(D, 4096, 1e4)
    pos = (torch.arange(M) % 256).int()
    qkv = torch.empty(M, 3 * H * D, dtype=BF, device=DEV)
    ops.linear_qkv_rope(to_dev(x, BF), to_dev(wq, BF), None, None, to_dev(cos), to_dev(sin), to_dev(pos), None, None,
                        None, 1e-6, H, H, D, return_kv=True, q_out=qkv[:, :H * D],
                        kv_out=(qkv[:, H * D:2 * H * D], qkv[:, 2 * H * D:]))
    ref = R.linear_fused(x, wq).view(M, 3, H, D)
    rp = pos.long()
    want = torch.cat([R.bf(R.apply_rope(ref[:, 0], cos[rp], sin[rp])), R.bf(R.apply_rope(ref[:, 1], cos[rp], sin[rp])),
                      ref[:, 2]], 1).reshape(M, -1)
    ok, err = bf_close(qkv, want, ulps=2, atol=2e-2)
    assert ok, err


@pytest.mark.parametrize("M,N,K", [(1, 512, 512), (512, 512, 512), (77, 512, 1536), (512, 512, 1536),
                                   (1100, 512, 1536), (300, 100, 512), (40, 512, 576)])
def test_linear_residual(M, N, K):
    """32 x 32 tiles while they fit one round of the chip (up to 512 rows of N = 512), the panel kernel beyond
    (1100 rows) and for K % 128 != 0 (576), ragged N (100)."""
    g = gen(M * 7 + K)
    a = R.bf(torch.randn(M, K, generator=g))
    w = R.bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    x = R.bf(torch.randn(M, N, generator=g) * 2)
    xd = to_dev(x, BF)
    ops.linear_residual(to_dev(a, BF), to_dev(w, BF), xd)
    delta = R.bf((a.double() @ w.double().t()).float())
    want = R.bf(x + delta)
    # exact unless the GEMM output sits on a bf16 rounding boundary: then one ulp of delta, which is
    # many ulps of x + delta when the two cancel
    ok, err = bf_close(xd, want, ulps=1, atol=2e-2)
    assert ok, err


@pytest.mark.parametrize("M,K", [(1, 512), (77, 512), (512, 512), (512, 1536), (1024, 512), (1100, 1536), (64, 576)])
def test_linear_residual_row_sums(M, K):
    """ss_out: the per-32-column-block sums of squares of the updated rows, and x unchanged by asking -- from the
    32 x 32 tiles and from the panel kernel (1024 and 1100 rows, K = 576)."""
    g = gen(M * 3 + K)
    N = 512
    a = R.bf(torch.randn(M, K, generator=g))
    w = R.bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    x = R.bf(torch.randn(M, N, generator=g) * 2)
    xd, xd2 = to_dev(x, BF), to_dev(x, BF)
    ss = torch.full((M, N // 32), float("nan"), device=DEV)
    ops.linear_residual(to_dev(a, BF), to_dev(w, BF), xd, ss_out=ss)
    ops.linear_residual(to_dev(a, BF), to_dev(w, BF), xd2)
    assert torch.equal(xd, xd2)
    want = _row_ss(xd.float().cpu())
    assert torch.allclose(ss.cpu(), want, rtol=1e-5, atol=0), float((ss.cpu() - want).abs().max())


@pytest.mark.parametrize("M", [1, 100, 512, 1024])
@pytest.mark.parametrize("mode", ["swiglu", "bf16", "f32", "nonorm", "swiglu_ss", "bf16_ss", "f32_ss"])
def test_norm_linear(M, mode):
    """swiglu_ss: the 32 x 96 tiles up to one round of the chip (512 rows), the panel kernel at 1024 rows."""
    use_ss = mode.endswith("_ss")
    mode = mode.replace("_ss", "")
    g = gen(M + len(mode))
    K, Fd = 512, 1536
    x = R.bf(torch.randn(M, K, generator=g) * 3)
    nw = R.bf(torch.rand(K, generator=g) + 0.5)
    N = 2 * Fd if mode == "swiglu" else 768
    w = R.bf(torch.randn(N, K, generator=g) / math.sqrt(K))
    h = x if mode == "nonorm" else R.rmsnorm_fused(x, nw, 1e-6)
    out = ops.norm_linear(to_dev(x, BF), None if mode == "nonorm" else to_dev(nw, BF), 1e-6, to_dev(w, BF),
                          swiglu=mode == "swiglu", out_dtype=torch.float32 if mode == "f32" else None,
                          ss=to_dev(_row_ss(x)) if use_ss else None)
    y = (h.double() @ w.double().t()).float()
    if mode == "swiglu":
        ref = R.swiglu_fused(R.bf(y[:, :Fd]), R.bf(y[:, Fd:]))
        ok, err = bf_close(out, ref, ulps=4, atol=3e-3)
    elif mode == "f32":
        ok, err = torch.allclose(out.cpu(), y, rtol=1e-5, atol=2e-3), float((out.cpu() - y).abs().max())
    else:
        ok, err = bf_close(out, R.bf(y), ulps=1, atol=2e-3)
    # (atol: a one-ulp flip of one normalised element moves y by |w| ulp(h) ~ 4e-4)
    assert ok, err


def test_select_update_with_final_norm():
    g = gen(99)
    B, d, V = 64, 512, 7
    x = R.bf(torch.randn(B, d, generator=g) * 2)
    nw = R.bf(torch.rand(d, generator=g) + 0.5)
    w = R.bf(torch.randn(V, d, generator=g) / math.sqrt(d) * 3)
    bias = torch.zeros(V)
    bias[[R.PAD, R.BOS]] = float("-inf")
    tail = torch.zeros(V, dtype=torch.bool)
    homo = torch.zeros(V, dtype=torch.bool)
    h = R.rmsnorm_fused(x, nw, 1e-6)
    logits = (h.double() @ w.double().t()).float()
    tok = torch.full((B,), 3)
    run = torch.zeros(B, dtype=torch.long)
    want, _, margin = _select_ref(logits, tok, run, bias, tail, homo, 0, 0.0, torch.zeros(B))
    d_tok = to_dev(tok)
    pos = torch.full((B,), 10)
    out = torch.full((B, 4), R.PAD, dtype=torch.long, device=DEV)
    ops.select_update(to_dev(bias), to_dev(tail), to_dev(homo), 0, d_tok, to_dev(run), to_dev(pos),
                      to_dev(torch.full((B,), 9)), None, out, None, None, None, R.EOS, R.PAD,
                      h=to_dev(x, BF), norm_w=to_dev(nw, BF), eps=1e-6, w_head=to_dev(w, BF))
    got = d_tok.cpu()
    assert bool(((got == want) | (margin < 1e-2)).all())
    assert torch.equal(out[:, 1].cpu(), got)
