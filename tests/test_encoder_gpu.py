"""The HIP encoder (viktor_amd.encoder) against the encoder oracle (oracle/encoder.py), kernel by kernel and
end to end.

Tolerances: the kernels follow the oracle's "bf16" rounding points, so single ops agree to a few bf16 ulps
(accumulation order differs); the full encoder is compared with the oracle's bf16 mode (relative L2 error)
and with its fp32 mode by per-frame cosine similarity -- the reference's own criterion for its koi encoder
is a mean cosine above 0.95 against PyTorch (tests/gpu_check.py:106-107). A mixed batch must equal each
chunk encoded alone bit for bit (tests/gpu_check.py:103-105).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import encoder as E
from oracle.reference import apply_rope, bf, rope_tables
from viktor_amd import _lib
from viktor_amd._lib import HipLibraryError, call, ptr
from viktor_amd.encoder import DoradoEncoder

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _enc(depth, seed=0):
    cfg = E.with_depth(E.SUP_CFG, depth)
    params = E.encoder_params(cfg, seed=seed)
    enc = DoradoEncoder(cfg, DEV).load_state_dict(params)
    return cfg, params, enc


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


def test_gemm_rows_epilogues_and_row_determinism():
    g = torch.Generator().manual_seed(0)
    M, N, K = 700, 320, 512
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    st = _lib.stream_handle()
    want = x.double() @ w[:N].double().t()
    y32 = torch.empty(M, N, dtype=torch.float32, device=DEV)
    call("vk_gemm_rows", ptr(xd), ptr(wd), ptr(y32), M, N, K, 1, st)
    assert (y32.double().cpu() - want).abs().max() < 1e-3
    y16 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    call("vk_gemm_rows", ptr(xd), ptr(wd), ptr(y16), M, N, K, 0, st)
    assert torch.equal(y16.cpu(), y32.cpu().to(torch.bfloat16))
    sw = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    call("vk_gemm_rows", ptr(xd), ptr(wd), ptr(sw), M, N, K, 2, st)
    gt, up = bf(want[:, :N].float()), bf((x.double() @ w[N:].double().t()).float())
    ref = bf(bf(F.silu(gt)) * up)
    assert (sw.float().cpu() - ref).abs().max() <= 2 * 2 ** -8 * ref.abs().max()
    # the same rows inside a larger product give the same bits
    big = torch.cat([torch.randn(3000, K, generator=g).to(torch.bfloat16), x]).to(DEV)
    yb = torch.empty(big.shape[0], N, dtype=torch.float32, device=DEV)
    call("vk_gemm_rows", ptr(big), ptr(wd), ptr(yb), big.shape[0], N, K, 1, st)
    assert torch.equal(yb[3000:], y32)


def test_deepnorm_rmsnorm():
    g = torch.Generator().manual_seed(1)
    n = 37
    y = torch.randn(n, 512, generator=g)
    b = bf(0.1 * torch.randn(512, generator=g))
    x = torch.randn(n, 512, generator=g).to(torch.bfloat16)
    w = bf(1 + 0.1 * torch.randn(512, generator=g))
    alpha = 2.4494897
    xd, yd, bd, wd = x.to(DEV), y.to(DEV), b.to(DEV), w.to(DEV)  # held until the kernel has run
    call("vk_deepnorm_rmsnorm", ptr(yd), ptr(bd), ptr(xd), alpha, ptr(wd), 1e-5, n, 512, _lib.stream_handle())
    r = bf(bf(y + b) + bf(alpha * x.float()))
    want = r * torch.rsqrt((r * r).mean(-1, keepdim=True) + 1e-5) * w
    got = xd.float().cpu()
    assert (got - want).abs().max() <= 2 ** -7 * want.abs().max()
    assert (got - bf(want)).abs().gt(0).float().mean() < 0.01  # nearly every element equal after rounding


@pytest.mark.parametrize("T,window", [(1024, (127, 128)), (64, (127, 128)), (320, (0, 0)), (192, (3, 200)),
                                      (448, (300, 5)), (256, (1000, 1000))])
def test_window_attention_matches_oracle(T, window):
    g = torch.Generator().manual_seed(T + window[0])
    H = 8
    lens = [T, 128, T]
    rows = sum(lens)
    qkv = torch.randn(rows, 3 * H * 64, generator=g).to(torch.bfloat16)
    cos, sin = rope_tables(64, 4096, 10000.0)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    blocks = [(c, qs) for c, f in enumerate(lens) for qs in range(0, f, 128)]
    plan = torch.tensor(np.asarray(blocks, dtype=np.int32).reshape(-1))
    out = torch.empty(rows, H * 64, dtype=torch.bfloat16, device=DEV)
    dev = [t.to(DEV) for t in (qkv, cu, plan, cos, sin)]  # held until the kernel has run
    call("vk_window_attention", ptr(dev[0]), 3 * H * 64, ptr(dev[1]), ptr(dev[2]), len(blocks), len(lens), max(lens),
         H, 64, ptr(dev[3]), ptr(dev[4]), 4096, window[0], window[1], ptr(out), H * 64, _lib.stream_handle())
    torch.cuda.synchronize()
    got = out.float().cpu()
    for c in range(len(lens)):
        a, n = int(cu[c]), lens[c]
        x = qkv[a:a + n].float().view(n, 3, H, 64)
        q = bf(apply_rope(x[:, 0], cos[:n], sin[:n]))
        k = bf(apply_rope(x[:, 1], cos[:n], sin[:n]))
        want = E.band_attention(q.double(), k.double(), x[:, 2].double(), window).float().reshape(n, H * 64)
        err = (got[a:a + n] - want).abs().max().item()
        assert err < 2e-2, (c, err)


def test_conv_stack_matches_oracle():
    cfg, params, enc = _enc(0)
    ref = E.RefEncoder(cfg, params, "bf16")
    lens = [768, 2304, 12288, 768]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(2))
    got = enc.forward_varlen(sig.to(DEV), lens).float().cpu()
    want = ref.forward_varlen(sig, lens)
    assert got.shape == want.shape == (sum(lens) // 12, 512)
    # same rounding points; fp32 sums in another order flip a few last bits
    assert (got - want).abs().max() <= 4 * 2 ** -8 * max(1.0, want.abs().max().item())
    assert _rel(got, want) < 3e-3


def test_encoder_two_layers_matches_oracle():
    cfg, params, enc = _enc(2, seed=3)
    lens = [1536, 768, 3072]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(4))
    got = enc.forward_varlen(sig.to(DEV), lens).float().cpu()
    want16 = E.RefEncoder(cfg, params, "bf16").forward_varlen(sig, lens)
    want32 = E.RefEncoder(cfg, params, "fp32").forward_varlen(sig, lens)
    assert _rel(got, want16) < 1e-2
    cosim = F.cosine_similarity(got.double(), want32.double(), dim=1)
    assert cosim.min() > 0.995, float(cosim.min())


def test_encoder_full_depth_cosine():
    """18 layers (the SUP depth) on a full 12288-sample chunk and a short one."""
    cfg, params, enc = _enc(18, seed=5)
    lens = [12288, 1536]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(6))
    got = enc.forward_varlen(sig.to(DEV), lens).float().cpu()
    want = E.RefEncoder(cfg, params, "fp32").forward_varlen(sig, lens)
    cosim = F.cosine_similarity(got.double(), want.double(), dim=1)
    assert cosim.mean() > 0.99 and cosim.min() > 0.95, (float(cosim.mean()), float(cosim.min()))
    assert torch.isfinite(got).all()


def test_mixed_batch_equals_each_chunk_alone():
    cfg, params, enc = _enc(2, seed=7)
    lens = [12288, 768, 5376, 768, 12288]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(8)).to(DEV)
    packed = enc.forward_varlen(sig, lens)
    alone, off = [], 0
    for n in lens:
        alone.append(enc.forward_varlen(sig[off:off + n], [n]))
        off += n
    assert torch.equal(packed, torch.cat(alone))
    # forward([N, 1, T]) is forward_varlen over N equal chunks
    x = sig[:3 * 768].view(3, 1, 768)
    assert torch.equal(enc.forward(x), enc.forward_varlen(sig[:3 * 768], [768] * 3).view(3, 64, 512))


def test_encode_chunks_drops_padding_frames():
    cfg, params, enc = _enc(1, seed=9)
    lens, valid = [12288, 1536], [12288, 1000]
    sig = torch.randn(sum(lens), generator=torch.Generator().manual_seed(10)).to(DEV)
    packed = enc.forward_varlen(sig, lens)
    frames, flens = enc.encode_chunks(sig, lens, valid)
    assert flens == [1024, 84]  # ceil(1000 / 12)
    assert torch.equal(frames, torch.cat([packed[:1024], packed[1024:1024 + 84]]))


def test_unsupported_shapes_raise():
    with pytest.raises(HipLibraryError):
        DoradoEncoder(E.TINY_CFG, DEV)  # d_model 32
    cfg, params, enc = _enc(0)
    with pytest.raises(HipLibraryError):
        enc.forward_varlen(torch.zeros(100, device=DEV), [100])  # not a multiple of the stride


def test_basecaller_encode_windows():
    """Basecaller.encode (viktor/model.py:89-117): full windows whole, short windows at their padded length with
    ceil(valid / stride) frames kept and the rest zero -- each window equal to encoding it alone."""
    from viktor_amd.model import Basecaller
    from viktor_amd.tokenizer import KmerTokenizer
    cfg, params, enc = _enc(1, seed=11)
    model = Basecaller(enc, KmerTokenizer(1))
    S = 3072
    valid = [3072, 1000, 3072, 20]
    sig = torch.randn(len(valid), 1, S, generator=torch.Generator().manual_seed(12)).to(DEV)
    frames, plens = model.encode(sig, torch.tensor(valid))
    assert frames.shape == (4, S // 12, 512) and plens.tolist() == [256, 84, 256, 2]
    for b, v in enumerate(valid):
        n = S if v == S else -(-v // 768) * 768
        alone = enc.forward_varlen(sig[b, 0, :n].contiguous(), [n])
        k = int(plens[b])
        assert torch.equal(frames[b, :k], alone[:k])
        assert not frames[b, k:].any()
