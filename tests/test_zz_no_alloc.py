"""vk_decode_attention_noalloc through the C ABI: the same output, bit for bit, as vk_decode_attention with a
caller workspace, on two calls in a row -- the second with a smaller batch -- both taking the key-split
path whose partials live in the library's static scratch array."""

import ctypes

import pytest
import torch

from viktor_amd import _lib, hip_ops as ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _workspace_bytes(B, S):
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().vk_decode_attention_workspace(B, 8, S, ctypes.byref(n)), "workspace query")
    return n.value


def _noalloc(q, k, v, lengths, rows=None):
    out = torch.empty_like(q)
    B, S = q.shape[0], k.shape[1]
    rc = _lib.load().vk_decode_attention_noalloc(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(lengths), _lib.ptr(rows), k.shape[0], _lib.ptr(out), B, 8, 2,
        64, k.stride(0), k.stride(1), S, _lib.stream_handle())
    _lib.check(rc, "vk_decode_attention_noalloc")
    return out


@pytest.mark.parametrize("use_rows", [False, True])
def test_noalloc_matches_workspace_entry_point(use_rows):
    torch.manual_seed(91 + int(use_rows))
    for B, S in ((96, 3073), (20, 1500)):  # two calls in a row, the second smaller
        assert _workspace_bytes(B, S) > 0  # both split the key range: the static scratch is used
        Bc = B + 2
        k = torch.randn(Bc, S, 2, 64, device=DEV).to(torch.bfloat16)
        v = torch.randn(Bc, S, 2, 64, device=DEV).to(torch.bfloat16)
        q = torch.randn(B, 8, 64, device=DEV).to(torch.bfloat16)
        lens = torch.randint(1, S + 1, (B,), device=DEV, dtype=torch.int32)
        lens[0], lens[1] = 1, S
        rows = torch.randperm(Bc, device=DEV)[:B].int() if use_rows else None
        want = ops.decode_attention(q, k, v, lens, rows=rows)
        got = _noalloc(q, k, v, lens, rows)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (B, S, float((got.float() - want.float()).abs().max()))


def test_noalloc_rejects_bad_arguments_on_the_host():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    rc = lib.vk_decode_attention_noalloc(p, p, p, p, None, 2, p, 4, 8, 2, 64, 3072 * 128, 128, 3072, None)
    assert rc == 1 and b"cache holds 2 rows" in lib.vk_last_error()
    rc = lib.vk_decode_attention_noalloc(p, p, p, p, None, 4, p, 4, 8, 2, 128, 3072 * 128, 128, 3072, None)
    assert rc == 3
