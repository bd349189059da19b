"""The C-ABI boundary on the CPU: the library exists, loads, exports every entry point the header
declares, and the product path fails loudly without a ROCm device (no compute calls here)."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

from viktor_amd import _lib, hip_ops
from viktor_amd.synthetic import make_model

from .conftest import ROOT

HEADER = os.path.join(ROOT, "include", "viktor_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(vk_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_table():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "run python -m viktor_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (vk_\w+)", out))
    missing = set(declared_symbols()) - exported
    assert not missing, missing


def test_library_loads_and_reports_version():
    lib = _lib.load()
    assert lib.vk_version() >= 100
    assert isinstance(lib.vk_last_error(), bytes)


def test_argument_errors_return_status_without_device_work():
    """Invalid arguments are rejected on the host before any launch (null pointers / bad sizes)."""
    lib = _lib.load()
    rc = lib.vk_linear(None, None, None, 4, 8, 32, 0, 0, None, None)
    assert rc == 1 and b"null" in lib.vk_last_error()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    rc = lib.vk_linear(p, p, p, 4, 8, 30, 0, 0, None, None)  # K % 32 != 0
    assert rc == 1 and b"K" in lib.vk_last_error()
    rc = lib.vk_decode_attention(p, p, p, p, None, 4, p, 4, 8, 2, 128, 128, 128, 16, None, 0, None)  # head_dim 128
    assert rc == 3
    # a cache of 2 sequence rows cannot serve 4 queries without a row map
    rc = lib.vk_decode_attention(p, p, p, p, None, 2, p, 4, 8, 2, 64, 3072 * 128, 128, 3072, None, 0, None)
    assert rc == 1 and b"cache holds 2 rows" in lib.vk_last_error()
    # logp_stride below the output columns would overlap rows
    rc = lib.vk_select_update(p, None, None, 1e-6, None, 0, 0, p, p, p, 0, 0.0, None, 0, 0, 0, p, None, p, None,
                              None, None, p, 16, 16, None, None, None, p, 8, 4, 7, 2, 0, None)
    assert rc == 1 and b"logp_stride" in lib.vk_last_error()
    # Gumbel uniforms whose row stride cannot hold u_cols x V entries
    rc = lib.vk_select_update(p, None, None, 1e-6, None, 0, 0, p, p, p, 0, 1.0, p, 16, 16, 1, p, None, p, None,
                              None, None, p, 16, 16, None, None, None, None, 0, 8, 7, 2, 0, None)
    assert rc == 1 and b"Gumbel" in lib.vk_last_error()
    rc = lib.vk_linear_residual_big(p, p, p, 0, 4, 96, 64, None, 1.0, p, None, None)  # N % 128 != 0
    assert rc == 1 and b"N" in lib.vk_last_error()
    rc = lib.vk_linear_residual_big(p, p, p, 0, 4, 128, 64, None, 1.0, None, None, None)  # no sums-of-squares output
    assert rc == 1 and b"null" in lib.vk_last_error()
    rc = lib.vk_linear_residual_big(p, p, p, 7, 4, 128, 64, None, 1.0, p, None, None)  # residual dtype
    assert rc == 1 and b"dtype" in lib.vk_last_error()
    rc = lib.vk_rmsnorm_apply_ss(p, 0, p, 8, p, 0, p, 4, 12, 1e-6, None)  # d % 8 != 0
    assert rc == 1 and b"d=12" in lib.vk_last_error()
    rc = lib.vk_rmsnorm_apply_ss(p, 1, p, 8, p, 1, p, 4, 512, 1e-6, None)  # fp32 x written over by bf16 h
    assert rc == 1 and b"fp32 x" in lib.vk_last_error()
    rc = lib.vk_rmsnorm_f32(p, p, p, 4, 4096, 1e-6, None)  # d above 2048
    assert rc == 1 and b"d=4096" in lib.vk_last_error()
    # fp32 QK-norm weights with bf16 rotary tables
    rc = lib.vk_linear_qkv_rope(p, p, 4, 512, p, p, 1, 1e-6, p, p, 0, 16, p, None, None, p, 512, None, None, 0, 0, 0,
                                0, p, p, 128, None, 8, 2, 64, None)
    assert rc == 1 and b"fp32 rotary tables" in lib.vk_last_error()
    rc = lib.vk_rmsnorm_backward(p, 1, p, 0, p, 0, None, p, None, p, 4, 512, 1e-6, None)  # fp32 x with bf16 weights
    assert rc == 3
    rc = lib.vk_timestamp(None, 0, None)
    assert rc == 1 and b"null" in lib.vk_last_error()
    rc = lib.vk_timestamp(p, -1, None)
    assert rc == 1 and b"negative" in lib.vk_last_error()
    with pytest.raises(_lib.HipLibraryError):
        _lib.check(rc, "decode_attention")


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    w = torch.ones(512, dtype=torch.bfloat16)
    with pytest.raises(_lib.HipLibraryError):
        hip_ops.add_rmsnorm(x, w, 1e-6)
    with pytest.raises(_lib.HipLibraryError):
        hip_ops.linear(x, torch.zeros(64, 512, dtype=torch.bfloat16))


def test_product_has_no_cpu_fallback():
    from viktor_amd import DecodeEngine
    m = make_model(1, n_layers=1)
    with pytest.raises(_lib.HipLibraryError):
        m.decoder(torch.zeros(1, 4, 512))
    with pytest.raises(_lib.HipLibraryError):
        DecodeEngine(m, 2, 4, 8)


def test_unknown_backends_raise_value_error():
    """viktor/fast_decoder.py:29-30 and the engine's backend argument: only the HIP kernels exist here
    ('auto' / 'hip'; 'triton' is accepted as the reference's other in-tree name), anything else is a
    ValueError before any device work."""
    from viktor_amd import DecodeEngine
    from viktor_amd.fast_decoder import FastDecoder
    m = make_model(1, n_layers=1)
    for name in ("flash", "torch", ""):
        with pytest.raises(ValueError, match="backend"):
            FastDecoder(m.decoder, attention_backend=name)
    with pytest.raises(ValueError, match="backend"):
        DecodeEngine(m, 2, 4, 8, backend="torch")
    assert FastDecoder(m.decoder, attention_backend="triton").attention_backend == "hip"


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.HipLibraryError):
        _lib.load.__wrapped__ if hasattr(_lib.load, "__wrapped__") else None
        saved = _lib._lib
        try:
            _lib._lib = None
            _lib.load(str(tmp_path / "absent.so"))
        finally:
            _lib._lib = saved


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "viktor_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in re.sub(r"#.*", "", text).split("import") or "import oracle" not in text, f
                assert "from oracle" not in text and "import oracle" not in text, f


def test_attention_plan_orders_longest_first():
    plan = hip_ops.AttentionPlan([130, 64, 1], [130, 200, 1], [0, 0, 0], "cpu", causal=True)
    flat = plan.plan.tolist()
    pairs = list(zip(flat[::2], flat[1::2]))
    # blocks: seq0 at 0, 64, 128; seq1 at 0; seq2 at 0 -- work = keys visible to the block's last query
    assert pairs[0] in ((1, 0),) and sorted(pairs) == [(0, 0), (0, 64), (0, 128), (1, 0), (2, 0)]
    assert plan.total_q == 195 and plan.cu_q.tolist() == [0, 130, 194, 195]
    with pytest.raises(AssertionError):
        hip_ops.AttentionPlan([5], [4], [0], "cpu", causal=True)


def test_kv_cache_pad_rows_layout():
    """KVCache(pad_rows=p): k / v are [L, B, max_len, Hkv, D] views whose sequence stride is (max_len + p) rows
    (what the kernels take as the cache's sequence stride); the pad rows are never part of the view."""
    from viktor_amd.decoder import DecoderConfig, KVCache
    cfg = DecoderConfig(vocab_size=7, n_layers=2)
    c = KVCache(cfg, 3, 10, torch.bfloat16, "cpu", pad_rows=5)
    row = cfg.n_kv_heads * cfg.head_dim
    assert c.k.shape == c.v.shape == (2, 3, 10, cfg.n_kv_heads, cfg.head_dim) and c.max_len == 10
    assert c.k.stride() == c.v.stride() == (3 * 15 * row, 15 * row, row, cfg.head_dim, 1)
    c.k.fill_(1)
    base = c.k.as_strided((2 * 3 * 15 * row,), (1,))  # the padded storage behind the view
    assert float(base.sum()) == 2 * 3 * 10 * row
    assert float(base.view(2, 3, 15, row)[:, :, 10:].abs().sum()) == 0
    assert KVCache(cfg, 3, 10, torch.bfloat16, "cpu").k.is_contiguous()


def test_batch_weights_map_bases_to_tokens():
    """Basecaller.batch with per-base weights (the GSPO update's SFT term): a k-mer token weighs its lowest
    base weight, a partial tail token its lowest real base, EOS 1, padding 0 (viktor/model.py:133-145)."""
    m = make_model(4, n_layers=1)
    seqs = ["ACGTACGTAC", "ACG"]
    weights = [[1, 1, 0, 1, 1, 1, 1, 1, 0.5, 1], [1, 0.2, 1]]
    tokens_in, targets, w = m.batch(seqs, weights)
    assert w.shape == targets.shape
    assert w[0, :4].tolist() == [0.0, 1.0, 0.5, 1.0] and float(w[0, 4:].sum()) == 0.0
    assert abs(float(w[1, 0]) - 0.2) < 1e-7 and float(w[1, 1]) == 1.0
    _, _, w_none = m.batch(seqs)
    assert torch.equal(w_none, (targets != 0).float())


def test_key_block_plan_covers_every_key_once():
    plan = hip_ops.KeyBlockPlan([1, 128, 129, 300], "cpu")
    blocks = plan.plan.view(-1, 2).tolist()
    assert plan.n_blocks == 1 + 1 + 2 + 3
    assert sorted(blocks) == sorted([[0, 0], [1, 0], [2, 0], [2, 128], [3, 0], [3, 128], [3, 256]])
    work = [[1, 128, 129, 300][s] - k for s, k in blocks]
    assert work == sorted(work, reverse=True)  # longest work (most rows at or below the block) first


def _attention_plan_loops(q_lens, k_lens, causal, block=64):
    """The work list as nested loops: (work, sequence, first query) per 64-query block, sorted stably by
    decreasing work."""
    blocks = []
    for i, (ql, kl) in enumerate(zip(q_lens, k_lens)):
        for qs in range(0, ql, block):
            blocks.append((min(kl, kl - ql + qs + block) if causal else kl, i, qs))
    blocks.sort(key=lambda b: -b[0])
    return [v for _, i, qs in blocks for v in (i, qs)] or [0, 0]


def test_attention_and_prefill_plans_match_loop_forms():
    """The host-built plans (vectorised) against their loop forms: block order, offsets, kept-row indices."""
    import random
    from viktor_amd.fast_decoder import PrefillPlan
    from viktor_amd.hip_ops import AttentionPlan
    rng = random.Random(3)
    for trial in range(20):
        n = rng.randint(1, 40)
        k_lens = [rng.choice([1, 63, 64, 65, 128, rng.randint(1, 3000)]) for _ in range(n)]
        causal = trial % 3 != 0
        q_lens = [rng.randint(0, kl) if causal else rng.randint(0, 300) for kl in k_lens]
        plan = AttentionPlan(q_lens, k_lens, [7 * i for i in range(n)], "cpu", causal=causal)
        assert plan.plan.tolist() == _attention_plan_loops(q_lens, k_lens, causal)
        assert plan.cu_q.tolist() == [sum(q_lens[:j]) for j in range(n + 1)]
        assert plan.k_lens.tolist() == k_lens and plan.n_blocks == sum((q + 63) // 64 for q in q_lens)
        seq = [max(1, kl) for kl in k_lens]
        keep = [rng.randint(1, s) for s in seq]
        pp = PrefillPlan(seq, "cpu", keep=keep)
        cu = pp.cu
        assert pp.last_idx.tolist() == [cu[j + 1] - kk + i for j, kk in enumerate(keep) for i in range(kk)]
