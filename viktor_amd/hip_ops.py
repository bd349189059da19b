"""Decoder ops on the gfx950 HIP kernels (libviktor_hip.so), with the call signatures of the reference's
fused ops so FastDecoder / DecodeEngine code reads the same:

  add_rmsnorm, embed_rmsnorm, qkv_rope_cache, linear, swiglu, greedy_update   (viktor/triton_ops.py)
  decode_attention                                                              (viktor/decode_attention.py)
  varlen_attention  (flash_attn_varlen_func as used at viktor/fast_decoder.py:68-73)
  select_update     (LM head + DecodeEngine._select + step bookkeeping, viktor/engine.py:79-116)
  gspo_score, group_advantage  (scripts/gspo.py:340-353, 446-477)

Outputs are allocated with torch.empty on the input's device; documented in-place updates: x in
add_rmsnorm, the KV cache in qkv_rope_cache, the decode state in greedy_update / select_update.
Every launch goes to torch.cuda.current_stream(), so ops can be captured in a torch.cuda graph.
Preconditions are checked here and raise AssertionError as the reference's asserts do; a kernel
status other than OK raises HipLibraryError.
"""

import ctypes

import numpy as np

import torch

from . import _lib
from ._lib import VK_DTYPE_BF16, VK_DTYPE_F32, call, ptr, require_device, stream_handle

BF16 = torch.bfloat16


def _require(cond, msg):
    if not cond:
        raise AssertionError(msg)


def _contig(*ts):
    return all(t is None or t.is_contiguous() for t in ts)


def add_rmsnorm(x, w, eps, delta=None):
    """x [n, d] bf16 (updated in place by += delta); returns RMSNorm(x) * w [n, d] bf16.
    Reference: viktor/triton_ops.py:34-40."""
    require_device(x, "add_rmsnorm")
    _require(x.dim() == 2 and x.dtype == BF16 and w.dtype == BF16 and w.shape == (x.shape[1],), "add_rmsnorm: shapes")
    _require(delta is None or (delta.shape == x.shape and delta.dtype == BF16), "add_rmsnorm: delta shape")
    _require(_contig(x, w, delta), "add_rmsnorm: contiguous tensors")
    n, d = x.shape
    h = torch.empty_like(x)
    call("vk_add_rmsnorm", ptr(x), ptr(delta), ptr(w), ptr(h), n, d, float(eps), stream_handle())
    return h


def embed_rmsnorm(tok, emb, w, eps):
    """tok [n] int64 -> (x = emb[tok] [n, d], RMSNorm(x) * w). Reference: viktor/triton_ops.py:163-169."""
    require_device(emb, "embed_rmsnorm")
    _require(tok.dim() == 1 and tok.dtype == torch.long and emb.dim() == 2 and emb.dtype == BF16, "embed_rmsnorm: shapes")
    _require(_contig(tok, emb, w), "embed_rmsnorm: contiguous tensors")
    n, d = tok.shape[0], emb.shape[1]
    x = torch.empty(n, d, dtype=emb.dtype, device=emb.device)
    h = torch.empty_like(x)
    call("vk_embed_rmsnorm", ptr(tok), ptr(emb), emb.shape[0], ptr(w), ptr(x), ptr(h), n, d, float(eps),
         stream_handle())
    return x, h


def qkv_rope_cache(qkv, q_norm_w, k_norm_w, cos, sin, pos, seq, k_cache, v_cache, eps, n_heads, n_kv_heads,
                   head_dim, return_kv=False, rope_pos=None):
    """qkv [n, (H + 2 Hkv) D]; pos/seq [n] int32 cache position and cache row of each token; cos/sin
    [S, D/2] (fp32 or bf16); k_cache/v_cache [B, S, Hkv, D] (one layer, may be None when return_kv).
    rope_pos [n]: RoPE positions when they differ from pos. Returns q [n, H, D] (and packed k, v
    [n, Hkv, D] with return_kv). Reference: viktor/triton_ops.py:94-108."""
    require_device(qkv, "qkv_rope_cache")
    n = qkv.shape[0]
    _require(qkv.dtype == BF16 and qkv.shape[1] == (n_heads + 2 * n_kv_heads) * head_dim, "qkv_rope_cache: qkv shape")
    _require(pos.dtype == torch.int32 and pos.shape == (n,), "qkv_rope_cache: pos must be int32 [n]")
    _require(rope_pos is None or (rope_pos.dtype == torch.int32 and rope_pos.shape == (n,)), "qkv_rope_cache: rope_pos")
    _require(cos.shape == sin.shape and cos.dim() == 2 and cos.shape[1] == head_dim // 2 and cos.dtype == sin.dtype
             and cos.dtype in (torch.float32, BF16), "qkv_rope_cache: cos/sin tables")
    _require(_contig(qkv, q_norm_w, k_norm_w, cos, sin, pos, rope_pos), "qkv_rope_cache: contiguous tensors")
    if k_cache is not None:
        _require(seq is not None and seq.dtype == torch.int32 and seq.shape == (n,), "qkv_rope_cache: seq")
        _require(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride() and k_cache.dim() == 4
                 and k_cache.shape[2:] == (n_kv_heads, head_dim) and k_cache.stride(3) == 1
                 and k_cache.stride(2) == head_dim and k_cache.dtype == BF16, "qkv_rope_cache: cache layout")
    else:
        _require(return_kv, "qkv_rope_cache: nowhere to write k/v")
    q = torch.empty(n, n_heads, head_dim, dtype=qkv.dtype, device=qkv.device)
    k = v = None
    if return_kv:
        k = torch.empty(n, n_kv_heads, head_dim, dtype=qkv.dtype, device=qkv.device)
        v = torch.empty_like(k)
    tdt = VK_DTYPE_F32 if cos.dtype == torch.float32 else VK_DTYPE_BF16
    if k_cache is not None:
        sb, ss, rows, clen = k_cache.stride(0), k_cache.stride(1), k_cache.shape[0], k_cache.shape[1]
    else:
        sb = ss = rows = clen = 0
    _require(q_norm_w.dtype == k_norm_w.dtype and q_norm_w.dtype in (BF16, torch.float32), "qkv_rope_cache: norm weights")
    wdt = VK_DTYPE_F32 if q_norm_w.dtype == torch.float32 else VK_DTYPE_BF16
    call("vk_qkv_rope_cache", ptr(qkv), ptr(q_norm_w), ptr(k_norm_w), wdt, ptr(cos), ptr(sin), tdt, cos.shape[0], ptr(pos),
         ptr(rope_pos), ptr(seq), ptr(q), ptr(k_cache), ptr(v_cache), sb, ss, rows, clen, ptr(k), ptr(v), n,
         float(eps), n_heads, n_kv_heads, head_dim, stream_handle())
    return (q, k, v) if return_kv else q


def linear_qkv_rope(x, w, q_norm_w, k_norm_w, cos, sin, pos, seq, k_cache, v_cache, eps, n_heads, n_kv_heads,
                    head_dim, return_kv=False, rope_pos=None, q_out=None, kv_out=None, qkv_out=None):
    """The Wqkv product with qkv_rope_cache fused into its epilogue: x [n, K] @ w [(H + 2 Hkv) D, K]^T, then
    per-head QK-norm (q_norm_w / k_norm_w; both None: none) and RoPE at pos (or rope_pos) on the q and k heads,
    q to [n, H, D], k / v to the cache rows (seq, pos) and / or packed [n, Hkv, D] (return_kv). The rounding
    points of linear + qkv_rope_cache (viktor/triton_ops.py:43-108, 138-146). q_out / kv_out: caller's buffers
    (q_out [n, >= H D] rows; kv_out = (k, v) [n, >= Hkv D] rows, any row stride). fp32 norm weights (with fp32
    tables): the autocast forward's QK-norm with fp32 master weights (viktor/decoder.py:63-67 under autocast).
    qkv_out: a bf16 [n, (H + 2 Hkv) D] buffer that also receives the unrotated product (as linear(x, w) returns
    it), for the QK-norm + RoPE backward."""
    require_device(x, "linear_qkv_rope")
    n, K = x.shape
    H, HKV, D = n_heads, n_kv_heads, head_dim
    _require(x.dtype == w.dtype == BF16 and w.shape == ((H + 2 * HKV) * D, K) and _contig(x, w),
             "linear_qkv_rope: x / w")
    _require(cos.shape == sin.shape and cos.dim() == 2 and cos.shape[1] == D // 2 and cos.dtype == sin.dtype
             and cos.dtype in (torch.float32, BF16) and _contig(cos, sin), "linear_qkv_rope: cos/sin tables")
    for t in (pos, rope_pos, seq):
        _require(t is None or (t.dtype == torch.int32 and t.shape == (n,) and t.is_contiguous()),
                 "linear_qkv_rope: pos / rope_pos / seq int32 [n]")
    q = q_out if q_out is not None else torch.empty(n, H, D, dtype=BF16, device=x.device)
    _require(q.stride(-1) == 1, "linear_qkv_rope: q rows")
    k = v = None
    if return_kv:
        if kv_out is not None:
            k, v = kv_out
        else:
            k = torch.empty(n, HKV, D, dtype=BF16, device=x.device)
            v = torch.empty_like(k)
        _require(k.stride(0) == v.stride(0) and k.stride(-1) == 1 and v.stride(-1) == 1, "linear_qkv_rope: k / v rows")
    if k_cache is not None:
        _require(seq is not None and pos is not None and k_cache.shape == v_cache.shape and
                 k_cache.stride() == v_cache.stride() and k_cache.dim() == 4 and k_cache.shape[2:] == (HKV, D) and
                 k_cache.stride(3) == 1 and k_cache.stride(2) == D and k_cache.dtype == BF16,
                 "linear_qkv_rope: cache layout")
        sb, ss, rows, clen = k_cache.stride(0), k_cache.stride(1), k_cache.shape[0], k_cache.shape[1]
    else:
        _require(return_kv, "linear_qkv_rope: nowhere to write k/v")
        sb = ss = rows = clen = 0
    _require(qkv_out is None or (qkv_out.dtype == BF16 and qkv_out.shape == (n, (H + 2 * HKV) * D)
                                 and qkv_out.is_contiguous()), "linear_qkv_rope: qkv_out bf16 [n, (H + 2 Hkv) D]")
    tdt = VK_DTYPE_F32 if cos.dtype == torch.float32 else VK_DTYPE_BF16
    _require((q_norm_w is None) == (k_norm_w is None), "linear_qkv_rope: q and k norm weights go together")
    wdt = VK_DTYPE_BF16
    if q_norm_w is not None:
        _require(q_norm_w.dtype == k_norm_w.dtype and q_norm_w.dtype in (BF16, torch.float32) and q_norm_w.shape == (D,)
                 and k_norm_w.shape == (D,) and _contig(q_norm_w, k_norm_w), "linear_qkv_rope: norm weights [D]")
        wdt = VK_DTYPE_F32 if q_norm_w.dtype == torch.float32 else VK_DTYPE_BF16
        _require(wdt == VK_DTYPE_BF16 or tdt == VK_DTYPE_F32, "linear_qkv_rope: fp32 norm weights need fp32 tables")
    call("vk_linear_qkv_rope", ptr(x), ptr(w), n, K, ptr(q_norm_w), ptr(k_norm_w), wdt, float(eps), ptr(cos), ptr(sin), tdt,
         cos.shape[0], ptr(pos), ptr(rope_pos), ptr(seq), ptr(q), q.stride(0), ptr(k_cache), ptr(v_cache), sb, ss,
         rows, clen, ptr(k), ptr(v), 0 if k is None else k.stride(0), ptr(qkv_out), H, HKV, D, stream_handle())
    return (q, k, v) if return_kv else q


def linear_residual_big(a, w, x, bias=None, alpha=1.0, out=None):
    """Large-M residual product, in place. bf16 x: x = bf16(bf16(a @ w^T + bias) + bf16(alpha x)) (alpha 1, no
    bias: add_rmsnorm's x += delta, viktor/triton_ops.py:17-31; with the out_proj bias and the DeepNorm alpha:
    viktor/encoder.py:106-108). fp32 x: x = alpha x + bf16(a @ w^T + bias), the residual add of an fp32 stream and
    a bf16 product under torch.autocast (viktor/decoder.py:118-120). Returns the row sums of squares of the new x
    per 64-column block [M, N / 64] fp32, for rmsnorm_apply. out: the new stream goes there (same shape and dtype
    as x) and x is left as it was."""
    require_device(a, "linear_residual_big")
    M, K = a.shape
    N = w.shape[0]
    _require(a.dtype == w.dtype == BF16 and x.dtype in (BF16, torch.float32) and w.shape[1] == K and x.shape == (M, N)
             and _contig(a, w, x, bias), "linear_residual_big: shapes")
    _require(bias is None or (bias.dtype == torch.float32 and bias.shape == (N,)), "linear_residual_big: bias fp32 [N]")
    _require(out is None or (out.shape == x.shape and out.dtype == x.dtype and out.is_contiguous()
                             and out.data_ptr() != x.data_ptr()), "linear_residual_big: out buffer")
    ss = torch.empty(M, N // 64, dtype=torch.float32, device=a.device)
    xdt = VK_DTYPE_F32 if x.dtype == torch.float32 else VK_DTYPE_BF16
    dst, src = (x, None) if out is None else (out, x)
    call("vk_linear_residual_big", ptr(a), ptr(w), ptr(dst), xdt, M, N, K, ptr(bias), float(alpha), ptr(ss),
         ptr(src), stream_handle())
    return ss


def rmsnorm_apply(x, ss, w, eps, out=None):
    """h = bf16(x * rsqrt(sum(ss[row]) / d + eps) * w): the RMSNorm of x with its row sums of squares handed over
    in block partials (linear_residual_big). x and w bf16, or fp32 (the autocast forward's residual stream and
    master weights); h bf16. out may be x itself when x is bf16."""
    require_device(x, "rmsnorm_apply")
    n, d = x.shape
    _require(x.dtype in (BF16, torch.float32) and w.dtype in (BF16, torch.float32) and w.shape == (d,) and
             ss.dtype == torch.float32 and ss.shape[0] == n and _contig(x, ss, w), "rmsnorm_apply: shapes")
    h = out if out is not None else torch.empty(n, d, dtype=BF16, device=x.device)
    _require(h.dtype == BF16 and h.shape == (n, d) and h.is_contiguous(), "rmsnorm_apply: out bf16 [n, d]")
    xdt = VK_DTYPE_F32 if x.dtype == torch.float32 else VK_DTYPE_BF16
    wdt = VK_DTYPE_F32 if w.dtype == torch.float32 else VK_DTYPE_BF16
    call("vk_rmsnorm_apply_ss", ptr(x), xdt, ptr(ss), ss.shape[1], ptr(w), wdt, ptr(h), n, d, float(eps),
         stream_handle())
    return h


def rmsnorm_f32(x, w, eps, out=None):
    """h = bf16(x * rsqrt(mean(x^2) + eps) * w) of an fp32 stream x [n, d] with fp32 weights w [d]: nn.RMSNorm
    (fp32) cast to bf16 at the next product's autocast input (viktor/decoder.py:118 under torch.autocast)."""
    require_device(x, "rmsnorm_f32")
    n, d = x.shape
    _require(x.dtype == w.dtype == torch.float32 and w.shape == (d,) and _contig(x, w), "rmsnorm_f32: x, w fp32")
    h = out if out is not None else torch.empty(n, d, dtype=BF16, device=x.device)
    call("vk_rmsnorm_f32", ptr(x), ptr(w), ptr(h), n, d, float(eps), stream_handle())
    return h


def linear(x, w, swiglu=False, out_dtype=None, out=None, gu_out=None):
    """x [M, K] @ w[N, K]^T on bf16 MFMA. swiglu: w is gate_up [2F, K] and the result silu(gate) * up
    [M, F]; gu_out (swiglu only: a bf16 [M, 2F] buffer) also receives the gate | up product itself.
    out_dtype: torch.float32 for unrounded logits. Reference: viktor/triton_ops.py:138-146
    (also serves the F.linear calls of the prefill path)."""
    require_device(x, "linear")
    _require(x.dim() == 2 and w.dim() == 2 and x.shape[1] == w.shape[1], "linear: shapes")
    _require(x.dtype == BF16 and w.dtype == BF16, "linear: bf16 operands")
    _require(_contig(x, w), "linear: contiguous operands")
    M, K = x.shape
    N = w.shape[0] // 2 if swiglu else w.shape[0]
    _require(not swiglu or w.shape[0] % 2 == 0, "linear: swiglu needs gate_up [2F, K]")
    odt = out_dtype or x.dtype
    _require(odt in (BF16, torch.float32), "linear: out dtype")
    if out is None:
        out = torch.empty(M, N, dtype=odt, device=x.device)
    else:
        _require(out.shape == (M, N) and out.dtype == odt and out.is_contiguous(), "linear: out buffer")
    _require(gu_out is None or (swiglu and gu_out.dtype == BF16 and gu_out.shape == (M, 2 * N)
                                and gu_out.is_contiguous()), "linear: gu_out bf16 [M, 2F] with swiglu")
    call("vk_linear", ptr(x), ptr(w), ptr(out), M, N, K, int(bool(swiglu)),
         VK_DTYPE_F32 if odt == torch.float32 else VK_DTYPE_BF16, ptr(gu_out), stream_handle())
    return out


def group_rows_equal(x, group_size):
    """True when every member x[b] of the groups of group_size consecutive members equals its group's first
    member bit for bit (x contiguous [B, ...], B a multiple of group_size, x[b] a multiple of 16 bytes). One
    pass over x on the device, then one flag read back. No reference counterpart: the reference runs every
    repeated window (scripts/gspo.py:444)."""
    require_device(x, "group_rows_equal")
    G = int(group_size)
    B = x.shape[0]
    _require(G >= 1 and B % G == 0 and x.is_contiguous(), "group_rows_equal: contiguous [B, ...], B % G == 0")
    member_bytes = x[0].numel() * x.element_size() if B else 0
    _require(member_bytes % 16 == 0 and x.data_ptr() % 16 == 0, "group_rows_equal: 16-byte members")
    if B == 0 or G == 1:
        return True
    flag = torch.zeros(1, dtype=torch.int32, device=x.device)
    call("vk_group_rows_equal", ptr(x), B // G, G, member_bytes, ptr(flag), stream_handle())
    return int(flag.item()) == 0


def swiglu(gu):
    """gu [n, 2F] (gate | up) -> silu(gate) * up [n, F]. Reference: viktor/triton_ops.py:223-229."""
    require_device(gu, "swiglu")
    _require(gu.dim() == 2 and gu.shape[1] % 2 == 0 and gu.dtype == BF16 and gu.is_contiguous(), "swiglu: gu")
    n, f2 = gu.shape
    out = torch.empty(n, f2 // 2, dtype=gu.dtype, device=gu.device)
    call("vk_swiglu", ptr(gu), ptr(out), n, f2 // 2, stream_handle())
    return out


_ws_cache = {}


def decode_attention_workspace(B, H, max_len, device):
    """Scratch for the key-split partials of decode_attention (None when no split is needed)."""
    nbytes = ctypes.c_int64(0)
    _lib.check(_lib.load().vk_decode_attention_workspace(B, H, max_len, ctypes.byref(nbytes)), "decode_attention_workspace")
    if nbytes.value == 0:
        return None
    return torch.empty(nbytes.value, dtype=torch.uint8, device=device)


def decode_attention(q, k, v, lengths, block=64, workspace=None, rows=None):
    """q [B, H, D]; k/v [Bc, S, Hkv, D] (one layer of the cache); lengths [B] int32, including the current
    token, 1 <= lengths <= S. Sequence b attends to cache row rows[b] (rows [B] int32; None: row b, which
    needs Bc >= B). Only the valid prefix of each row is read. Returns [B, H, D] bf16.
    workspace: preallocated key-split scratch (needed inside graph capture; allocated here otherwise).
    Reference: viktor/decode_attention.py:41-53 (block is accepted for the signature); rows is the
    cache_batch_idx of flash_attn_with_kvcache at viktor/fast_decoder.py:86-89."""
    require_device(q, "decode_attention")
    B, H, D = q.shape
    HK = k.shape[2]
    _require(q.is_contiguous() and H % HK == 0 and H // HK <= 16 and D == 64, "decode_attention: q layout")
    _require(q.dtype == k.dtype == v.dtype == BF16, "decode_attention: bf16 tensors")
    _require(k.shape == v.shape and k.dim() == 4, "decode_attention: k / v shapes")
    _require(k.stride() == v.stride() and k.stride(-1) == 1 and k.stride(-2) == D, "decode_attention: cache layout")
    _require(lengths.shape == (B,) and lengths.dtype == torch.int32 and lengths.is_contiguous(),
             "decode_attention: lengths")
    if rows is None:
        _require(k.shape[0] >= B, f"decode_attention: {B} queries but the cache holds {k.shape[0]} sequences")
    else:
        _require(rows.shape == (B,) and rows.dtype == torch.int32 and rows.is_contiguous(), "decode_attention: rows")
    S = k.shape[1]
    if workspace is None:
        key = (B, H, S, q.device)
        workspace = _ws_cache.get(key)
        if workspace is None and key not in _ws_cache:
            workspace = decode_attention_workspace(B, H, S, q.device)
            _ws_cache[key] = workspace
    out = torch.empty_like(q)
    wsz = 0 if workspace is None else workspace.numel() * workspace.element_size()
    call("vk_decode_attention", ptr(q), ptr(k), ptr(v), ptr(lengths), ptr(rows), k.shape[0], ptr(out), B, H, HK, D,
         k.stride(0), k.stride(1),
         S, ptr(workspace), wsz, stream_handle())
    return out


def decode_attention_grouped_workspace(B, G, pre_max, suf_max, device):
    nbytes = ctypes.c_int64(0)
    _lib.check(_lib.load().vk_decode_attention_grouped_workspace(B, G, pre_max, suf_max, ctypes.byref(nbytes)),
               "decode_attention_grouped_workspace")
    return torch.empty(nbytes.value, dtype=torch.uint8, device=device)


def decode_attention_grouped_layout(B, G, pre_max, suf_max):
    """(query members per workgroup, parts per subgroup) of decode_attention_grouped at these sizes: G or G / 2
    (groups split by member), and 1 part (one launch) or more (a merge launch follows)."""
    m, n = ctypes.c_int32(0), ctypes.c_int32(0)
    _lib.check(_lib.load().vk_decode_attention_grouped_layout(B, G, pre_max, suf_max, ctypes.byref(m), ctypes.byref(n)),
               "decode_attention_grouped_layout")
    return m.value, n.value


def decode_attention_grouped(q, k_prefix, v_prefix, prefix_len, k_suffix, v_suffix, suffix_len, group_size,
                             workspace=None):
    """Decode attention of B = P * G sequences whose groups of G consecutive rows share a prefix: sequence b
    attends to prefix rows [0, prefix_len[b // G]) of k/v_prefix [P, S_pre, 2, 64] then to its own rows
    [0, suffix_len[b]) of k/v_suffix [B, S_suf, 2, 64]. Returns [B, 8, 64] bf16 (each prefix row is read once
    per group)."""
    require_device(q, "decode_attention_grouped")
    B, H, D = q.shape
    G = int(group_size)
    _require(q.is_contiguous() and q.dtype == BF16 and H == 8 and D == 64, "decode_attention_grouped: q")
    _require(B % G == 0 and k_prefix.shape[0] == B // G and k_suffix.shape[0] == B, "decode_attention_grouped: batch")
    for a, b in ((k_prefix, v_prefix), (k_suffix, v_suffix)):
        _require(a.stride() == b.stride() and a.stride(-1) == 1 and a.stride(-2) == D and a.dtype == b.dtype == BF16,
                 "decode_attention_grouped: cache layout")
    _require(prefix_len.dtype == torch.int32 and prefix_len.shape == (B // G,) and suffix_len.dtype == torch.int32
             and suffix_len.shape == (B,), "decode_attention_grouped: lengths int32")
    if workspace is None:
        workspace = decode_attention_grouped_workspace(B, G, k_prefix.shape[1], k_suffix.shape[1], q.device)
    out = torch.empty_like(q)
    call("vk_decode_attention_grouped", ptr(q), ptr(k_prefix), ptr(v_prefix), ptr(prefix_len), k_prefix.stride(0),
         k_prefix.stride(1), k_prefix.shape[1], ptr(k_suffix), ptr(v_suffix), ptr(suffix_len), k_suffix.stride(0),
         k_suffix.stride(1), k_suffix.shape[1], ptr(out), B, G, H, k_prefix.shape[2], D, ptr(workspace),
         workspace.numel(), stream_handle())
    return out


class AttentionPlan:
    """Host-built work list of vk_varlen_attention: one (sequence, first query row) entry per 64-query
    block, ordered by decreasing key count so the longest blocks start first. Device tensors."""

    BLOCK = 64

    def __init__(self, q_lens, k_lens, k_off, device, causal=True, p_lens=None, p_off=None):
        """p_lens / p_off (prefixed key ranges, vk_varlen_attention_prefixed): sequence i's first p_lens[i] of its
        k_lens[i] keys are rows of a prefix buffer from element p_off[i]; the rest are its k_off rows."""
        import numpy as np
        q = np.asarray([int(a) for a in q_lens], dtype=np.int64)
        k = np.asarray([int(a) for a in k_lens], dtype=np.int64)
        _require(len(q) == len(k) == len(k_off), "AttentionPlan: length mismatch")
        _require(bool(((q >= 0) & (k >= 0) & ((k >= q) | (not causal))).all()),
                 "AttentionPlan: causal needs k_len >= q_len")
        # blocks (sequence i, first query qs) for qs = 0, 64, .. < q_len, in sequence order, then stably sorted by
        # decreasing key count (ties keep that order)
        nb = (q + self.BLOCK - 1) // self.BLOCK
        seq = np.repeat(np.arange(len(q), dtype=np.int64), nb)
        qs = (np.arange(int(nb.sum()), dtype=np.int64) - np.repeat(np.cumsum(nb) - nb, nb)) * self.BLOCK
        work = np.minimum(k[seq], k[seq] - q[seq] + qs + self.BLOCK) if causal else k[seq]
        order = np.argsort(-work, kind="stable")
        cu = np.concatenate([[0], np.cumsum(q)]).astype(np.int64)
        self.n_seq = len(q)
        self.n_blocks = len(order)
        self.total_q = int(cu[-1])
        self.causal = causal
        flat = np.stack([seq[order], qs[order]], 1).reshape(-1) if len(order) else np.zeros(2, dtype=np.int64)
        self.plan = torch.from_numpy(flat.astype(np.int32)).to(device)
        self.cu_q = torch.from_numpy(cu.astype(np.int32)).to(device)
        self.k_lens = torch.from_numpy((k if len(k) else np.zeros(1, np.int64)).astype(np.int32)).to(device)
        self.k_off = torch.tensor([int(o) for o in k_off] or [0], dtype=torch.int64).to(device)
        self.p_lens = self.p_off = None
        if p_lens is not None:
            pl = np.asarray([int(a) for a in p_lens], dtype=np.int64)
            _require(len(pl) == len(q) == len(p_off) and bool(((pl >= 0) & (pl <= k)).all()),
                     "AttentionPlan: prefix lengths within the key counts")
            self.p_lens = torch.from_numpy((pl if len(pl) else np.zeros(1, np.int64)).astype(np.int32)).to(device)
            self.p_off = torch.tensor([int(o) for o in p_off] or [0], dtype=torch.int64).to(device)


def varlen_attention(q, k, v, plan: AttentionPlan, stride_tok=None, out=None, lse=None, prefix=None):
    """Packed-query GQA attention following `plan`. q [total_q, H, D] bf16; k/v: base tensors (packed
    [n, Hkv, D] rows or one cache layer [B, S, Hkv, D]) addressed by plan.k_off + key * stride_tok
    elements. Returns [total_q, H, D] bf16. lse [total_q, H] fp32 (optional, written): each row's
    log-sum-exp of its scaled scores in log2 units, for attention_backward.
    prefix = (k_prefix, v_prefix) with a plan built with p_lens / p_off: each sequence's first p_lens keys are rows
    of those tensors (p_off + key * their row stride), the rest rows of k / v (vk_varlen_attention_prefixed).
    Reference: flash_attn_varlen_func at viktor/fast_decoder.py:68-73."""
    require_device(q, "varlen_attention")
    total, H, D = q.shape
    HK = k.shape[-2]
    _require(total == plan.total_q and q.dtype == k.dtype == v.dtype == BF16, "varlen_attention: q shape / dtype")
    _require(q.is_contiguous() and k.stride(-1) == 1 and k.stride(-2) == D and k.stride() == v.stride(),
             "varlen_attention: layouts")
    if stride_tok is None:
        stride_tok = k.stride(-3)
    if out is None:
        out = torch.empty_like(q)
    _require(lse is None or (lse.dtype == torch.float32 and lse.shape == (total, H) and lse.is_contiguous()),
             "varlen_attention: lse [total_q, H] fp32")
    _require((prefix is None) == (plan.p_lens is None), "varlen_attention: prefix tensors go with a prefixed plan")
    if prefix is None:
        call("vk_varlen_attention", ptr(q), ptr(k), ptr(v), ptr(plan.cu_q), ptr(plan.k_off), ptr(plan.k_lens),
             ptr(plan.plan), plan.n_blocks, plan.n_seq, stride_tok, ptr(out), int(plan.causal), H, HK, D, ptr(lse),
             stream_handle())
        return out
    kp, vp = prefix
    _require(kp.dtype == vp.dtype == BF16 and kp.shape[-2:] == (HK, D) and kp.stride(-1) == 1 and kp.stride(-2) == D
             and kp.stride() == vp.stride(), "varlen_attention: prefix layouts")
    call("vk_varlen_attention_prefixed", ptr(q), ptr(k), ptr(v), ptr(plan.cu_q), ptr(plan.k_off), ptr(plan.k_lens),
         ptr(plan.plan), plan.n_blocks, plan.n_seq, stride_tok, ptr(kp), ptr(vp), ptr(plan.p_off), ptr(plan.p_lens),
         kp.stride(-3), ptr(out), int(plan.causal), H, HK, D, ptr(lse), stream_handle())
    return out


def select_update(bias, is_tail, is_homo, homo_stop, tok, run, pos, plen, rope_off, out, pos32, seqlens, rpos32, eos,
                  pad, logits=None, h=None, w_head=None, round_bf16=False, temperature=0.0, uniforms=None,
                  logp_out=None, norm_w=None, eps=1e-6, cache_base=None, gumbel=False):
    """One step's token choice + state update for every sequence (fused LM head when h, w_head are given;
    with norm_w, h is the residual stream and the final RMSNorm runs first). See vk_select_update in
    include/viktor_hip.h for the exact rule order. logp_out: [B] fp32 (this step's chosen-token log-prob), or
    [B, >= out columns] fp32, where the log-prob goes to the output column the token is written to.
    gumbel: sampled steps take the reference's Gumbel-max choice (viktor/engine.py:80-83) from uniforms
    [B, T, V] (one per vocabulary entry) instead of the inverse CDF at uniforms [B, T]."""
    ref = logits if logits is not None else h
    require_device(ref, "select_update")
    B = tok.shape[0]
    V = bias.shape[0]
    if logits is not None:
        _require(logits.shape == (B, V) and logits.dtype == torch.float32 and logits.is_contiguous(), "select_update: logits")
        d = 0
    else:
        _require(h.dim() == 2 and h.shape[0] == B and w_head.shape == (V, h.shape[1]) and h.dtype == BF16
                 and w_head.dtype == BF16 and _contig(h, w_head), "select_update: h / w_head")
        d = h.shape[1]
    for t, dt in ((tok, torch.long), (pos, torch.long), (run, torch.long), (plen, torch.long), (rope_off, torch.long),
                  (cache_base, torch.long),
                  (pos32, torch.int32), (seqlens, torch.int32), (rpos32, torch.int32)):
        _require(t is None or (t.dtype == dt and t.shape == (B,) and t.is_contiguous()), "select_update: state tensors")
    _require(out.dim() == 2 and out.shape[0] == B and out.dtype == torch.long and out.stride(1) == 1, "select_update: out")
    _require(is_tail.dtype in (torch.bool, torch.uint8) and is_homo.dtype in (torch.bool, torch.uint8), "select_update: masks")
    if temperature > 0 and gumbel:
        _require(uniforms is not None and uniforms.dtype == torch.float32 and uniforms.dim() == 3
                 and uniforms.shape[0] == B and uniforms.shape[2] == V and uniforms.stride(2) == 1
                 and uniforms.stride(1) == V, "select_update: Gumbel uniforms [B, T, V] fp32")
    elif temperature > 0:
        _require(uniforms is not None and uniforms.dtype == torch.float32 and uniforms.dim() == 2
                 and uniforms.shape[0] == B and uniforms.stride(1) == 1, "select_update: uniforms [B, T] fp32")
    us, uc = (uniforms.stride(0), uniforms.shape[1]) if uniforms is not None else (0, 0)
    _require(norm_w is None or (norm_w.shape == (d,) and norm_w.dtype == BF16), "select_update: norm_w")
    lp_stride = 0
    if logp_out is not None:
        _require(logp_out.dtype == torch.float32 and logp_out.shape[0] == B and logp_out.dim() in (1, 2)
                 and logp_out.stride(-1) == 1, "select_update: logp_out [B] or [B, T] fp32")
        if logp_out.dim() == 2:
            _require(logp_out.shape[1] >= out.shape[1], "select_update: logp_out columns")
            lp_stride = logp_out.stride(0)
    call("vk_select_update", ptr(logits), ptr(h), ptr(norm_w), float(eps), ptr(w_head), d, int(bool(round_bf16)),
         ptr(bias), ptr(is_tail),
         ptr(is_homo), int(homo_stop), float(temperature), ptr(uniforms), us, uc, int(bool(gumbel)), ptr(tok), ptr(run), ptr(pos), ptr(plen),
         ptr(rope_off), ptr(cache_base), ptr(out), out.stride(0), out.shape[1], ptr(pos32), ptr(seqlens), ptr(rpos32), ptr(logp_out), lp_stride, B, V,
         int(eos), int(pad), stream_handle())


def norm_qkv_rope_cache(x, norm_w, eps, w_qkv, q_norm_w, k_norm_w, cos, sin, pos, seq, k_cache, v_cache, n_heads,
                        n_kv_heads, head_dim, rope_pos=None, tok=None, x_store=None, ss=None):
    """Decode-step fusion: h = RMSNorm(x) * norm_w (or, with tok, x = emb[tok] where `x` is the embedding
    table, stored into x_store; norm_w None: h = x), qkv = h @ w_qkv^T, then QK-norm + RoPE + KV-cache write
    as qkv_rope_cache. Returns q [M, H, D]. Same rounding points as add_rmsnorm + linear + qkv_rope_cache.
    ss: the [M, K / 32] fp32 row sums of squares linear_residual(ss_out=...) left for x (K = 512)."""
    require_device(x, "norm_qkv_rope_cache")
    M = tok.shape[0] if tok is not None else x.shape[0]
    K = x.shape[1]
    _require(x.dtype == BF16 and w_qkv.dtype == BF16 and w_qkv.shape == ((n_heads + 2 * n_kv_heads) * head_dim, K),
             "norm_qkv_rope_cache: shapes")
    _require(tok is None or (tok.dtype == torch.long and x_store is not None and x_store.shape == (M, K)
                             and norm_w is not None),
             "norm_qkv_rope_cache: embedding gather needs tok int64, x_store [M, K] and norm_w")
    _require(pos.dtype == torch.int32 and seq.dtype == torch.int32 and pos.shape == (M,) and seq.shape == (M,),
             "norm_qkv_rope_cache: pos / seq int32 [M]")
    _require(rope_pos is None or (rope_pos.dtype == torch.int32 and rope_pos.shape == (M,)), "norm_qkv_rope_cache: rope_pos")
    _require(cos.dtype == sin.dtype and cos.dtype in (torch.float32, BF16) and cos.shape[1] == head_dim // 2,
             "norm_qkv_rope_cache: tables")
    _require(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride() and k_cache.stride(3) == 1
             and k_cache.stride(2) == head_dim, "norm_qkv_rope_cache: cache layout")
    _require(_contig(x, norm_w, w_qkv, q_norm_w, k_norm_w, cos, sin, pos, seq, rope_pos, tok, x_store, ss),
             "norm_qkv_rope_cache: contiguous tensors")
    _require(ss is None or (ss.dtype == torch.float32 and ss.shape == (M, K // 32)), "norm_qkv_rope_cache: ss [M, K/32]")
    q = torch.empty(M, n_heads, head_dim, dtype=BF16, device=x.device)
    call("vk_norm_qkv_rope_cache", ptr(x), ptr(tok), x.shape[0] if tok is not None else 0, ptr(x_store), ptr(norm_w),
         float(eps), ptr(w_qkv), ptr(q_norm_w), ptr(k_norm_w), ptr(cos), ptr(sin),
         VK_DTYPE_F32 if cos.dtype == torch.float32 else VK_DTYPE_BF16, cos.shape[0], ptr(pos), ptr(rope_pos), ptr(seq),
         ptr(q), ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.shape[0], k_cache.shape[1], M,
         K, n_heads, n_kv_heads, head_dim, ptr(ss), stream_handle())
    return q


def linear_residual(a, w, x, ss_out=None):
    """x += a @ w^T in place (bf16 GEMM output added to the bf16 residual, rounded as linear + add_rmsnorm).
    ss_out [M, N / 32] fp32 (N = 512): per-row partial sums of squares of the updated x (one per 32 columns),
    for the next norm."""
    require_device(a, "linear_residual")
    M, K = a.shape
    _require(a.dtype == w.dtype == x.dtype == BF16 and w.shape[1] == K and x.shape == (M, w.shape[0]),
             "linear_residual: shapes")
    _require(_contig(a, w, x, ss_out), "linear_residual: contiguous tensors")
    _require(ss_out is None or (ss_out.dtype == torch.float32 and ss_out.shape == (M, w.shape[0] // 32)),
             "linear_residual: ss_out [M, N/32] fp32")
    call("vk_linear_residual", ptr(a), ptr(w), ptr(x), M, w.shape[0], K, ptr(ss_out), stream_handle())
    return x


def norm_linear(x, norm_w, eps, w, swiglu=False, out_dtype=None, ss=None):
    """act(RMSNorm(x) * norm_w @ w^T) for small M (norm_w None: no norm); act = SwiGLU over [gate; up].
    ss: the [M, K / 32] fp32 row sums of squares linear_residual(ss_out=...) left for x (K = 512)."""
    require_device(x, "norm_linear")
    M, K = x.shape
    _require(x.dtype == w.dtype == BF16 and w.shape[1] == K, "norm_linear: shapes")
    _require(_contig(x, norm_w, w, ss), "norm_linear: contiguous tensors")
    _require(ss is None or (ss.dtype == torch.float32 and ss.shape == (M, K // 32)), "norm_linear: ss [M, K/32]")
    N = w.shape[0] // 2 if swiglu else w.shape[0]
    odt = out_dtype or BF16
    y = torch.empty(M, N, dtype=odt, device=x.device)
    call("vk_norm_linear", ptr(x), ptr(norm_w), float(eps), ptr(w), ptr(y), M, N, K, int(bool(swiglu)),
         VK_DTYPE_F32 if odt == torch.float32 else VK_DTYPE_BF16, ptr(ss), stream_handle())
    return y


def greedy_update(logits, bias, is_tail, is_homo, homo_stop, tok, run, pos, plen, rope_off, out, pos32, seqlens,
                  rpos32, eos, pad):
    """One greedy step's bookkeeping from fp32 logits [B, V] (reference: viktor/triton_ops.py:200-209)."""
    select_update(bias, is_tail, is_homo, homo_stop, tok, run, pos, plen, rope_off, out, pos32, seqlens, rpos32, eos,
                  pad, logits=logits)


def gspo_score(logits, targets, mask=None, old_lp=None, n_bases=None, adv=None, eps_lo=4e-4, eps_hi=4e-4, inv_n=None,
               grad=True):
    """Per-token log pi of the targets and, with old_lp / n_bases / adv, the GSPO sequence ratio, the
    clipped objective and dL/dlogits.

    logits [B, T, V] bf16 or fp32; targets [B, T] int64 (PAD-clamped to 0 as the reference gathers);
    mask [B, T] bool. Returns dict(lp [B, T], and with the ratio inputs: s [B], pg [B], loss [] and
    dlogits [B, T, V] fp32 when grad). inv_n defaults to 1 / B (loss = mean over the B sequences)."""
    require_device(logits, "gspo_score")
    _require(logits.dim() == 3 and logits.dtype in (BF16, torch.float32) and logits.is_contiguous(), "gspo_score: logits")
    B, T, V = logits.shape
    _require(targets.shape == (B, T) and targets.dtype == torch.long and targets.is_contiguous(), "gspo_score: targets")
    dev = logits.device
    lp = torch.empty(B, T, dtype=torch.float32, device=dev)
    res = {"lp": lp}
    ratio = old_lp is not None
    s = pg = loss = dl = None
    m8 = None
    if ratio:
        _require(mask is not None and adv is not None and n_bases is not None, "gspo_score: ratio needs mask, n_bases, adv")
        _require(old_lp.shape == (B, T) and old_lp.dtype == torch.float32 and old_lp.is_contiguous(), "gspo_score: old_lp")
        _require(mask.shape == (B, T), "gspo_score: mask")
        _require(n_bases.shape == (B,) and adv.shape == (B,), "gspo_score: n_bases / adv")
        m8 = mask.to(torch.uint8).contiguous()
        n_bases = n_bases.to(torch.float32).contiguous()
        adv = adv.to(torch.float32).contiguous()
        s = torch.empty(B, dtype=torch.float32, device=dev)
        pg = torch.empty_like(s)
        loss = torch.empty((), dtype=torch.float32, device=dev)
        if grad:
            dl = torch.empty(B, T, V, dtype=torch.float32, device=dev)
        res.update(s=s, pg=pg, loss=loss)
        if grad:
            res["dlogits"] = dl
    inv = float(1.0 / B if inv_n is None else inv_n) if B else 0.0
    call("vk_gspo_score", ptr(logits), VK_DTYPE_BF16 if logits.dtype == BF16 else VK_DTYPE_F32, ptr(targets), ptr(m8),
         ptr(old_lp), ptr(n_bases), ptr(adv), float(eps_lo), float(eps_hi), inv, ptr(lp), ptr(s), ptr(pg), ptr(loss),
         ptr(dl), B, T, V, stream_handle())
    return res


def group_advantage(reward, std_floor=None, eps=None):
    """Group-normalised advantages of reward [G, n] fp32: (r - mean) / max(std, std_floor) (the reference's
    rule, scripts/gspo.py:447-450) or (r - mean) / (std + eps). Returns (adv [G, n], live [G] bool)."""
    require_device(reward, "group_advantage")
    _require((std_floor is None) != (eps is None), "group_advantage: give std_floor or eps")
    r = reward.to(torch.float32).contiguous()
    G, n = r.shape
    adv = torch.empty_like(r)
    live = torch.empty(G, dtype=torch.uint8, device=r.device)
    mode, param = (0, std_floor) if std_floor is not None else (1, eps)
    call("vk_group_advantage", ptr(r), G, n, mode, float(param), ptr(adv), ptr(live), stream_handle())
    return adv, live.bool()


# ---- the GSPO update's backward and optimizer step -------------------------------------------------------
class KeyBlockPlan:
    """(sequence, first key) per 128-key block of causal self-attention over packed sequences, longest work
    (most query rows at or below the block) first: the dK / dV work list of attention_backward."""

    BLOCK = 128

    def __init__(self, seq_lens, device, extra=None, chunk=None):
        """extra (the shared-prefix layout of vk_attention_backward_prefixed): per sequence, a list of (first
        packed row, rows) query segments that see every key of the sequence (their samples' token rows against a
        shared prefix). Such a sequence's key blocks get work items for its own rows, in chunks of at most `chunk`
        rows (default: the longest segment), in partial slots 0, 1, .., and one item per segment in the slots
        after the largest own-chunk count; the slots are summed in order. Those sequences come first in the
        packing and carry the same number of segments."""
        lens = [int(n) for n in seq_lens]
        self.n_slots, self.n_part = 0, 0
        self.part = None
        if extra is None:
            blocks = sorted(((n - ks, i, ks) for i, n in enumerate(lens) for ks in range(0, n, self.BLOCK)),
                            key=lambda b: -b[0])
            flat = [v for _, i, ks in blocks for v in (i, ks)] or [0, 0]
        else:
            _require(len(extra) == len(lens), "KeyBlockPlan: one segment list per sequence")
            segs = [list(e or []) for e in extra]
            with_x = [i for i, e in enumerate(segs) if e]
            cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
            n_own = 0
            if with_x:
                _require(with_x == list(range(len(with_x))) and len({len(segs[i]) for i in with_x}) == 1,
                         "KeyBlockPlan: sequences with segments first, each with the same number")
                C = int(chunk) if chunk else max(int(xn) for i in with_x for _, xn in segs[i])
                C = max(C, 32)
                n_own = max(-(-lens[i] // C) for i in with_x)
                self.n_slots = n_own + len(segs[0])
                self.n_part = int(cu[len(with_x)])
            items = []
            for i, n in enumerate(lens):
                for ks in range(0, n, self.BLOCK):
                    if segs[i]:
                        for c, r in enumerate(range(ks, n, C)):
                            items.append((min(C, n - r), i, ks, r, -min(C, n - r), c))
                        items += [(int(xn), i, ks, int(x0), int(xn), n_own + j) for j, (x0, xn) in enumerate(segs[i])]
                    else:
                        items.append((n - ks, i, ks, ks, -(n - ks), -1))
            items.sort(key=lambda b: -b[0])
            flat = [v for it in items for v in it[1:]] or [0, 0, 0, -1, -1]
            blocks = items
        self.n_blocks = len(blocks)
        self.prefixed = extra is not None
        self.plan = torch.tensor(flat, dtype=torch.int32).to(device)

    def partials(self, hkv, d, device):
        """The plan's partial-slot workspace (k, v) [n_slots, n_part, hkv, d] fp32, zeroed once: every call with
        this plan writes the same (slot, row) entries, so the ones no item writes stay zero."""
        if self.part is None:
            k = torch.zeros(self.n_slots, self.n_part, hkv, d, dtype=torch.float32, device=device)
            self.part = (k, torch.zeros_like(k))
        return self.part


def attention_backward(q, k, v, out, dout, lse, q_plan: AttentionPlan, k_plan: KeyBlockPlan, stride_tok=None):
    """Gradients of causal GQA self-attention over the packed sequences of q_plan (q_lens == k_lens, keys of
    sequence i at rows cu[i].. of k / v). q / out / dout [n, 8, 64] bf16, k / v [n, 2, 64] (row stride
    stride_tok), lse [n, 8] from varlen_attention(..., lse=). Returns dq [n, 8, 64], dk, dv [n, 2, 64] fp32.
    Shared-prefix layout (q_plan with p_lens / p_off, k_plan with extra segments): sequence i's queries first see
    p_lens[i] prefix keys (rows of k / v from element p_off[i]) and its key blocks also collect the gradients of
    its extra query segments (vk_attention_backward_prefixed).
    Reference: the backward of flash_attn_func(causal=True) at viktor/decoder.py:82-87."""
    require_device(q, "attention_backward")
    n, H, D = q.shape
    HK = k.shape[-2]
    _require(q.dtype == k.dtype == v.dtype == out.dtype == dout.dtype == BF16, "attention_backward: bf16 tensors")
    _require(_contig(q, out, dout, lse) and k.stride(-1) == 1 and k.stride(-2) == D and k.stride() == v.stride(),
             "attention_backward: layouts")
    _require(q_plan.total_q == n and out.shape == q.shape == dout.shape and lse.shape == (n, H)
             and lse.dtype == torch.float32, "attention_backward: shapes")
    if stride_tok is None:
        stride_tok = k.stride(-3)
    dd = torch.empty(n, H, dtype=torch.float32, device=q.device)
    dq = torch.empty(n, H, D, dtype=torch.float32, device=q.device)
    dk = torch.empty(n, HK, D, dtype=torch.float32, device=q.device)
    dv = torch.empty_like(dk)
    prefixed = q_plan.p_lens is not None or k_plan.prefixed
    if not prefixed:
        call("vk_attention_backward", ptr(q), ptr(k), ptr(v), ptr(out), ptr(dout), ptr(lse), ptr(q_plan.cu_q),
             q_plan.n_seq, ptr(q_plan.plan), q_plan.n_blocks, ptr(k_plan.plan), k_plan.n_blocks, n, stride_tok,
             ptr(dd), ptr(dq), ptr(dk), ptr(dv), H, HK, D, stream_handle())
        return dq, dk, dv
    _require(q_plan.p_lens is not None and k_plan.prefixed,
             "attention_backward: a shared-prefix layout needs both plans' prefix fields")
    part_k = part_v = None
    if k_plan.n_slots:
        part_k, part_v = k_plan.partials(HK, D, q.device)
    call("vk_attention_backward_prefixed", ptr(q), ptr(k), ptr(v), ptr(out), ptr(dout), ptr(lse), ptr(q_plan.cu_q),
         q_plan.n_seq, ptr(q_plan.plan), q_plan.n_blocks, ptr(k_plan.plan), k_plan.n_blocks, n, stride_tok,
         ptr(q_plan.p_lens), ptr(q_plan.p_off), ptr(part_k), ptr(part_v), k_plan.n_part, k_plan.n_slots, ptr(dd),
         ptr(dq), ptr(dk), ptr(dv), H, HK, D, stream_handle())
    return dq, dk, dv


_wgrad_ws = {}


def wgrad(a, b, out_dtype=BF16):
    """Weight gradient a^T b [Ka, Kb] over the rows of a [N, Ka] and b [N, Kb] (bf16, unit column stride):
    fp32 accumulation in row slices summed in a fixed order, rounded to bf16 once (or fp32). Ka % 256 == 0,
    Kb % 128 == 0. The workspace is cached per (N, Ka, Kb, device)."""
    require_device(a, "wgrad")
    _require(a.dim() == 2 and b.dim() == 2 and a.shape[0] == b.shape[0] and a.dtype == b.dtype == BF16,
             "wgrad: a [N, Ka], b [N, Kb] bf16")
    _require(a.stride(1) == 1 and b.stride(1) == 1, "wgrad: unit column stride")
    N, Ka = a.shape
    Kb = b.shape[1]
    key = (N, Ka, Kb, a.device)
    ws = _wgrad_ws.get(key)
    if ws is None:
        n = ctypes.c_int64(0)
        call("vk_wgrad_workspace", N, Ka, Kb, ctypes.byref(n))
        ws = torch.empty(max(int(n.value), 16), dtype=torch.uint8, device=a.device)
        if len(_wgrad_ws) >= 8:  # a backward uses a handful of shapes; keep the cache bounded
            _wgrad_ws.clear()
        _wgrad_ws[key] = ws
    out = torch.empty(Ka, Kb, dtype=out_dtype, device=a.device)
    call("vk_wgrad", ptr(a), a.stride(0), ptr(b), b.stride(0), N, Ka, Kb, ptr(out),
         VK_DTYPE_BF16 if out_dtype == BF16 else VK_DTYPE_F32, ptr(ws), ws.numel(), stream_handle())
    return out


def bias_act(y, bias, gelu):
    """Projector linear epilogue: y [n, d] fp32 (the product), bias [d] fp32 -> gelu False: bf16(y + b);
    gelu True: (pre, out) = (bf16(y + b), bf16(gelu(pre))), the exact erf GELU. Reference: viktor/model.py:35
    (nn.Linear, nn.GELU() under torch.autocast bf16)."""
    require_device(y, "bias_act")
    _require(y.dim() == 2 and y.dtype == torch.float32 and bias.dtype == torch.float32 and bias.shape == (y.shape[1],)
             and _contig(y, bias), "bias_act: y [n, d] fp32, bias [d] fp32, contiguous")
    n, d = y.shape
    out = torch.empty(n, d, dtype=BF16, device=y.device)
    pre = torch.empty(n, d, dtype=BF16, device=y.device) if gelu else None
    call("vk_bias_act", ptr(y), ptr(bias), ptr(pre), ptr(out), n, d, int(bool(gelu)), stream_handle())
    return (pre, out) if gelu else out


def act_backward(dout, pre=None):
    """Projector backward rows: dout [n, d] bf16. With pre (the GELU input, bf16 [n, d]): returns (din bf16 =
    dout gelu'(pre), bias gradient fp32 [d] = column sums of din); without: the column sums of dout (fp32 [d]).
    Column sums in a fixed order."""
    require_device(dout, "act_backward")
    _require(dout.dim() == 2 and dout.dtype == BF16 and _contig(dout, pre)
             and (pre is None or (pre.shape == dout.shape and pre.dtype == BF16)), "act_backward: shapes")
    n, d = dout.shape
    b = ctypes.c_int32(0)
    call("vk_act_backward_blocks", n, d, ctypes.byref(b))
    part = torch.empty(b.value, d, dtype=torch.float32, device=dout.device)
    din = torch.empty_like(dout) if pre is not None else None
    call("vk_act_backward", ptr(pre), ptr(dout), ptr(din), ptr(part), b.value, n, d, int(pre is not None),
         stream_handle())
    return (din, colsum(part)) if pre is not None else colsum(part)


def embed_grad(d_rows, tokens, vocab):
    """Token-embedding gradient: fp32 [vocab, d] with row v = the sum of d_rows[r] (bf16 or fp32 [n, d], unit
    column stride) over tokens[r] == v (int64 [n]), summed in a fixed order. Reference: the backward of
    nn.Embedding, viktor/decoder.py:127, as viktor/model.py:77 gathers it."""
    require_device(d_rows, "embed_grad")
    _require(d_rows.dim() == 2 and d_rows.dtype in (BF16, torch.float32) and d_rows.stride(1) == 1,
             "embed_grad: d_rows [n, d] bf16 or fp32")
    _require(tokens.shape == (d_rows.shape[0],) and tokens.dtype == torch.long and tokens.is_contiguous(),
             "embed_grad: tokens [n] int64")
    n, d = d_rows.shape
    nb = ctypes.c_int64(0)
    call("vk_embed_grad_workspace", n, vocab, d, ctypes.byref(nb))
    ws = torch.empty(max(int(nb.value) // 4, 4), dtype=torch.float32, device=d_rows.device)
    out = torch.empty(vocab, d, dtype=torch.float32, device=d_rows.device)
    ddt = VK_DTYPE_F32 if d_rows.dtype == torch.float32 else VK_DTYPE_BF16
    call("vk_embed_grad", ptr(d_rows), ddt, d_rows.stride(0), ptr(tokens), n, vocab, d, ptr(out), ptr(ws),
         4 * ws.numel(), stream_handle())
    return out


def _norm_blocks(n):
    b = ctypes.c_int32(0)
    _lib.check(_lib.load().vk_rmsnorm_backward_blocks(n, ctypes.byref(b)), "rmsnorm_backward_blocks")
    return b.value


def colsum(part, out=None, accumulate=False):
    """Column sums of part [rows, cols] fp32 in a fixed order (into out [cols], added when accumulate)."""
    rows, cols = part.shape
    if out is None:
        out = torch.empty(cols, dtype=torch.float32, device=part.device)
    _require(part.is_contiguous() and part.dtype == torch.float32 and out.shape == (cols,)
             and out.dtype == torch.float32, "colsum: shapes")
    call("vk_colsum", ptr(part), ptr(out), rows, cols, int(bool(accumulate)), stream_handle())
    return out


def rmsnorm_backward(x, w, dy, eps, dres=None, dx=None, dx_bf16=None):
    """Backward of h = rmsnorm(x) * w (x [n, 512] and w [512] both bf16 or both fp32, dy [n, 512] bf16 or fp32):
    returns (dx fp32 [n, 512] = the norm's input gradient + dres, dw fp32 [512]). dx may be dres (in place).
    dx_bf16 (a bf16 [n, 512] buffer): also receives dx.to(bfloat16), written by the same kernel.
    Reference: nn.RMSNorm of the decoder blocks, viktor/decoder.py:110-124."""
    require_device(x, "rmsnorm_backward")
    n, d = x.shape
    _require(x.dtype == w.dtype and x.dtype in (BF16, torch.float32) and dy.shape == x.shape
             and dy.dtype in (BF16, torch.float32), "rmsnorm_backward: dtypes")
    _require(_contig(x, w, dy, dres) and (dres is None or (dres.dtype == torch.float32 and dres.shape == x.shape)),
             "rmsnorm_backward: layouts")
    _require(dx_bf16 is None or (dx_bf16.dtype == BF16 and dx_bf16.shape == x.shape and dx_bf16.is_contiguous()),
             "rmsnorm_backward: dx_bf16 bf16 [n, d]")
    if dx is None:
        dx = dres if dres is not None else torch.empty(n, d, dtype=torch.float32, device=x.device)
    part = torch.empty(_norm_blocks(n), d, dtype=torch.float32, device=x.device)
    xdt = VK_DTYPE_F32 if x.dtype == torch.float32 else VK_DTYPE_BF16
    call("vk_rmsnorm_backward", ptr(x), xdt, ptr(w), xdt, ptr(dy),
         VK_DTYPE_F32 if dy.dtype == torch.float32 else VK_DTYPE_BF16, ptr(dres), ptr(dx), ptr(dx_bf16), ptr(part), n,
         d, float(eps), stream_handle())
    return dx, colsum(part)


def qknorm_rope_backward(qkv, q_norm_w, k_norm_w, cos, sin, rope_pos, dq, dk, dv, eps, n_heads, n_kv_heads, head_dim):
    """Backward of the QK-norm + RoPE stage: qkv [n, (H + 2 Hkv) D] bf16 (projection output), dq / dk / dv fp32
    attention-input gradients, rope_pos [n] int32 rows of cos/sin [S, D/2]. Returns (dqkv bf16 [n, (H + 2 Hkv) D],
    d q_norm.weight fp32 [D], d k_norm.weight fp32 [D]). Reference: viktor/decoder.py:62-66."""
    require_device(qkv, "qknorm_rope_backward")
    n = qkv.shape[0]
    _require(qkv.dtype == BF16 and qkv.shape[1] == (n_heads + 2 * n_kv_heads) * head_dim, "qknorm_rope_backward: qkv")
    _require(dq.shape == (n, n_heads, head_dim) and dk.shape == dv.shape == (n, n_kv_heads, head_dim)
             and dq.dtype == dk.dtype == dv.dtype == torch.float32, "qknorm_rope_backward: gradients")
    _require(rope_pos.dtype == torch.int32 and rope_pos.shape == (n,), "qknorm_rope_backward: rope_pos")
    _require(_contig(qkv, q_norm_w, k_norm_w, cos, sin, rope_pos, dq, dk, dv), "qknorm_rope_backward: layouts")
    _require(q_norm_w.dtype == k_norm_w.dtype and q_norm_w.dtype in (BF16, torch.float32),
             "qknorm_rope_backward: norm weights bf16 or fp32")
    wdt = VK_DTYPE_F32 if q_norm_w.dtype == torch.float32 else VK_DTYPE_BF16
    dqkv = torch.empty_like(qkv)
    part = torch.empty(_norm_blocks(n), 2 * head_dim, dtype=torch.float32, device=qkv.device)
    tdt = VK_DTYPE_F32 if cos.dtype == torch.float32 else VK_DTYPE_BF16
    call("vk_qknorm_rope_backward", ptr(qkv), ptr(q_norm_w), ptr(k_norm_w), wdt, ptr(cos), ptr(sin), tdt, cos.shape[0],
         ptr(rope_pos), ptr(dq), ptr(dk), ptr(dv), ptr(dqkv), ptr(part), n, n_heads, n_kv_heads, head_dim, float(eps),
         stream_handle())
    dw = colsum(part)
    return dqkv, dw[:head_dim], dw[head_dim:]


def swiglu_backward(gu, dout):
    """gu [n, 2F] (gate | up) bf16, dout [n, F] bf16 -> d gu [n, 2F] bf16 of silu(gate) * up.
    Reference: F.silu(gate) * up at viktor/decoder.py:127."""
    require_device(gu, "swiglu_backward")
    n, F2 = gu.shape
    _require(gu.dtype == dout.dtype == BF16 and dout.shape == (n, F2 // 2) and _contig(gu, dout),
             "swiglu_backward: shapes")
    dgu = torch.empty_like(gu)
    call("vk_swiglu_backward", ptr(gu), ptr(dout), ptr(dgu), n, F2 // 2, stream_handle())
    return dgu


def grad_norm_clip(g, max_norm, n_partials=512):
    """[||g||_2, min(1, max_norm / (||g|| + 1e-6))] of the flat fp32 gradient g, on the device
    (nn.utils.clip_grad_norm_, scripts/gspo.py:492)."""
    require_device(g, "grad_norm_clip")
    _require(g.dtype == torch.float32 and g.is_contiguous() and g.dim() == 1, "grad_norm_clip: flat fp32 gradient")
    part = torch.empty(n_partials, dtype=torch.float32, device=g.device)
    out = torch.empty(2, dtype=torch.float32, device=g.device)
    call("vk_grad_norm_clip", ptr(g), g.numel(), float(max_norm), ptr(part), n_partials, ptr(out), stream_handle())
    return out


def adamw(p, g, m, v, lr, betas, eps, weight_decay, step, coef=None):
    """One AdamW step over flat fp32 p / g / m / v (torch.optim.AdamW, scripts/gspo.py:368), the gradient
    scaled by coef[1] when given (grad_norm_clip's clip coefficient)."""
    require_device(p, "adamw")
    _require(all(t.dtype == torch.float32 and t.is_contiguous() and t.shape == p.shape for t in (p, g, m, v)),
             "adamw: flat fp32 buffers of one shape")
    call("vk_adamw", ptr(p), ptr(g), ptr(m), ptr(v), p.numel(), ptr(coef), float(lr), float(betas[0]), float(betas[1]),
         float(eps), float(weight_decay), int(step), stream_handle())
