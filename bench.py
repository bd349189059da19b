"""GSPO rollout throughput on one MI355X: 64 prefixes x group 8 = 512 sequences, 2048-frame prefixes,
1024 sampled tokens each (temperature 1.0, supplied uniforms), 8-layer d512 decoder, vocab 7.

One step = one full rollout: prefill of the prefixes (projector + 8 layers, BOS-only last layer) + 1023
graph-replayed decode steps, with the frames already resident in HBM. value = 512 * 1024 tokens per
rollout / seconds per rollout. The engine receives all 512 sequences' frames, as the rollout hands them
over; with --group-size 8 (default) it checks that each group of 8 shares its window, prefills each window
once and keeps one prefix KV copy per group (--group-size 1: every sequence prefilled and cached on its own).

Extra objects on the JSON line:
  roofline      decode attention, the dominant kernel: algorithmic bytes per call (every K/V byte the call
                must read once -- the shared prefix once per group, each sequence's own rows -- plus q and
                out) / its average duration inside the captured decode step: device timestamp nodes captured
                right before and after each layer's attention launch (less the dispatch gap a back-to-back pair
                of them measures), read at 32 evenly spaced steps of a rollout. Also
                kept: eager_* (HIP events over eager calls at the same lengths, rotating over the 8 layers'
                caches so no call finds its bytes in the Infinity Cache) and warm_* (back to back on one layer);
                traffic = measured HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by a copy
                kernel; read from profiles/decode_attention_traffic.json when present, else null).
  cpu_baseline  the CPU oracle (the reference's fp32 torch path restated) on this host's usable cores: the
                CPU-plumbing configuration at full size (4 sequences x 2048-frame prefix x 64 greedy tokens,
                8 layers, seed 0); tokens/s, with the host's CPU count, affinity, quota and model.
  decode_roofline_ms / decode_hbm_frac  the rollout's decode against its own HBM roofline: every attended K/V
                position once per step (the shared prefix once per group), the new positions written, the
                weights read once per step, at 8 TB/s.
  configs       the other configurations, each against its own roofline: the rollout without prefix sharing
                (every sequence prefilled and cached alone, as the reference does), varlen prefill + 4-mer
                decode (1024 sequences, 340 tokens, vocab 343), scoring (512 x (2048 + 700..1024) forward +
                loss + dL/dlogits) and the 4096-sequence stress decode (51.5 GB of KV cache).
  prefill       the rollout's prefill (projector + 8 layers with a BOS-only last layer, once per window
                when the prefix KV is shared): algorithmic flops (projector, 2 x weights per row less what the
                BOS-only last layer skips, causal attention 1024 n (n + 1) per layer and window, the LM head of
                the BOS row) / prefill_ms, against 2.5 PFLOP/s bf16.
  gspo_reward   a rollout's 512 rewards on the device (strict identity, scripts/gspo.py:446) straight from the
                output tokens: 64 synthetic 0.9-1.1 kb labels (5% of bases unscored), each window's 8 calls the
                label with 5% substitutions / insertions / deletions, as token rows of 1024 (EOS after the
                call); ms per rollout (device token decode + label packing + the DP kernel) and DP cells per
                second (label x call bases). (The random-weight model of the rollout ends its calls after a
                few bases, so its own output would time an almost empty DP.)
  gspo_update   one micro-batch of the GSPO update (scripts/gspo.py:471-493 with --micro 32): 32 calls = 4
                windows x 8 calls of 2048 frames + 768 tokens (the 1024-token rollout's calls padded to a
                multiple of 128), teacher-forced forward + backward of the sequence-ratio loss into the fp32
                projector and decoder weights + clip + AdamW step, with each window's prefix run once for its
                calls (and timed again unshared, every call's full window); ms per micro-batch and the MFMA
                fraction of its algorithmic flops (GEMMs 3 x 2 x weights per row, causal attention 3.5 x the
                forward's per layer: forward + the standard 2.5 x backward) against 2.5 PFLOP/s bf16.
  encoder       the frames producer for one rollout's windows: 128 chunks of 12288 samples (64 windows x 2048
                frames) through the SUP-shaped encoder (5 convolutions, 18 DeepNorm layers, d_model 512, window
                (127, 128)) with seeded random weights; ms, chunks/s and the MFMA fraction of its algorithmic
                flops (convolutions, 4 products per layer, window attention over the keys each frame sees).
Usage: python bench.py [--gpus 1] [--steps 3] [--warmup 1] [--no-cpu] [--no-configs]
       python bench.py --mode encoder|prefill|scoring|update [--steps N]   (that object alone, N timed repetitions;
                                                    scoring / update: [--forms shared|unshared|shared,unshared])
       python bench.py --mode configs                       (the other configurations alone)
       python bench.py --mode kernels [--group-size G]      (the decode-attention traffic probe)
       python bench.py --mode products [--steps N] [--phase-stamps]   (the decode step's layer loop, captured)
"""

import argparse
import copy
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GSPO rollout tokens/sec on 1 MI355X (512 seq x 1024 tok); % HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
UPDATE_MICRO, UPDATE_T = 32, 768
ENC_CHUNKS = 128  # 64 windows x 2048 frames = 128 chunks of 12288 samples at stride 12
PREFIXES, GROUP, P, NEW = 64, 8, 2048, 1024
KV_ROW_BYTES = 2 * 2 * 64 * 2  # K + V, 2 KV heads, head_dim 64, bf16: one attended position of one layer


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def build_model(dev):
    from viktor_amd.synthetic import make_model
    m = make_model(1, n_layers=8, seed=0, rope_theta=1e6)
    g = copy.deepcopy(m).to(dev)
    g.projector.to(torch.bfloat16)
    g.decoder.to(torch.bfloat16)
    return m, g.eval()


def prefill_flops(windows, frames, layers=8, d=512, weights_per_layer=3014656, vocab=7):
    """Algorithmic flops of the shared-prefix prefill: per window of n = frames + 1 rows (frames + BOS), the
    projector (two 512 x 512 products per frame), 2 x weights per row for the decoder products, less the
    last layer's work the BOS-only last layer skips for the frame rows (o, gate_up, down and the q part of
    qkv: 5,242,880 flops per row), causal attention 1024 n (n + 1) in each of the first layers-1 layers and
    the BOS query's 2 x 2 x 8 x 64 x n in the last, and the LM head of the BOS row."""
    n = frames + 1
    proj = 2 * 2 * d * d * frames
    gemm = n * 2 * weights_per_layer * layers - frames * 5242880
    attn = (layers - 1) * 1024 * n * (n + 1) + 2 * 2 * 8 * 64 * n
    head = 2 * d * vocab
    return windows * (proj + gemm + attn + head)


def _attention_call(eng, layer, q, lens, plen=None):
    """One decode-attention launch of the engine's kind on layer `layer` of its caches."""
    from viktor_amd import hip_ops as ops
    cache = eng.cache
    if eng.G > 1:
        pc = eng.prefix_cache
        return lambda: ops.decode_attention_grouped(q, pc.k[layer], pc.v[layer], plen, cache.k[layer],
                                                    cache.v[layer], lens, eng.G, workspace=eng.grouped_workspace)
    return lambda: ops.decode_attention(q, cache.k[layer], cache.v[layer], lens, workspace=eng.fast.decode_workspace)


WEIGHT_BYTES = 2 * (8 * 3014656)  # the decoder's matmul weights in bf16, read once per decode step


def prefill_flops_lens(frame_lens, vocab=7):
    """prefill_flops summed over windows of the given frame counts."""
    return sum(prefill_flops(1, int(n), vocab=vocab) for n in frame_lens)


def decode_roofline_ms(attended, steps, B):
    """HBM-roofline time of `steps` decode steps: each step reads every attended K/V position of every layer
    (attended(j) positions at step j, 4096 B each over the 8 layers), writes B new positions and reads the
    weights once."""
    total = sum(attended(j) * 8 * KV_ROW_BYTES + B * 8 * KV_ROW_BYTES + WEIGHT_BYTES for j in range(steps))
    return total / (HBM_PEAK_GBS * 1e9) * 1e3


def _timed(fn, reps=1):
    """ms per call of fn() with HIP events on the current stream (after one untimed call)."""
    fn()
    e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    e[0].record()
    for _ in range(reps):
        fn()
    e[1].record()
    torch.cuda.synchronize()
    return e[0].elapsed_time(e[1]) / reps


def _bf16_model(k, dev, seed=0):
    from viktor_amd.synthetic import make_model
    m = make_model(k, n_layers=8, seed=seed, rope_theta=1e6)
    g = copy.deepcopy(m).to(dev)
    g.projector.to(torch.bfloat16)
    g.decoder.to(torch.bfloat16)
    return g.eval()


def _master_model(k, dev, seed=0):
    """The fp32 master model on the device, as the reference's scoring runs it (under torch.autocast)."""
    from viktor_amd.synthetic import make_model
    return make_model(k, n_layers=8, seed=seed, rope_theta=1e6).to(dev).eval()


def rollout_ungrouped(dev, gm, fr, u):
    """The rollout configuration as the reference runs it: every one of the 512 sequences prefilled and cached
    on its own (no prefix sharing, scripts/gspo.py:444 + viktor/engine.py:168-201); 1024 sampled tokens."""
    from viktor_amd import DecodeEngine
    B = PREFIXES * GROUP
    eng = DecodeEngine(gm, B, NEW, P, temperature=1.0, group_size=1)
    plens = [P] * B

    def run():
        eng.set_uniforms(u)
        eng.generate(fr, plens, steps=NEW)

    ms = _timed(run)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    eng.set_uniforms(u)
    e[0].record()
    eng.prefill(fr, plens)
    e[1].record()
    eng.decode(NEW)
    e[2].record()
    torch.cuda.synchronize()
    avg_s, alg = decode_attention_timing(eng, plens, NEW - 1)
    roof = decode_roofline_ms(lambda j: B * (P + 2 + j), NEW - 1, B)
    out = {"tokens_per_s": round(B * NEW / (ms / 1e3), 1), "ms_per_rollout": round(ms, 2),
           "prefill_ms": round(e[0].elapsed_time(e[1]), 2), "decode_ms": round(e[1].elapsed_time(e[2]), 2),
           "decode_roofline_ms": round(roof, 1), "decode_hbm_frac": round(roof / e[1].elapsed_time(e[2]), 4),
           "attention": {"avg_launch_us": round(avg_s * 1e6, 2), "alg_bytes_per_launch": int(alg),
                         "achieved_gbs": round(alg / avg_s / 1e9, 1),
                         "frac": round(alg / avg_s / 1e9 / HBM_PEAK_GBS, 4)}}
    del eng
    torch.cuda.empty_cache()
    return out


def varlen_kmer_config(dev, steps=340):
    """Variable-length prefill + 4-mer decode: 1024 sequences, prefixes uniform in [1200, 2048] frames (packed,
    no padding frames), vocab 343, greedy, 340 tokens (prefill token + 339 graph steps)."""
    from viktor_amd import DecodeEngine
    from viktor_amd.synthetic import varlen_lengths
    gm = _bf16_model(4, dev)
    B = 1024
    lens = [int(n) for n in varlen_lengths(B, 1200, 2048, seed=3)]
    g = torch.Generator(device=dev).manual_seed(4)
    fr = torch.randn(sum(lens), 512, generator=g, device=dev).to(torch.bfloat16)
    eng = DecodeEngine(gm, B, steps, max(lens), temperature=0.0)
    eng.generate(fr, lens, steps=steps)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    torch.cuda.synchronize()
    e[0].record()
    eng.prefill(fr, lens)
    e[1].record()
    eng.decode(steps)
    e[2].record()
    torch.cuda.synchronize()
    pre, dec = e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])
    pf = prefill_flops_lens(lens, vocab=343)
    tot = sum(lens)
    roof = decode_roofline_ms(lambda j: tot + B * (2 + j), steps - 1, B)
    avg_s, alg = decode_attention_timing(eng, lens, steps - 1, n_points=16)
    out = {"sequences": B, "prefix_frames": "U[1200, 2048]", "vocab": 343, "new_tokens": steps,
           "tokens_per_s": round(B * steps / ((pre + dec) / 1e3), 1), "prefill_ms": round(pre, 2),
           "decode_ms": round(dec, 2), "prefill_alg_tflop": round(pf / 1e12, 2),
           "prefill_mfma_frac": round(pf / (pre / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
           "decode_roofline_ms": round(roof, 1), "decode_hbm_frac": round(roof / dec, 4),
           "attention_frac": round(alg / avg_s / 1e9 / HBM_PEAK_GBS, 4)}
    del eng, fr
    torch.cuda.empty_cache()
    return out


def scoring_config(dev, reps=2, forms=("shared", "unshared")):
    """GSPO scoring: 512 sequences x (2048-frame prefix + 700..1024 response tokens), the teacher-forced forward
    of token_logprobs (scripts/gspo.py:340-353), then the sequence-ratio loss and its gradient w.r.t. the
    logits (scripts/gspo.py:459-477), with the fp32 master model and the autocast rounding points the reference
    scores with (an fp32 residual stream). The sequences are a rollout's: 64 windows x 8 samples, each window's
    frames repeated for its samples (scripts/gspo.py:444). Timed twice: with group_size 8 (each window's prefix
    run once, the token rows attending to it; log-probs equal to the unshared forward's) and unshared, every
    window in full as the reference computes it.
    Algorithmic flops, unshared, per sequence of n = 2048 + L rows: the projector per frame, 2 x weights per row
    less the last layer's products for the prefix rows (only the L token rows need logits), causal attention
    1024 n (n + 1) per layer, the LM head per token. Shared: the projector and the prefix rows' products once per
    window, the prefix rows' causal attention in 7 layers (1024 P (P + 1) each), and per sample its L token rows'
    products, their attention to P + t + 1 keys (2048 (L P + L (L + 1) / 2) per layer) and the LM head."""
    from viktor_amd import gspo as G
    from viktor_amd.synthetic import scoring_inputs
    gm = _master_model(1, dev)
    B = PREFIXES * GROUP
    seqs, ended = scoring_inputs(B, 700, 1024, k=1, seed=5)
    g = torch.Generator(device=dev).manual_seed(6)
    fr = torch.randn(PREFIXES, P, 512, generator=g, device=dev).to(torch.bfloat16).repeat_interleave(GROUP, 0)
    plens = torch.full((B,), P, device=dev)
    # the old policy's log-probs (in the first form timed)
    lp, mask = G.token_logprobs(gm, fr, plens, seqs, ended, group_size=GROUP if "shared" in forms else 1)
    old = (lp + 0.05 * torch.randn(lp.shape, generator=g, device=dev)).contiguous()
    nb = torch.tensor([max(len(q), 1) for q in seqs], dtype=torch.float32, device=dev)
    adv = torch.randn(B, generator=g, device=dev)
    tin, tgt, _ = gm.batch(seqs, pad_to=128)
    tin, tgt = tin.to(dev), tgt.clamp(min=0).to(dev).contiguous()
    mask = mask.to(dev)

    def run(group):  # teacher-forced logits, then log-probs + ratio + clipped loss + dL/dlogits in one kernel
        logits = gm.logits(fr, tin, plens, group_size=group)
        G.ops.gspo_score(logits.contiguous(), tgt, mask, old, nb, adv, 3e-4, 4e-4, grad=True)

    ms = _timed(lambda: run(GROUP), reps) if "shared" in forms else None
    ms_full = _timed(lambda: run(1), reps) if "unshared" in forms else None
    L = [len(q) + 1 for q in seqs]
    flops = flops_full = 0
    for n_tok in L:
        n = P + n_tok
        flops_full += 2 * 2 * 512 * 512 * P + 2 * 3014656 * 8 * n - P * 5242880 + 8 * 1024 * n * (n + 1) + 2 * 512 * 7 * n_tok
        flops += 2 * 3014656 * 8 * n_tok + 8 * 2048 * (n_tok * P + n_tok * (n_tok + 1) // 2) + 2 * 512 * 7 * n_tok
    flops += PREFIXES * (2 * 2 * 512 * 512 * P + 2 * 3014656 * 8 * P - P * 5242880 + 7 * 1024 * P * (P + 1))
    out = {"sequences": B, "windows": PREFIXES, "group_size": GROUP, "response_tokens": "U[700, 1024]"}
    if ms is not None:
        tf = flops / (ms / 1e3) / 1e12
        out.update({"ms": round(ms, 2), "tokens_per_s": round(sum(L) / (ms / 1e3), 1),
                    "alg_tflop": round(flops / 1e12, 2), "achieved_tflops": round(tf, 1),
                    "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)})
    if ms_full is not None:
        out["unshared"] = {"ms": round(ms_full, 2), "tokens_per_s": round(sum(L) / (ms_full / 1e3), 1),
                           "alg_tflop": round(flops_full / 1e12, 2),
                           "mfma_frac": round(flops_full / (ms_full / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                           "note": "every window in full, as the reference scores them"}
    out.update({"includes": "projector + teacher-forced 8-layer forward (fp32 master weights, autocast rounding points, "
                       "padded to a multiple of 128 tokens as the reference pads) + LM head + log-probs, ratio, "
                       "clipped loss and dL/dlogits [512, T, 7]"})
    del fr
    torch.cuda.empty_cache()
    return out


def stress_config(dev, steps=32):
    """Large-batch greedy decode: 4096 sequences x 2048-frame prefixes, each on its own cache rows (51.5 GB of
    KV cache), vocab 7. Measured: the prefill, `steps` graph-replayed decode steps right after it, and the
    decode-attention kernel at the lengths of the whole 1024-step decode (8-layer rotation)."""
    from viktor_amd import DecodeEngine
    gm = _bf16_model(1, dev)
    B = 4096
    g = torch.Generator(device=dev).manual_seed(7)
    fr = torch.randn(B * P, 512, generator=g, device=dev).to(torch.bfloat16)
    eng = DecodeEngine(gm, B, NEW, P, temperature=0.0)
    plens = [P] * B
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    eng.generate(fr, plens, steps=steps)
    torch.cuda.synchronize()
    e[0].record()
    eng.prefill(fr, plens)
    e[1].record()
    eng.decode(steps)
    e[2].record()
    torch.cuda.synchronize()
    pre, dec = e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])
    avg_s, alg = decode_attention_timing(eng, plens, NEW - 1, n_points=8, rounds=1)
    early_roof = decode_roofline_ms(lambda j: B * (P + 2 + j), steps - 1, B)
    out = {"sequences": B, "kv_cache_gb": round(2 * eng.cache.k.numel() * 2 / 1e9, 2), "prefill_ms": round(pre, 1),
           "prefill_mfma_frac": round(prefill_flops(B, P) / (pre / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
           "decode_ms_per_step_early": round(dec / (steps - 1), 3),
           "decode_hbm_frac_early": round(early_roof / dec, 4),
           "attention": {"avg_launch_us": round(avg_s * 1e6, 1), "alg_bytes_per_launch": int(alg),
                         "achieved_gbs": round(alg / avg_s / 1e9, 1),
                         "frac": round(alg / avg_s / 1e9 / HBM_PEAK_GBS, 4)}}
    del eng, fr
    torch.cuda.empty_cache()
    return out


def other_configs(dev, gm, fr, u):
    """The benchmark's other configurations, each with its own roofline (see the functions)."""
    log("config: rollout without prefix sharing")
    res = {"gspo_rollout_unshared": rollout_ungrouped(dev, gm, fr, u)}
    log("config: varlen prefill + 4-mer decode")
    res["varlen_kmer"] = varlen_kmer_config(dev)
    log("config: scoring")
    res["scoring"] = scoring_config(dev)
    log("config: 4096-sequence stress")
    res["stress_4096"] = stress_config(dev)
    return res


def decode_attention_timing(eng, prefix_lens, steps, n_points=32, rounds=2, warm=False):
    """Average duration (HIP events on the launch stream) and algorithmic bytes of one decode-attention call at
    the attended lengths of decode steps j = 0 .. steps - 1, sampled at n_points evenly spaced steps. Sequence
    b attends prefix_lens[b] + 1 positions (frames + BOS) and j + 1 own tokens at step j.

    As in the captured rollout, each timed call reads a layer whose K/V no recent call has touched: the calls
    rotate over the 8 layers' caches (`rounds` passes of 8 calls per point, after one untimed pass), so
    nothing the call reads is still in the 256 MB Infinity Cache from the call before -- exactly the situation
    of layer i's attention inside a decode step, which follows the other 7 layers' attention reads. warm=True
    instead repeats one layer's call back to back (5 calls), whose bytes then come partly from that cache."""
    B, G = eng.B, eng.G
    dev = eng.cache.k.device
    layers = eng.cache.k.shape[0]
    q = torch.randn(B, 8, 64, device=dev).to(torch.bfloat16)
    pl = torch.as_tensor(prefix_lens, dtype=torch.int64)
    js = [round(i * (steps - 1) / (n_points - 1)) for i in range(n_points)]
    total_ms, total_bytes, launches = 0.0, 0.0, 0
    stream = torch.cuda.current_stream()
    plen = None
    if G > 1:
        plen = (pl[::G] + 1).to(torch.int32).to(dev)
    for j in js:
        if G > 1:
            lens = torch.full((B,), j + 1, dtype=torch.int32, device=dev)
            kv_rows = int((pl[::G] + 1).sum()) + B * (j + 1)
        else:
            lens = (pl + 2 + j).to(torch.int32).to(dev)
            kv_rows = int((pl + 2 + j).sum())
        calls = [_attention_call(eng, i, q, lens, plen) for i in range(layers)]
        seq = [calls[3]] * 5 if warm else calls * rounds
        for c in ([calls[3]] if warm else calls):  # untimed: first-launch costs, and the rotation's start state
            c()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for c in seq:
            c()
        e1.record(stream)
        e1.synchronize()
        total_ms += e0.elapsed_time(e1)
        launches += len(seq)
        total_bytes += len(seq) * (kv_rows * KV_ROW_BYTES + 2 * B * 8 * 64 * 2)
    avg_s = total_ms / 1e3 / launches
    return avg_s, total_bytes / launches


def in_graph_attention_timing(gm, fr, u, plens, group_size, n_points=32):
    """The decode attention inside the captured rollout step itself: a second engine of the benchmark's shape
    captures its step with a device timestamp (vk_timestamp, a one-thread kernel storing the GPU's constant-rate
    clock) right before and right after each layer's attention launch, and a back-to-back pair at the step's end;
    it runs the rollout's prefill and its 1023 steps by single-step replays and, at n_points evenly spaced steps,
    waits for the step and reads the stamps. A launch's time is its pair's interval less the back-to-back pair's
    (the dispatch gap between two graph nodes). Returns (average seconds per launch, algorithmic bytes per launch
    averaged over the same steps)."""
    import ctypes
    from viktor_amd import DecodeEngine
    from viktor_amd._lib import call, stream_handle
    B = PREFIXES * GROUP
    eng = DecodeEngine(gm, B, NEW, P, temperature=1.0, group_size=group_size, cuda_graph=False, check_every=1)
    layers = eng.cache.k.shape[0]
    stamps = torch.zeros(2 * layers + 2, dtype=torch.int64, device=gm.decoder.lm_head.weight.device)
    khz = ctypes.c_int64(0)
    call("vk_timestamp_rate_khz", ctypes.byref(khz))
    stamp = lambda i: call("vk_timestamp", stamps.data_ptr(), i, stream_handle())
    eng.fast.attn_marks = lambda i, k: stamp(2 * i + k)
    step = eng._step

    def step_with_gap():  # the step, then the back-to-back pair
        step()
        stamp(2 * layers)
        stamp(2 * layers + 1)

    eng._step = step_with_gap
    try:
        eng._capture()
    finally:
        eng.fast.attn_marks = None
        eng._step = step
    eng.set_uniforms(u)
    eng.prefill(fr, plens)
    steps = NEW - 1
    js = {round(i * (steps - 1) / (n_points - 1)) for i in range(n_points)}
    pl = torch.as_tensor(plens, dtype=torch.int64)
    total_ticks, total_bytes, launches = 0, 0.0, 0
    for j in range(steps):
        eng.graph.replay()
        if j in js:
            t = stamps.cpu()  # waits for the step
            gap = int(t[2 * layers + 1] - t[2 * layers])
            total_ticks += sum(int(t[2 * i + 1] - t[2 * i]) - gap for i in range(layers))
            if group_size > 1:
                kv_rows = int((pl[::group_size] + 1).sum()) + B * (j + 1)
            else:
                kv_rows = int((pl + 2 + j).sum())
            total_bytes += layers * (kv_rows * KV_ROW_BYTES + 2 * B * 8 * 64 * 2)
            launches += layers
    torch.cuda.synchronize()
    del eng
    torch.cuda.empty_cache()
    return total_ticks / (khz.value * 1e3) / launches, total_bytes / launches


def _cpu_info():
    """Host CPU facts for the baseline: logical CPUs, the ones this process may run on, the cgroup quota."""
    info = {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()
        if quota != "max":
            info["cgroup_cpus"] = round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            info["model"] = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "?")
    except OSError:
        info["model"] = "?"
    return info


def cpu_baseline(runs=3):
    """The CPU oracle in fp32 (the reference's torch path restated: viktor/decoder.py + viktor/engine.py with the
    torch backend) on the CPU-plumbing configuration at full size: 4 sequences x 2048-frame prefixes of N(0, 1)
    features, 8 layers, 64 greedy steps, weights and frames from seed 0 -- `runs` runs (about 3.4 s each on 16
    EPYC cores). Threads: every CPU this process may use (the affinity set, capped by a cgroup CPU quota)."""
    from oracle import reference as R
    from viktor_amd.synthetic import frames, make_model
    info = _cpu_info()
    threads = info["affinity"]
    if "cgroup_cpus" in info:
        threads = max(1, min(threads, int(info["cgroup_cpus"])))
    torch.set_num_threads(threads)
    m = make_model(1, n_layers=8, seed=0, rope_theta=1e6)
    n_seq, steps = 4, 64
    eng = R.RefEngine(R.RefModel(m, "fp32"), steps, temperature=0.0)
    fr = frames(n_seq, P, 512, seed=0)
    t0 = time.perf_counter()
    for _ in range(runs):
        eng.run([fr[i] for i in range(n_seq)])
    dt = time.perf_counter() - t0
    return {"value": round(runs * n_seq * steps / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the CPU-plumbing configuration at full size, {runs} runs: {n_seq} sequences x {P}-frame "
                      f"prefix x {steps} greedy tokens (prefill + decode), 8 layers, fp32 CPU restatement of the "
                      f"reference torch path; {dt:.1f} s", "host": info}


def reward_timing(tokenizer, reps=5):
    """A rollout's rewards on the device from output tokens (see the module docstring)."""
    import numpy as np
    from viktor_amd import reward as RW
    rng = np.random.default_rng(11)
    labels = ["".join(rng.choice(list("ACGT"), int(n))) for n in rng.integers(900, 1100, PREFIXES)]
    weights = [(rng.random(len(l)) > 0.05).astype(np.float32) for l in labels]
    rows = np.zeros((PREFIXES * GROUP, NEW), dtype=np.int64)  # PAD
    for i in range(PREFIXES * GROUP):
        call = []
        for ch in labels[i // GROUP]:
            u = rng.random()
            if u < 0.05 / 3:
                continue
            call.append(rng.choice(list("ACGT")) if u < 0.1 / 3 else ch)
            if rng.random() < 0.05 / 3:
                call.append(rng.choice(list("ACGT")))
        call = call[:NEW - 1]
        rows[i, :len(call)] = [3 + "ACGT".index(b) for b in call]
        rows[i, len(call)] = 2  # EOS
    tokens = torch.from_numpy(rows).to("cuda")
    for _ in range(2):
        res = RW.gspo_rewards_from_tokens(tokens, tokenizer, labels, weights, GROUP)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        res = RW.gspo_rewards_from_tokens(tokens, tokenizer, labels, weights, GROUP)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    _, _, lens, _ = RW.calls_from_tokens(tokens, tokenizer)
    call_len = lens.cpu().numpy()
    cells = float(sum(len(labels[i // GROUP]) * int(n) for i, n in enumerate(call_len)))
    return {"rewards": int(tokens.shape[0]), "ms_per_rollout": round(ms, 3), "cells_per_s": round(cells / (ms / 1e3), 1),
            "mean_call_bases": round(float(call_len.mean()), 1), "mean_reward": round(float(res["reward"].mean()), 4),
            "includes": "token decode on the device + packing of the labels + the DP kernel"}


def encoder_timing(reps=3):
    """The encoder for one rollout's windows (see the module docstring): ms and MFMA fraction."""
    from viktor_amd.encoder import DoradoEncoder
    from viktor_amd.synthetic import SUP_ENCODER_CFG, encoder_state_dict, signal
    dev = torch.device("cuda", 0)
    enc = DoradoEncoder(SUP_ENCODER_CFG, dev).load_state_dict(encoder_state_dict(seed=12))
    n_chunks, chunk = ENC_CHUNKS, SUP_ENCODER_CFG["basecaller"]["chunksize"]
    sig = signal(n_chunks * chunk, seed=13).to(dev)
    lens = [chunk] * n_chunks
    for _ in range(2):
        out = enc.forward_varlen(sig, lens)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record()
    for _ in range(reps):
        out = enc.forward_varlen(sig, lens)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    flops = enc.flops_per_chunk(chunk) * n_chunks
    tflops = flops / (ms / 1e3) / 1e12
    assert torch.isfinite(out).all()
    return {"chunks": n_chunks, "chunk_samples": chunk, "frames": int(out.shape[0]),
            "layers": enc.depth, "ms": round(ms, 2), "chunks_per_s": round(n_chunks / (ms / 1e3), 1),
            "samples_per_s": round(n_chunks * chunk / (ms / 1e3), 1), "alg_tflop": round(flops / 1e12, 3),
            "achieved_tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}


def prefill_timing(reps=3, prefill_batch=128, group_size=GROUP):
    """The rollout's shared-prefix prefill alone (64 windows of 2048 frames, one prefill per group): ms per
    prefill with HIP events, and the achieved rate on prefill_flops."""
    from viktor_amd import DecodeEngine
    from viktor_amd.synthetic import frames, uniforms
    dev = torch.device("cuda", 0)
    _, gm = build_model(dev)
    B = PREFIXES * group_size
    fr = frames(PREFIXES, P, 512, seed=0).to(dev).repeat_interleave(group_size, 0).reshape(-1, 512)
    eng = DecodeEngine(gm, B, NEW, P, temperature=1.0, prefill_batch=prefill_batch, group_size=group_size)
    eng.set_uniforms(uniforms(B, NEW, seed=1).to(dev))
    for _ in range(2):
        eng.prefill(fr, [P] * B)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record()
    for _ in range(reps):
        eng.prefill(fr, [P] * B)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    windows = PREFIXES if group_size > 1 else B
    flops = prefill_flops(windows, P)
    tflops = flops / (ms / 1e3) / 1e12
    return {"windows_prefilled": windows, "ms": round(ms, 2), "alg_tflop": round(flops / 1e12, 3),
            "achieved_tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}


def update_timing(steps=3, warmup=2, forms=("shared", "unshared")):
    """One GSPO update micro-batch on the HIP training path (see the module docstring): times and flops. The
    micro-batch is whole groups, as the reference's update loop takes them (scripts/gspo.py:453, 466-468): 4
    windows x 8 calls, each window's frames repeated for its calls. Timed with group_size 8 (each window's prefix
    rows once, the backward summing its calls' gradients into them) and unshared (every call's full window, as
    the reference computes it)."""
    from viktor_amd import train as TR
    from viktor_amd.gspo import sequence_ratio_loss
    from viktor_amd.synthetic import frames, make_model
    dev = torch.device("cuda", 0)
    B, T = UPDATE_MICRO, UPDATE_T
    ng = B // GROUP
    m = make_model(1, n_layers=8, seed=7).to(dev)
    opt = TR.HipAdamW(list(m.parameters()), lr=1e-6, betas=(0.9, 0.95), weight_decay=0.0, max_grad_norm=1.0)
    g = torch.Generator().manual_seed(8)
    fr = frames(ng, P, 512, seed=9).to(dev).repeat_interleave(GROUP, 0).contiguous()
    pl = torch.full((B,), P, device=dev)
    tok = torch.randint(3, 7, (B, T), generator=g).to(dev)
    tgt = torch.randint(3, 7, (B, T), generator=g).to(dev)
    mask = torch.ones(B, T, dtype=torch.bool, device=dev)
    nb = torch.full((B,), float(T), device=dev)
    adv = torch.randn(B, generator=g).to(dev)
    with torch.no_grad():
        z0 = TR.train_logits(m, fr, tok, pl, group_size=GROUP if "shared" in forms else 1)
        old = torch.log_softmax(z0.float(), -1).gather(-1, tgt[..., None])[..., 0]

    def run(group):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        acc = [0.0, 0.0, 0.0]
        for it in range(warmup + steps):
            opt.zero_grad()
            ev[0].record()
            z = TR.train_logits(m, fr, tok, pl, group_size=group)
            loss = sequence_ratio_loss(z, tgt, mask, old, nb, adv, 4e-4, 4e-4, 1.0 / B)[0]
            ev[1].record()
            loss.backward()
            ev[2].record()
            opt.step()
            ev[3].record()
            torch.cuda.synchronize()
            if it >= warmup:
                for i in range(3):
                    acc[i] += ev[i].elapsed_time(ev[i + 1]) / steps
        return acc

    acc = run(GROUP) if "shared" in forms else None
    acc_full = run(1) if "unshared" in forms else None
    weights = 8 * 3014656  # decoder matmul weights
    n = P + T
    rows_full = B * n
    gemm_full = 3 * 2 * weights * rows_full + 3 * 2 * 2 * 512 * 512 * B * P + 3 * 2 * 512 * 7 * B * T
    attn_full = 3.5 * 1024 * n * (n + 1) * 8 * B
    rows = ng * P + B * T
    gemm = 3 * 2 * weights * rows + 3 * 2 * 2 * 512 * 512 * ng * P + 3 * 2 * 512 * 7 * B * T
    attn = 3.5 * 8 * (1024 * P * (P + 1) * ng + (1024 * T * (T + 1) + 2048 * T * P) * B)
    out = {"microbatch": f"{B} calls = {ng} windows x {GROUP} ({P} frames + {T} tokens), 8 layers, "
                         "fwd + bwd + clip + AdamW", "group_size": GROUP}
    if acc is not None:
        ms = sum(acc)
        tflops = (gemm + attn) / (ms / 1e3) / 1e12
        out.update({"ms_per_microbatch": round(ms, 2), "forward_ms": round(acc[0], 2),
                    "backward_ms": round(acc[1], 2), "optimizer_ms": round(acc[2], 3),
                    "calls_per_s": round(B / (ms / 1e3), 1), "alg_tflop": round((gemm + attn) / 1e12, 2),
                    "achieved_tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)})
    if acc_full is not None:
        ms_full = sum(acc_full)
        out["unshared"] = {"ms_per_microbatch": round(ms_full, 2), "forward_ms": round(acc_full[0], 2),
                           "backward_ms": round(acc_full[1], 2),
                           "rows_per_s": round(rows_full / (ms_full / 1e3), 1),
                           "alg_tflop": round((gemm_full + attn_full) / 1e12, 2),
                           "mfma_frac": round((gemm_full + attn_full) / (ms_full / 1e3) / 1e12 /
                                              MFMA_BF16_PEAK_TFLOPS, 4),
                           "note": "every call's full window, as the reference computes it"}
    return out


def kernels_mode(group, reps=5):
    """Only the dominant kernel at the rollout's mean shape plus a plain 256 MiB device copy of known size,
    for hardware-counter runs (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE): the copy's counter readings give
    the scale factor from counter units to bytes. group 1: 512 sequences x 2561 attended positions of a
    3073-position cache layer; group G: 512 / G shared 2049-position prefixes + 512 own 512-position rows, in
    the engine's padded cache layout."""
    from viktor_amd import hip_ops as ops
    dev = torch.device("cuda", 0)
    B, S, L = PREFIXES * GROUP, P + 1 + NEW, P + 2 + (NEW - 2) // 2
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, 8, 64, device=dev, generator=g).to(torch.bfloat16)
    if group == 1:
        kc = torch.randn(B, S, 2, 64, device=dev, generator=g).to(torch.bfloat16)
        vc = torch.randn(B, S, 2, 64, device=dev, generator=g).to(torch.bfloat16)
        lens = torch.full((B,), L, dtype=torch.int32, device=dev)
        ws = ops.decode_attention_workspace(B, 8, S, dev)
        call = lambda: ops.decode_attention(q, kc, vc, lens, workspace=ws)
        alg_rows = B * L
    else:  # the engine's padded sequence strides
        from viktor_amd import DecodeEngine
        pp, op = DecodeEngine.PREFIX_PAD_ROWS, DecodeEngine.OWN_PAD_ROWS
        kp = torch.randn(B // group, P + 1 + pp, 2, 64, device=dev, generator=g).to(torch.bfloat16)[:, :P + 1]
        vp = torch.randn(B // group, P + 1 + pp, 2, 64, device=dev, generator=g).to(torch.bfloat16)[:, :P + 1]
        ks = torch.randn(B, NEW + op, 2, 64, device=dev, generator=g).to(torch.bfloat16)[:, :NEW]
        vs = torch.randn(B, NEW + op, 2, 64, device=dev, generator=g).to(torch.bfloat16)[:, :NEW]
        plen = torch.full((B // group,), P + 1, dtype=torch.int32, device=dev)
        slen = torch.full((B,), L - P - 1, dtype=torch.int32, device=dev)
        ws = ops.decode_attention_grouped_workspace(B, group, P + 1, NEW, dev)
        call = lambda: ops.decode_attention_grouped(q, kp, vp, plen, ks, vs, slen, group, workspace=ws)
        alg_rows = (B // group) * (P + 1) + B * (L - P - 1)
    for _ in range(reps):
        call()
    x = torch.ones(128 << 20, dtype=torch.bfloat16, device=dev)  # 256 MiB
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    alg = alg_rows * KV_ROW_BYTES + 2 * B * 8 * 64 * 2
    print(json.dumps({"group": group, "decode_attention_alg_bytes": alg, "copy_bytes_each_way": x.numel() * 2, "reps": reps}))


# The decode step's small products at the rollout's 512 rows (d 512, ffn 1536, 8 + 2 x 2 heads of 64): their
# operands (weights, activations, row sums, K/V rows written) per launch, the algorithmic bytes of each.
PRODUCT_BYTES = {
    "qkv": 512 * 512 * 2 + 512 * 16 * 4 + 768 * 512 * 2 + 512 * 512 * 2 + 512 * 512,
    "o": 512 * 512 * 2 + 512 * 512 * 2 + 2 * 512 * 512 * 2 + 512 * 16 * 4,
    "gate_up": 512 * 512 * 2 + 512 * 16 * 4 + 3072 * 512 * 2 + 512 * 1536 * 2,
    "down": 512 * 1536 * 2 + 512 * 1536 * 2 + 2 * 512 * 512 * 2 + 512 * 16 * 4,
}
PRODUCT_FLOPS = {"qkv": 2 * 512 * 512 * 768, "o": 2 * 512 * 512 * 512, "gate_up": 2 * 512 * 512 * 3072,
                 "down": 2 * 512 * 1536 * 512}
PRODUCT_WGS = {"qkv": 192, "o": 256, "gate_up": 256, "down": 256}


def products_mode(reps=50, stamps=False):
    """The decode step's layer loop at the rollout's mean step (512 sequences in 64 groups of 8, 2049 shared
    prefix positions + 512 own positions each) through FastDecoder.decode_residual: per layer norm + qkv + QK-norm
    + RoPE + cache write, grouped attention, o + residual, norm + gate_up + SwiGLU, down + residual (layer 0 from a
    handed-in residual stream instead of the embedding gather; no LM head). It is captured once in a HIP graph and
    replayed `reps` times, so the four products run between attention launches that stream the caches, as in the
    rollout; then a plain 256 MiB device copy (the counter scale of rocprofv3 FETCH_SIZE / WRITE_SIZE runs).
    stamps: the profiling build (libviktor_hip_stamps.so) is loaded instead of the product library and the
    per-workgroup phase timestamps of the last replay are summarised per product (layers 1-7: their qkv takes the
    handed-over row sums, as in the rollout)."""
    import ctypes
    from viktor_amd import _lib as L
    if stamps:
        from viktor_amd.build import STAMPS_LIB
        L.load(STAMPS_LIB)  # before anything else loads the product library
    from viktor_amd import hip_ops as ops
    from viktor_amd import DecodeEngine
    from viktor_amd.decoder import KVCache
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _, gm = build_model(dev)
    fast, cfg = gm.decoder.fast(), gm.decoder.cfg
    B, G = PREFIXES * GROUP, GROUP
    own = (NEW - 2) // 2 + 1  # own rows attended at the rollout's mean step, the new one included
    gen = torch.Generator(device=dev).manual_seed(0)
    cache = KVCache(cfg, B, NEW, torch.bfloat16, dev, pad_rows=DecodeEngine.OWN_PAD_ROWS)
    pc = KVCache(cfg, B // G, P + 1, torch.bfloat16, dev, pad_rows=DecodeEngine.PREFIX_PAD_ROWS)
    for t in (cache.k, cache.v, pc.k, pc.v):
        t.normal_(generator=gen)
    plen32 = torch.full((B // G,), P + 1, dtype=torch.int32, device=dev)
    seqlens = torch.full((B,), own, dtype=torch.int32, device=dev)
    pos32 = torch.full((B,), own - 1, dtype=torch.int32, device=dev)
    rpos32 = pos32 + (P + 1)
    rows = torch.arange(B, dtype=torch.int32, device=dev)
    gws = ops.decode_attention_grouped_workspace(B, G, P + 1, NEW, dev)
    x0 = torch.randn(B, cfg.d_model, device=dev, generator=gen).to(torch.bfloat16)
    x = x0.clone()

    def step():
        x.copy_(x0)
        fast.decode_residual(pos32, rows, seqlens, cache, rope_pos=rpos32, x=x, prefix=(pc, plen32, G, gws))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    layers = cfg.n_layers
    order = ["qkv", "o", "gate_up", "down"]  # the stamped launches of a layer, in launch order
    slots = 8 * sum(PRODUCT_WGS.values()) * layers
    buf = torch.zeros(slots, dtype=torch.int64, device=dev)
    if stamps:
        L.call("vk_phase_stamps_set", ctypes.c_void_p(buf.data_ptr()), ctypes.c_int64(slots))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    if stamps:
        used = ctypes.c_int64(0)
        L.call("vk_phase_stamps_used", ctypes.byref(used))
        assert used.value == slots, f"stamped launches took {used.value} slots, expected {slots}"
        L.call("vk_phase_stamps_set", ctypes.c_void_p(0), ctypes.c_int64(0))
    graph.replay()
    ms = _timed(graph.replay, reps)
    out = {"workload": "decode step layer loop, 512 sequences (64 groups x 8), 2049 prefix + 512 own positions, "
                       "8 layers, captured", "reps": reps, "ms_per_step": round(ms, 4),
           "product_alg_bytes": PRODUCT_BYTES, "product_flops": PRODUCT_FLOPS}
    if stamps:
        khz = ctypes.c_int64(0)
        L.call("vk_timestamp_rate_khz", ctypes.byref(khz))
        us = 1e3 / khz.value  # microseconds per tick
        t = buf.cpu().view(-1, 8)
        names = ["first_data", "normalise", "k_loop", "tile_sum", "epilogue"]
        summary, off = {}, 0
        spans = {k: [] for k in order}
        phases = {k: [] for k in order}
        starts = {k: [] for k in order}
        for layer in range(layers):
            for k in order:
                n = PRODUCT_WGS[k]
                w = t[off:off + n, :6].double()
                off += n
                if layer == 0:
                    continue
                spans[k].append(float(w[:, 5].max() - w[:, 0].min()) * us)
                phases[k].append(((w[:, 1:6] - w[:, 0:5]) * us).mean(0))
                starts[k].append(float((w[:, 0] - w[:, 0].min()).mean()) * us)
        for k in order:
            ph = torch.stack(phases[k]).mean(0)
            summary[k] = {"workgroups": PRODUCT_WGS[k], "span_us": round(sum(spans[k]) / len(spans[k]), 3),
                          "mean_start_offset_us": round(sum(starts[k]) / len(starts[k]), 3),
                          **{f"{nm}_us": round(float(v), 3) for nm, v in zip(names, ph)},
                          "workgroup_us": round(float(ph.sum()), 3)}
        out["phases"] = summary
        out["phase_slots"] = "0 entry, 1 first operands landed, 2 K loop start, 3 K loop end, 4 tile summed, 5 end"
    print(json.dumps(out), flush=True)
    del graph
    cp = torch.ones(128 << 20, dtype=torch.bfloat16, device=dev)  # 256 MiB
    cp2 = torch.empty_like(cp)
    for _ in range(5):
        cp2.copy_(cp)
    torch.cuda.synchronize()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other configurations' measurements")
    ap.add_argument("--prefill-batch", type=int, default=128)
    ap.add_argument("--mode", choices=["rollout", "kernels", "products", "encoder", "prefill", "configs", "update",
                                       "scoring"],
                    default="rollout",
                    help="kernels: decode-attention traffic probe; products: the decode step's layer loop captured "
                         "(kernel traces, counters, --phase-stamps); encoder / prefill / configs / update / scoring: "
                         "that object alone")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="products mode: load the phase-timestamp profiling build and summarise its stamps")
    ap.add_argument("--group-size", type=int, default=GROUP, help="sequences sharing one prefix KV copy (1: none)")
    ap.add_argument("--forms", default="shared,unshared",
                    help="--mode scoring / update: which forms to time (shared: each window's prefix once for its "
                         "calls; unshared: every call's full window)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the rollout path has no multi-GPU mode here (one process per GPU, "
              "whole GSPO groups per rank); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.mode == "kernels":
        kernels_mode(args.group_size)
        return
    if args.mode == "products":
        products_mode(reps=max(args.steps, 1), stamps=args.phase_stamps)
        return
    if args.mode == "encoder":
        print(json.dumps({"encoder": encoder_timing(reps=max(args.steps, 1))}), flush=True)
        return
    if args.mode == "configs":
        from viktor_amd.synthetic import frames, uniforms
        dev = torch.device("cuda", 0)
        _, gm = build_model(dev)
        fr = frames(PREFIXES, P, 512, seed=0).to(dev).repeat_interleave(GROUP, 0).reshape(-1, 512)
        u = uniforms(PREFIXES * GROUP, NEW, seed=1).to(dev)
        print(json.dumps({"configs": other_configs(dev, gm, fr, u)}), flush=True)
        return
    if args.mode == "scoring":
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        print(json.dumps({"scoring": scoring_config(dev, reps=max(args.steps, 1), forms=args.forms.split(","))}),
              flush=True)
        return
    if args.mode == "update":
        print(json.dumps({"gspo_update": update_timing(steps=max(args.steps, 1), warmup=args.warmup,
                                                       forms=args.forms.split(","))}), flush=True)
        return
    if args.mode == "prefill":
        print(json.dumps({"prefill": prefill_timing(reps=max(args.steps, 1), prefill_batch=args.prefill_batch,
                                                    group_size=args.group_size)}), flush=True)
        return
    from viktor_amd import DecodeEngine
    from viktor_amd.synthetic import frames, uniforms

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log("building model / inputs")
    _, gm = build_model(dev)
    B = PREFIXES * GROUP
    fr = frames(PREFIXES, P, 512, seed=0).to(dev).repeat_interleave(GROUP, 0).reshape(-1, 512)
    u = uniforms(B, NEW, seed=1).to(dev)
    plens = [P] * B
    eng = DecodeEngine(gm, B, NEW, P, temperature=1.0, prefill_batch=args.prefill_batch, group_size=args.group_size)
    torch.cuda.synchronize()

    def rollout():
        eng.set_uniforms(u)
        eng.generate(fr, plens, steps=NEW)

    log(f"warmup x{args.warmup}")
    for _ in range(args.warmup):
        rollout()
    torch.cuda.synchronize()
    # prefill / decode split of one rollout (reported, not the metric)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    eng.set_uniforms(u)
    e[0].record()
    eng.prefill(fr, plens)
    e[1].record()
    eng.decode(NEW)
    e[2].record()
    torch.cuda.synchronize()
    prefill_ms, decode_ms = e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])

    log(f"timed x{args.steps}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rollout()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    value = B * NEW * args.steps / dt

    log("decode-attention timing")
    eager_s, eager_bytes = decode_attention_timing(eng, plens, NEW - 1)
    warm_s, warm_bytes = decode_attention_timing(eng, plens, NEW - 1, warm=True)
    if args.group_size == 1:
        attn_kernels = "decode_attention (decode_attn_kernel)"
    else:
        from viktor_amd import hip_ops as ops
        members, parts = ops.decode_attention_grouped_layout(B, args.group_size, P + 1, eng.cache.k.shape[2])
        attn_kernels = (f"decode_attention_grouped (grouped_attn_kernel: {members} query members per workgroup, "
                        f"{parts} part(s)" + (" + grouped_combine_kernel)" if parts > 1 else ", no merge launch)"))
    achieved = None  # set from the in-graph timing below
    traffic = None
    tname = "decode_attention_traffic.json" if args.group_size == 1 else "decode_attention_grouped_traffic.json"
    tpath = os.path.join(ROOT, "profiles", tname)
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")
    windows = PREFIXES if args.group_size > 1 else B
    pf = prefill_flops(windows, P)
    prefill_obj = {"windows_prefilled": windows, "alg_tflop": round(pf / 1e12, 3),
                   "achieved_tflops": round(pf / (prefill_ms / 1e3) / 1e12, 1),
                   "mfma_frac": round(pf / (prefill_ms / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
    out = tokens_check = eng.out[:, :NEW].cpu()
    live = int(((out != 0) & (out != 2)).sum())
    del eng
    torch.cuda.empty_cache()
    log("decode-attention timing inside the captured step")
    avg_s, alg_bytes = in_graph_attention_timing(gm, fr, u, plens, args.group_size)
    achieved = alg_bytes / avg_s / 1e9
    # the decode's own HBM roofline: every attended K/V position once (the shared prefix once per group), the new
    # positions written, the weights read once per step
    if args.group_size > 1:
        dec_roof = decode_roofline_ms(lambda j: PREFIXES * (P + 1) + B * (j + 1), NEW - 1, B)
    else:
        dec_roof = decode_roofline_ms(lambda j: B * (P + 2 + j), NEW - 1, B)
    configs = {}
    if not args.no_configs:
        configs = other_configs(dev, gm, fr, u)
    log("gspo reward")
    reward = reward_timing(gm.tokenizer)
    log("gspo update micro-batch")
    update = update_timing()
    log("encoder")
    torch.cuda.empty_cache()
    encoder = encoder_timing()
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline()
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (N(0,1) frames, seeded random-init weights, "
                                                      "seeded uniforms)",
        "config": {"workload": "gspo_rollout", "sequences": B, "prefixes": PREFIXES, "group": GROUP,
                   "prefix_frames": P, "new_tokens": NEW, "vocab": 7, "layers": 8, "d_model": 512,
                   "heads": "8q/2kv x 64", "temperature": 1.0, "prefill_batch": args.prefill_batch,
                   "prefix_kv_shared_by": args.group_size,
                   "parallelism": "single GPU"},
        "prefill_ms": round(prefill_ms, 2), "decode_ms": round(decode_ms, 2),
        "decode_roofline_ms": round(dec_roof, 1), "decode_hbm_frac": round(dec_roof / decode_ms, 4),
        "prefill": prefill_obj,
        "live_tokens_per_rollout": live,
        "roofline": {"kernel": attn_kernels,
                     "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "avg_launch_us": round(avg_s * 1e6, 2),
                     "alg_bytes_per_launch": int(alg_bytes),
                     "timing": "inside the captured decode step: device timestamp nodes right before and after each "
                               "layer's attention launch, less the dispatch gap of a back-to-back pair, read at 32 "
                               "evenly spaced steps of a rollout",
                     "eager_avg_launch_us": round(eager_s * 1e6, 2),
                     "eager_frac": round(eager_bytes / eager_s / 1e9 / HBM_PEAK_GBS, 4),
                     "eager_timing": "HIP events over eager calls at the same steps' lengths, rotating over the 8 "
                                     "layers' caches",
                     "warm_avg_launch_us": round(warm_s * 1e6, 2),
                     "warm_frac": round(warm_bytes / warm_s / 1e9 / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
        "configs": configs,
        "gspo_reward": reward,
        "gspo_update": update,
        "encoder": encoder,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
