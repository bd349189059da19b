"""Greedy or sampled decoding of variable-length prefixes on the HIP kernels: static KV cache, packed
prefill with a BOS-only last layer, one captured HIP graph per decode step.

Call surface and state machine of viktor/engine.py:31-220 (DecodeEngine). Each sequence's prefix is its
projected encoder frames + BOS, so every sequence decodes at its own position; finished sequences keep
running and emit PAD, which keeps every step shape-static and graph-capturable. A step is
  embed + RMSNorm -> 8 decoder layers -> fused LM head + token choice + grammar + state update,
with all state in preallocated device tensors and no host synchronisation inside the step.

Sampling (temperature > 0) draws each token from softmax(logits / T) by the inverse CDF at one uniform
per (sequence, output column): `uniforms` [B, max_new_tokens]; or, with sampling="gumbel", by the
reference's own Gumbel-max formula at one uniform per (sequence, output column, vocabulary entry):
`uniforms` [B, max_new_tokens, V]. The reference draws those uniforms from the device RNG inside its graph
(viktor/engine.py:80-83); here the engine fills the uniforms from the torch RNG at prefill unless the caller
supplied them (set_uniforms), which makes a rollout reproducible.

group_size = G > 1 (GSPO rollouts: each window repeated G times, scripts/gspo.py:444): consecutive groups
of G sequences must have identical prefixes (checked at prefill). The engine then prefills each window
once into a prefix cache [L, B / G, max_frames + 1, Hkv, D] and keeps only the sampled tokens per sequence
in `cache` [L, B, max_new_tokens, Hkv, D]; decode attention reads each prefix row once per group. Token
streams are those of the ungrouped engine up to the attention's summation order (prefix and suffix are
reduced separately, then merged).
"""

import torch

from . import _lib, hip_ops as ops
from ._lib import HipLibraryError, call, ptr
from .decoder import KVCache
from .fast_decoder import FastDecoder, PrefillPlan
from .tokenizer import BOS, EOS, PAD


class DecodeEngine:
    # unused rows after each sequence's rows (KVCache pad_rows) in the grouped layout's prefix and own-token
    # caches: at the rollout's shape the per-sequence strides become 2144 x 256 B (536 KiB) and 1056 x 256 B
    # (264 KiB) instead of 512 KiB + 256 B and 256 KiB
    PREFIX_PAD_ROWS = 95
    OWN_PAD_ROWS = 32

    def __init__(self, model, batch_size: int, max_new_tokens: int, max_frames: int, backend: str = "auto",
                 cuda_graph: bool = True, prefill_batch: int = 128, check_every: int = 32,
                 attention_backend: str = "auto", temperature: float = 0.0, max_homopolymer=64, group_size: int = 1,
                 logprobs: bool = False, force_eos_last: bool = False, sampling: str = "inverse_cdf"):
        self.model, self.dec = model, model.decoder
        self.temperature = float(temperature)
        # force_eos_last: the last output column (max_new_tokens - 1) is EOS for every sequence still running when
        # it is produced (a rollout capped at max_new_tokens ends with EOS); off by default, as the reference
        # scores a call that never ends as it stands (scripts/gspo.py:24-25)
        self.force_eos_last = bool(force_eos_last)
        # sampling (temperature > 0): "inverse_cdf" -- one uniform per (sequence, output column) through the CDF of
        # softmax(logits / T); "gumbel" -- the reference's formula, argmax(logits / T - log(-log(u))) with one uniform
        # per (sequence, output column, vocabulary entry), viktor/engine.py:80-83
        if sampling not in ("inverse_cdf", "gumbel"):
            raise ValueError(f"unknown sampling {sampling!r}: 'inverse_cdf' or 'gumbel'")
        self.gumbel = sampling == "gumbel"
        dev = self.dec.lm_head.weight.device
        self.dtype = self.dec.lm_head.weight.dtype
        self.pos_scale = getattr(model, "pos_scale", 1)
        if backend not in ("auto", "hip", "triton"):
            raise ValueError(f"unknown backend {backend!r}: this engine runs the HIP kernels ('auto' / 'hip')")
        if dev.type != "cuda" or torch.version.hip is None:
            raise HipLibraryError("DecodeEngine runs on a ROCm GPU (the model is on %s)" % dev)
        if self.dtype != torch.bfloat16:
            raise AssertionError("DecodeEngine needs the bf16 inference copy of the model (see gspo.bf16_copy)")
        self.backend = "hip"
        self.fast = FastDecoder(self.dec, attention_backend=attention_backend)
        self.B, self.max_new = batch_size, max_new_tokens
        self.prefill_batch, self.check_every = prefill_batch, check_every
        self._prefill_plans = {}
        max_len = max_frames + 1 + max_new_tokens
        assert max_len <= self.dec.cfg.max_seq_len
        self.max_frames = max_frames
        self.G = int(group_size)
        assert self.G >= 1 and batch_size % self.G == 0, "batch_size must be a multiple of group_size"
        if self.G == 1:
            self.cache = KVCache(self.dec.cfg, batch_size, max_len, self.dtype, dev)
            self.prefix_cache = None
        else:
            self.prefix_cache = KVCache(self.dec.cfg, batch_size // self.G, max_frames + 1, self.dtype, dev,
                                        pad_rows=self.PREFIX_PAD_ROWS)
            self.cache = KVCache(self.dec.cfg, batch_size, max(max_new_tokens, 2), self.dtype, dev,
                                 pad_rows=self.OWN_PAD_ROWS)
            self.prefix_len32 = torch.ones(batch_size // self.G, dtype=torch.int32, device=dev)
            self.cache_base = torch.zeros(batch_size, dtype=torch.long, device=dev)  # own-token row = pos - base
            self.grouped_workspace = ops.decode_attention_grouped_workspace(batch_size, self.G, max_frames + 1,
                                                                            self.cache.max_len, dev)

        self.tok = torch.full((batch_size,), BOS, dtype=torch.long, device=dev)
        self.pos = torch.zeros(batch_size, dtype=torch.long, device=dev)
        self.rope_off = torch.zeros(batch_size, dtype=torch.long, device=dev)  # RoPE position - cache position
        self.pos32 = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self.rpos32 = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self.seqlens = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self.rows = torch.arange(batch_size, dtype=torch.int32, device=dev)
        self.step_idx = torch.zeros(1, dtype=torch.long, device=dev)
        self.out = torch.full((batch_size, max_new_tokens), PAD, dtype=torch.long, device=dev)
        self.bos = torch.tensor([BOS], device=dev)
        tk = model.tokenizer
        self.bias = torch.zeros(tk.vocab_size, device=dev)
        self.bias[[PAD, BOS]] = float("-inf")
        self.is_tail = tk.tail_mask.to(dev)
        self.is_homo = torch.tensor([i >= 3 and len(t) == tk.k and len(set(t)) == 1 for i, t in enumerate(tk.strings)],
                                    device=dev)
        self.homo_stop = max_homopolymer // tk.k if max_homopolymer else 0  # run length in tokens that ends it
        self.run = torch.zeros(batch_size, dtype=torch.long, device=dev)
        self.plen = torch.zeros(batch_size, dtype=torch.long, device=dev)  # output column = pos - plen
        u_shape = (batch_size, max_new_tokens) + ((tk.vocab_size,) if self.gumbel else ())
        self.uniforms = torch.zeros(u_shape, dtype=torch.float32, device=dev)
        self._uniforms_set = False
        # logprobs=True: logp[b, j] = log-probability of output token j under the distribution it was chosen
        # from (log softmax of (logits + bias) / T, or of logits + bias when greedy), before the grammar rules
        self.logp = torch.zeros(batch_size, max_new_tokens, dtype=torch.float32, device=dev) if logprobs else None
        self.fast.decode_workspace = ops.decode_attention_workspace(batch_size, self.dec.cfg.n_heads,
                                                                    self.cache.max_len, dev)
        self.graph = None  # one captured step
        self.graph_multi = None  # check_every captured steps: one replay, no launch gaps between its steps
        if cuda_graph:
            self._capture()

    # ---- one decode step -----------------------------------------------------------------------
    def _step(self):
        # layers on the fused small-M kernels; the LM-head kernel applies the final norm, chooses the token
        # (greedy from fp32 logits, sampled from bf16 logits: the reference's two step kinds) and advances
        # the state. step_idx is advanced on the host after the replays (it is not read inside a step).
        if self.G == 1:
            x = self.fast.decode_residual(self.pos32, self.rows, self.seqlens, self.cache,
                                          rope_pos=None if self.pos_scale == 1 else self.rpos32, tok=self.tok)
        else:  # pos32 / seqlens index the own-token cache; RoPE runs at the absolute position rpos32
            x = self.fast.decode_residual(self.pos32, self.rows, self.seqlens, self.cache, rope_pos=self.rpos32,
                                          tok=self.tok, prefix=(self.prefix_cache, self.prefix_len32, self.G,
                                                                self.grouped_workspace))
        ops.select_update(self.bias, self.is_tail, self.is_homo, self.homo_stop, self.tok, self.run, self.pos,
                          self.plen, self.rope_off, self.out, self.pos32, self.seqlens, self.rpos32, EOS, PAD,
                          h=x, norm_w=self.dec.norm.weight, eps=self.dec.cfg.norm_eps, w_head=self.dec.lm_head.weight,
                          round_bf16=self.temperature > 0, temperature=self.temperature, uniforms=self.uniforms, gumbel=self.gumbel,
                          cache_base=None if self.G == 1 else self.cache_base, logp_out=self.logp)

    def _reset_state(self):
        self.pos.fill_(1)
        self.pos32.fill_(1)
        self.seqlens.fill_(2)
        self.rpos32.fill_(1)
        self.tok.fill_(BOS)
        self.step_idx.zero_()

    @torch.no_grad()
    def _capture(self):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                self._reset_state()
                self._step()
        torch.cuda.current_stream().wait_stream(s)
        self._reset_state()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        if self.check_every > 1:  # the steps between two early-exit checks, back to back in one graph
            self.graph_multi = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph_multi, pool=self.graph.pool()):
                for _ in range(self.check_every):
                    self._step()
        self.out.fill_(PAD)

    # ---- prefill -------------------------------------------------------------------------------
    def _packing(self, lens, row0, cache, dev):
        """Index layout of one prefill sub-batch, built on the host from the frame counts and uploaded once
        (the engine keeps it while the sub-batch's lengths repeat). Sequence j occupies packed rows
        [s_j, s_j + lens[j] + 1): its frames, then BOS in the last row; every row carries its cache position
        (0 .. lens[j]), cache row (row0 + j) and RoPE position (position * pos_scale)."""
        import numpy as np
        n = len(lens)
        seq_lens = [L + 1 for L in lens]
        plan = PrefillPlan(seq_lens, dev, rows=list(range(row0, row0 + n)), keep=[1] * n, cache=cache)
        starts = np.asarray(plan.cu[:-1], dtype=np.int64)
        within = np.concatenate([np.arange(m, dtype=np.int64) for m in seq_lens])  # position inside the sequence
        owner = np.repeat(np.arange(n, dtype=np.int64), seq_lens)                  # sequence of each packed row
        is_frame = within < np.repeat(np.asarray(lens, dtype=np.int64), seq_lens)
        frame_rows = (starts[owner] + within)[is_frame]                             # where frame rows land
        bos_rows = starts + np.asarray(lens, dtype=np.int64)

        def up(a, dt):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device=dev, dtype=dt)

        pos = up(within, torch.int32)
        rpos = None if self.pos_scale == 1 else up(within * self.pos_scale, torch.int32)
        return plan, up(frame_rows, torch.long), up(bos_rows, torch.long), pos, up(owner + row0, torch.int32), rpos

    def _prefill_hip(self, prefix, lens, row0, cache):
        """Packs the projected frames prefix [sum(lens), d] of cache rows row0.. with a BOS row after each
        sequence, runs the layers (the last one for the BOS rows only) and returns the final-normed hidden
        state of each BOS row [len(lens), d]."""
        dev = prefix.device
        key = tuple(lens)
        cached = self._prefill_plans.get(row0)
        if cached is None or cached[0] != key:
            cached = key, self._packing(lens, row0, cache, dev)
            self._prefill_plans[row0] = cached
        plan, frame_rows, bos_rows, pos, seq, rpos = cached[1]
        x = torch.empty(plan.total, prefix.shape[1], dtype=self.dtype, device=dev)
        if len(set(lens)) == 1:  # equal lengths: the frame rows and the BOS rows are two strided views
            n, L = len(lens), lens[0]
            xv = x.view(n, L + 1, -1)
            xv[:, :L].copy_(prefix.view(n, L, -1))
            xv[:, L] = self.dec.embed.weight[BOS].to(self.dtype)
        else:
            x.index_copy_(0, frame_rows, prefix)
            x[bos_rows] = self.dec.embed.weight[BOS].to(self.dtype)
        return self.fast.prefill(x, pos, seq, None, plan.max_len, cache, rope_pos=rpos, plan=plan)

    def set_uniforms(self, u):
        """Uniforms in [0, 1) driving the sampled tokens (column j -> output token j): [B, max_new_tokens], or
        [B, max_new_tokens, vocab] with sampling="gumbel"."""
        assert u.shape == self.uniforms.shape
        self.uniforms.copy_(u)
        self._uniforms_set = True

    @torch.no_grad()
    def prefill(self, frames, frame_lens):
        """Encodes every sequence's prefix into the KV cache and picks its first output token.

        frames: the B windows' encoder frames stacked along dim 0 ([sum(frame_lens), d_enc]); frame_lens: B
        frame counts. Windows go through the projector and the decoder in sub-batches of prefill_batch; the
        first token comes from the BOS row's bf16-rounded logits (viktor/engine.py:191 rounds them the same
        way) and lands in out[:, 0]; the decode state then points at position frame_lens[b] + 1."""
        frame_lens = [int(n) for n in frame_lens]
        assert len(frame_lens) == self.B and frames.shape[0] == sum(frame_lens)
        assert all(0 < n <= self.max_frames for n in frame_lens), "frame count outside 1..max_frames"
        if self.temperature > 0 and not self._uniforms_set:
            self.uniforms.uniform_()
        self._uniforms_set = False
        offs = [0]
        for n in frame_lens:
            offs.append(offs[-1] + n)
        G = self.G
        if G > 1:  # one prefill per window: the first sequence of every group
            self._check_groups(frames, frame_lens, offs)
            lens_p = frame_lens[::G]
            # each group's first member's frames, gathered and converted to the compute dtype in one pass
            if len(set(frame_lens)) == 1:
                n = frame_lens[0]
                frames_p = frames.view(self.B // G, G, n, -1)[:, 0].to(self.dtype).reshape(-1, frames.shape[1])
            else:
                frames_p = torch.cat([frames[offs[b]:offs[b + 1]].to(self.dtype) for b in range(0, self.B, G)])
            offs_p = [0]
            for n in lens_p:
                offs_p.append(offs_p[-1] + n)
            cache, n_rows = self.prefix_cache, len(lens_p)
        else:
            frames_p, lens_p, offs_p, cache, n_rows = frames, frame_lens, offs, self.cache, self.B
        last = []
        for lo in range(0, n_rows, self.prefill_batch):
            hi = min(n_rows, lo + self.prefill_batch)
            prefix = self.model.projector(frames_p[offs_p[lo]:offs_p[hi]].to(self.dtype))
            last.append(self._prefill_hip(prefix, lens_p[lo:hi], lo, cache))
        h = torch.cat(last) if len(last) > 1 else last[0]
        if G > 1:
            h = h.repeat_interleave(G, 0)
            self.prefix_len32.copy_(torch.tensor([n + 1 for n in lens_p], dtype=torch.int32, device=h.device))
        self.tok.fill_(BOS)
        self.run.zero_()
        self.out.fill_(PAD)
        if self.logp is not None:  # columns past an early stop read 0, as out reads PAD there
            self.logp.zero_()
        self.plen.copy_(torch.tensor(frame_lens, device=self.pos.device))
        self.pos.copy_(self.plen)  # the select kernel writes column pos - plen = 0, then advances pos to plen + 1
        if G > 1:
            self.cache_base.copy_(self.plen + 1)  # the first sampled token goes to own-token row 0
        self.rope_off.copy_(self.plen * (self.pos_scale - 1))
        ops.select_update(self.bias, self.is_tail, self.is_homo, self.homo_stop, self.tok, self.run, self.pos,
                          self.plen, self.rope_off, self.out, self.pos32, self.seqlens, self.rpos32, EOS, PAD,
                          h=h.contiguous(), w_head=self.dec.lm_head.weight, round_bf16=True,
                          temperature=self.temperature, uniforms=self.uniforms, gumbel=self.gumbel,
                          cache_base=None if G == 1 else self.cache_base, logp_out=self.logp)
        self.step_idx.fill_(1)

    def _check_groups(self, frames, frame_lens, offs):
        """Every group of G consecutive sequences must carry the same prefix (lengths and frames)."""
        G = self.G
        for b in range(0, self.B, G):
            if any(frame_lens[b + m] != frame_lens[b] for m in range(G)):
                raise ValueError(f"group_size={G}: sequences {b}..{b + G - 1} have different prefix lengths")
        member_bytes = frame_lens[0] * frames.shape[1] * frames.element_size()
        if (len(set(frame_lens)) == 1 and frames.is_contiguous() and member_bytes % 16 == 0
                and frames.data_ptr() % 16 == 0):
            # equal lengths: one pass comparing each member with its group's first, bit for bit
            flag = torch.zeros(1, dtype=torch.int32, device=frames.device)
            call("vk_group_rows_equal", ptr(frames), self.B // G, G, member_bytes, ptr(flag), _lib.stream_handle())
            if int(flag.item()) != 0:
                raise ValueError(f"group_size={G}: the sequences of a group must share their prefix frames")
            return
        dev = frames.device
        lens = torch.tensor(frame_lens, device=dev)
        rows = torch.repeat_interleave(torch.arange(self.B, device=dev), lens, output_size=frames.shape[0])
        start = torch.tensor(offs[:-1], device=dev)
        lead = torch.div(rows, G, rounding_mode="floor") * G  # first sequence of the row's group
        src = start[lead] + torch.arange(frames.shape[0], device=dev) - start[rows]
        if not torch.equal(frames, frames[src]):
            raise ValueError(f"group_size={G}: the sequences of a group must share their prefix frames")

    @torch.no_grad()
    def decode(self, steps=None):
        """Continues every sequence after prefill and returns `out` [B, max_new_tokens].

        With steps=n the engine replays exactly n - 1 steps, so out[:, :n] holds n tokens per sequence
        (1 <= n <= max_new_tokens). With steps=None it runs up to max_new_tokens tokens and stops early once
        every sequence has emitted EOS (looked at after each check_every steps)."""
        if steps is not None and not 1 <= int(steps) <= self.max_new:
            raise ValueError(f"decode: steps must be in 1..max_new_tokens={self.max_new} (got {steps})")
        n = self.max_new - 1 if steps is None else int(steps) - 1
        done = 0
        while done < n:
            if self.graph_multi is not None and done % self.check_every == 0 and n - done >= self.check_every:
                self.graph_multi.replay()  # check_every steps
                done += self.check_every
            elif self.graph is not None:
                self.graph.replay()
                done += 1
            else:
                self._step()
                done += 1
            if steps is None and done % self.check_every == 0 and bool(((self.tok == EOS) | (self.tok == PAD)).all()):
                n = done
                break
        self.step_idx.add_(n)
        if self.force_eos_last and n == self.max_new - 1:
            # the last column holds a token only where the sequence was still running (PAD after its EOS
            # otherwise): that token becomes EOS
            last = self.out[:, self.max_new - 1]
            last.masked_fill_(last != PAD, EOS)
        return self.out

    def generate(self, frames, frame_lens, steps=None):
        """prefill + decode. The returned [B, max_new_tokens] token ids (PAD once a sequence has ended) are
        the engine's own `out` buffer, which the next call overwrites."""
        self.prefill(frames, frame_lens)
        return self.decode(steps)
