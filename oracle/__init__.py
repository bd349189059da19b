"""CPU oracle of the decoder rollout-and-scoring path -- TEST INFRASTRUCTURE, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker (or, for the CPU baseline, as the timed CPU restatement of the reference). The product
(viktor_amd) never imports it and has no CPU fallback.

oracle.reference restates, in PyTorch on the CPU:
  viktor/decoder.py (all), viktor/encoder.py:30-40 (rope tables), viktor/engine.py (the torch-backend
  state machine, _select), viktor/model.py:55-85 (teacher-forced logits), scripts/gspo.py:340-353 and
  446-477 (token log-probs, advantages, sequence ratio, clipped loss and its gradient),
in two numerics modes: "fp32" (the reference's fp32 semantics) and "fused" (bf16 storage between ops,
fp32 inside each op: the rounding points of viktor/triton_ops.py / the HIP kernels).

How each part is pinned (see tests/test_oracle.py):
  * decoder forward, engine greedy streams, teacher-forced logits, rope tables, tokenizer: golden vectors
    written by importing the reference's CPU path (tests/golden/make_golden.py);
  * RMSNorm / RoPE / attention / SwiGLU: closed forms and fp64 brute force on small inputs;
  * cached decode == full recompute (the reference's own invariant, tests/test_viktor.py:71-83);
  * inverse-CDF sampling from supplied uniforms (no reference counterpart: the reference samples with
    device Gumbel noise): closed-form boundary cases and a frequency test;
  * GSPO ratio / loss / gradient: torch autograd of the restated loss, closed form, special cases.
"""
