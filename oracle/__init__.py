"""CPU oracle for the chain-flow drafting hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``chain-flow_amd/``) imports, links or calls
anything under ``oracle/``; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, and only as the reference results are compared against or as the timed
CPU baseline, never as the thing measured or shipped.

It is a plain numpy restatement of the reference algorithm (Cosmos-YTU/chain-flow), one module per
part of the path, each function citing the reference ``file:line`` it follows (``cf/`` =
``src/chain_flow/``):

* ``flow``   -- ``TreeFlowDrafter.predict_hidden`` over ``HiddenKVFlowExpert`` chunk experts
  (init_latents, Euler integrate, pre_blocks / HiddenKVFlowBlock x L / post_blocks).
* ``head``   -- shortlisted lm_head, markov bias, fused path residual, log-softmax, top-k.
* ``beam``   -- ``_beam_chains`` / ``_beam_tree`` beam search and backtrack.
* ``gdn``    -- tree gated-delta-net recurrence and the sequential per-path reference.

Numerics. Every function computes in float64 (``prec``) and rounds to fp16 exactly where the
drafter's fp16 path materialises a tensor that the next op consumes (``numerics="fp16"``), or
nowhere (``numerics="fp32"``, the reference's fp32 CPU plumbing).  Inside the block stack the
residual stream is kept unrounded, as the reference's fused block kernel does
(``cf/csrc/fused_block.cu:517-520, 564, 658``): LayerNorm inputs are parked as fp16 before the
statistics (``fused_block.cu:291-304``), q/k/v, attention outputs and GELU outputs are fp16.

How each part is pinned (beyond the golden vectors under ``tests/golden/`` made from the
reference itself): see ``tests/test_oracle_*.py``.  Closed forms (init_latents, zero velocity,
identity head rows, single-node GDN step, beta=0 decay), library identities (attention against a
brute-force per-head loop, LayerNorm against its definition), invariants (causality of the
self-attention mask, context-row permutation invariance of cross-attention, chunk independence,
tree == per-path sequential recurrence) and brute-force beam enumeration on tiny vocabularies.
"""
