"""CPU oracle for the Qwen3 decode step -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``tilefoundry_amd``) imports this package. It is imported
only by ``tests/``, by ``__graft_entry__.smoke()`` as the checker, and by
``bench.py``'s ``cpu_baseline`` leg, where it is timed as the reference CPU path.

What it is: a plain-torch, CPU-only restatement of the authored HIR that the
reference's Qwen3-1.7B runtime is measured against
(``examples/qwen3_1_7b-tilelang/ref_src/model.py:107-387``), run the way the
reference evaluator runs it: every ``@func`` body op for op, each op at the dtype
the HIR declares, each op's value given by the torch call the evaluator's handler
makes (``src/tilefoundry/ir/hir/**``, handlers cited per function).  The greedy
loop restates ``ref_src/generation.py:24-85``.

How it is pinned (each check lives in ``tests/test_oracle_*.py``):

* f32 mode against Hugging Face ``Qwen3ForCausalLM`` built offline from a config
  dict with the same weights, full-sequence causal forward, every position --
  this fixes the RMSNorm order, RoPE, GQA grouping, SwiGLU, residual thread and
  the tied head (a dropped term, a wrong sign or a transposed operand fails it);
* attention against an f64 brute-force softmax (``fast/arbitrate.py:22-56``);
* ``argmax`` tie rule (first maximal index, constant row -> 0), as
  ``tests/ops/test_argmax.py:70-73`` and ``fast/kernels.py:303-306`` state;
* RoPE against the closed-form rotation and its norm-preservation invariant;
* paged-cache indexing against the contiguous cache under page permutations.

The bf16 mode is the same code at a different dtype: the rounding points are the
HIR's casts, and CPU torch decides each op's bf16 result as the evaluator would.
Where that can only be pinned by running the reference evaluator itself (whole
fused bf16 chains, bit for bit), parity is "unpinned" by import -- the reference
cannot be imported in this environment -- and is bounded by the f64 checks.
"""
