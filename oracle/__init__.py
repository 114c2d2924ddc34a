"""CPU oracle for the masked-component hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy (float64 unless a function says otherwise) and in a
small C library (`oracle/cpu_step.c`), the arithmetic of goodfire-ai/param-decomp's
masked-component path. Every function cites the reference file:line it follows.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may import
it, and only to check results (or as the timed CPU baseline). The product path
(`param_decomp_amd`) never imports it and fails loudly when its HIP library is missing.

Pinning (what checks each function besides a retyped formula):
- `threefry.threefry2x32`: Random123 known-answer vectors (Salmon et al., SC'11).
- `threefry` key chain, original layout: the published JAX documentation value of
  `split(PRNGKey(0))`.
- `threefry` key chain, partitionable layout: `split(k)[i] == fold_in(k, i)` and the
  Random123 vector at key (0,0), counter (0,0).
- `threefry.uniform`, fp32 and partitionable: the reference's stored fp32
  `jax.random.uniform` draws under `split(PRNGKey(3), 9)`
  (`param_decomp/param_decomp/tests/targets/stacked_parity/gen_stacked_fixtures.py:102`),
  bit for bit. The bf16 conversion (8 bits drawn, top 7 kept) is restated from JAX's
  published `_uniform`; no JAX is importable here and no stored bf16 draw exists, so the
  bf16 draw is "parity unpinned" against JAX beyond the range and grid checks.
- `moe_oracle`: finite differences of its hand-written backward and the every-expert
  dense spelling of a routed layer.
- squashing VJPs: the reference's 10 known-answer cotangents.
- smooth-L0 imp-min: the reference's closed-form tests.
- gate MLP, p-norm imp-min, masked linear and its backward: finite differences and
  brute-force loops on tiny inputs.
- routing / bucketing / grouped matmuls: the reference's routed-expert fixtures (E=8,
  K=2, T=24 with two empty experts; ragged dW sizes [7,0,19,1,0,26,37,0]) against dense
  brute force.
"""
