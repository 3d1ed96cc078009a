"""CPU oracle for the ColabFold legacy-kernel hot path: TEST INFRASTRUCTURE ONLY.

This package restates, in float64 numpy, what the reference's attention and fused pair-stack
kernels compute, so that the gfx950 HIP path can be checked against it on identical inputs.
Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it,
and there only as the checker (or, for `cpu_baseline`, as the timed CPU port). The product
path (`colabfold_legacy_kernels.hip`) never imports it and has no CPU fallback.

Modules:
  attention  flash-attention forward / backward / packed-gated-trim semantics
             (reference cuda/volta_mma_attn.cu, cuda/volta_mma_attn_bwd.cu, cuda/volta_attn.h,
             tests/test_attn_bwd.py, tests/test_packed_attention.py)
  fused      LayerNorm-fused pair-stack projections and the keep / padding rule
             (reference cuda/volta_gdp.h, cuda/volta_ops.cu, cuda/volta_fused_ffi.h)
  cpu_ref    the same attention and fused math in torch-CPU float32 (the stand-in for the
             reference tests' jnp ops on XLA-CPU, which cannot run here: jax is absent)

How each function is pinned (checked against something other than a retyping of itself) is
listed in each module's header; tests/test_oracle_*.py hold those checks.
"""
