"""CPU oracle for the triangle multiplicative update, the pair trunk and the 8-bit ESMC linear.

THIS PACKAGE IS TEST INFRASTRUCTURE. It is a CPU restatement of the reference's
arithmetic, used only to verify results: by ``tests/``, by
``__graft_entry__.smoke()`` and by ``bench.py``'s ``cpu_baseline`` leg. The
product path (the HIP kernels behind the C ABI in ``esmfold2-mlx_amd/``) never
imports, calls or falls back to anything here.

Modules:
  tmu        -- the triangle multiplicative update (outgoing / incoming), the
                contraction, LayerNorm, the pair driver, the block stack.
  q8         -- MLX-affine 8-bit group-64 dequantisation and the q8 linear.
  transition -- the pair transition (ReLU MLP, and the reference's SwiGLU).
  recycle    -- the parcae recycling step, the distogram expected distance and the
                p95 exit signal.
  esmc       -- the ESMC transformer block around the 8-bit linear (QK-LayerNorm,
                NeoX RoPE, chain-masked attention, SwiGLU, scaled residuals).

Every function cites the reference file:line it restates. Paths are relative
to the reference repository root (abhi0raj/esmfold2-mlx).

How each function is pinned (checks that would fail on a dropped term, a wrong
sign or index, or a transposed operand) is listed in each module's header and
exercised by tests/test_oracle_*.py.
"""
