"""esmfold2-mlx_amd: ESMFold2's triangle multiplicative update and 8-bit ESMC linear
as hand-written gfx950 (MI355X) HIP kernels behind a C ABI (include/esmfold2_amd.h).

Modules:
  build            -- compile libesmfold2_amd.so in-tree with hipcc (gfx950)
  capi             -- ctypes binding of the C ABI; raises, never falls back
  kernels          -- one functional wrapper per C entry point (torch tensors in/out)
  trimul           -- TriMul / TriMulPair: the forward(pair_grid, visibility) module contract
  q8               -- Q8Linear: the quantized_matmul(transpose=True, group 64, bits 8) contract
  esmc             -- EsmcBlock and HipEsmc: the ESMC language model around the 8-bit linear
  trunk            -- PairTransition, TrunkBlock and PairTrunk (the FoldingTrunk drop-in)
  recycle          -- ParcaeLoop (the 6B recycling loop) and its distogram exit signal
  var_hip_trimul   -- the reference-style variant plugin for the TMUs: apply(model)
  var_hip_trunk    -- the variant plugin replacing the whole folding trunk: apply(model)
  var_6b_hip_trunks -- the variant plugin replacing all four trunk stacks of the 6B model
  var_6b_hip_loop  -- the variant plugin installing the 6B parcae recycling loop (optional early exit)
  var_6b_hip_adaptive -- that loop with the reference's early-exit policy
  var_hip_adaptive_loops -- adaptive recycling of the folding trunk (AdaptiveTrunk)
  scratch          -- the device scratch buffer every module shares
  variants         -- apply_variants(model, names): the plugins by name, in order
  workloads        -- seeded synthetic inputs of the benchmark configurations
"""

from . import build, capi  # noqa: F401

__all__ = ["build", "capi", "kernels", "trimul", "q8", "esmc", "trunk", "recycle", "scratch", "var_hip_trimul",
           "var_hip_trunk", "var_6b_hip_trunks", "var_6b_hip_loop", "var_6b_hip_adaptive", "var_hip_adaptive_loops",
           "variants", "workloads"]


def __getattr__(name):
    if name in __all__[2:]:
        import importlib
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
