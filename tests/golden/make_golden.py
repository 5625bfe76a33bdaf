"""Writes the golden fixtures in this directory from the CPU oracle (fp64).

    python tests/golden/make_golden.py

Fixtures (small, regenerable from seeds):
  tmu_small.npz    TMU updates at L in {1, 2, 5, 17}, C = c = 128, both directions, with and
                   without a random pair mask; inputs are identified by seed and by the sha256 of
                   their bytes (the tests regenerate them and check the hash), outputs stored fp32.
  tmu_L76.json     the fp32 plumbing workload (outgoing only, z [1,76,76,128] N(0,1), seed 0):
                   sha256 of the fp32 output bytes, RMS, and a few slices.
  q8_small.npz     q8 inputs at M=4, K=128, N=64 and the exact dequantised weights as fp16 and
                   fp32 bit patterns, plus y = x . W^T in fp64.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import q8, tmu  # noqa: E402

TMU_LS = (1, 2, 5, 17)


def sha(t) -> str:
    a = t.numpy() if isinstance(t, torch.Tensor) else t
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def tmu_case(L: int, outgoing: bool, masked: bool):
    """Seeded inputs for one small TMU case (fp16 z, fp32 master weights, fp16 0/1 mask)."""
    seed = 1000 + 10 * L + 2 * int(outgoing) + int(masked)
    z, _, po, pi = tmu.make_pair_inputs(L, 128, 128, seed=seed, dtype=torch.float16, B=1)
    p = po if outgoing else pi
    mask = None
    if masked:
        g = torch.Generator().manual_seed(seed + 7)
        mask = (torch.rand(1, L, L, generator=g, dtype=torch.float32) > 0.3).to(torch.float16)
    return seed, z, mask, p


def main():
    out = {}
    for L in TMU_LS:
        for outgoing in (True, False):
            for masked in (False, True):
                seed, z, mask, p = tmu_case(L, outgoing, masked)
                with torch.no_grad():
                    y = tmu.trimul(z.double(), None if mask is None else mask.double(), p.to(torch.float64), outgoing)
                key = f"L{L}_{'out' if outgoing else 'in'}_{'mask' if masked else 'nomask'}"
                out[key + "_y"] = y.float().numpy()
                out[key + "_zsha"] = np.array(sha(z.view(torch.int16)))
                out[key + "_wsha"] = np.array(sha(p.w_bundle))
                out[key + "_seed"] = np.array(seed)
    np.savez_compressed(os.path.join(HERE, "tmu_small.npz"), **out)

    z, _, po, _ = tmu.make_pair_inputs(76, 128, 128, seed=0, dtype=torch.float32)
    with torch.no_grad():
        y = tmu.trimul(z.double(), None, po.to(torch.float64), True).float()
    summary = {
        "workload": "TMU outgoing, z [1,76,76,128] fp32 N(0,1), seed 0, all-ones mask, weights N(0,1/fan_in)",
        "z_sha256": sha(z), "w_bundle_sha256": sha(po.w_bundle),
        "y_sha256_fp32": sha(y), "y_rms": float(y.double().pow(2).mean().sqrt()),
        "y_0_0_0_8": y[0, 0, 0, :8].tolist(), "y_75_75_120_128": y[0, 75, 75, 120:].tolist(),
        "y_37_11_64_72": y[0, 37, 11, 64:72].tolist(),
    }
    with open(os.path.join(HERE, "tmu_L76.json"), "w") as f:
        json.dump(summary, f, indent=1)

    x, qq, s, b = q8.make_q8_inputs(4, 128, 64, seed=7)
    np.savez_compressed(os.path.join(HERE, "q8_small.npz"), x=x, q=qq, s=s, b=b,
                        w16=q8.dequant_f16(qq, s, b).view(np.uint16), w32=q8.dequant_f32(qq, s, b).view(np.uint32),
                        y=q8.q8_linear(x, qq, s, b))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
