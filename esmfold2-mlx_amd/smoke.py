"""One small run of each hot path on cuda:0, checked against the CPU oracle.

Imports the oracle (test infrastructure) only as the checker; the computation is
the HIP library's.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch


def _oracle():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if root not in sys.path:
        sys.path.insert(0, root)
    from oracle import q8 as oq8, tmu as otmu
    return otmu, oq8


def run() -> None:
    from .q8 import Q8Linear
    from .trimul import TriMul, TriMulPair

    otmu, oq8 = _oracle()
    assert torch.cuda.is_available(), "smoke needs a GPU"
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    # TMU pair, L=40 (one partial cell tile, one contraction tile), padded mask
    z, mask, po, pi = otmu.make_pair_inputs(40, 128, 128, seed=0, dtype=torch.float16, pad_from=33)
    pair = TriMulPair(TriMul.from_weights(po, device=dev), TriMul.from_weights(pi, device=dev))
    got = pair(z.to(dev), mask.to(dev)).float().cpu().double()
    ref = otmu.trimul_pair(z.double(), mask.double(), po.to(torch.float64), pi.to(torch.float64))
    err = float((got - ref).abs().max())
    rms = float((ref - z.double()).pow(2).mean().sqrt())  # RMS of the summed updates
    print(f"[smoke] TMU pair L=40 max|err| {err:.3e}  RMS(update) {rms:.3e}", flush=True)
    assert np.isfinite(err) and err <= 1e-2 * rms, "TMU pair differs from the oracle"

    # q8 linear
    x, q, s, b = oq8.make_q8_inputs(37, 256, 128, seed=0)
    lin = Q8Linear(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(b), device=dev)
    y = lin(torch.from_numpy(x).to(dev)).float().cpu().numpy().astype(np.float64)
    yr = oq8.q8_linear(x, q, s, b)
    rel = float(np.linalg.norm(y - yr) / np.linalg.norm(yr))
    w16 = lin.dequantized().cpu().numpy()
    exact = bool(np.array_equal(w16.view(np.uint16), oq8.dequant_f16(q, s, b).view(np.uint16)))
    print(f"[smoke] q8 linear rel err {rel:.3e}, dequant bit-exact {exact}", flush=True)
    assert rel <= 1e-3 and exact, "q8 linear differs from the oracle"
    torch.cuda.synchronize()
    print("[smoke] ok", flush=True)
