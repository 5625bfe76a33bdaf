"""bench.py's contract pieces that need no GPU: the one-GPU guard and the committed counter
summary it reads for ``roofline.traffic``."""

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_counter_summary_has_every_tmu_kernel():
    import bench

    t = bench.measured_traffic()
    for k in ("tmu_project_kernel", "tmu_contract_frag_kernel", "tmu_epilogue_kernel"):
        # one TMU launch moves 43.5 MB algorithmically; the measured traffic stays within 15% of it
        assert 0.95 * 43.5e6 < t[k] < 1.15 * 43.5e6, (k, t.get(k))


def test_kernel_trace_gives_each_tmu_kernel_a_mean():
    import bench

    # the line's roofline.profile_us is read from the committed trace at the L=238 grids
    for name, grid in (("esm::tmu_project_kernel<false, true>", 131072), ("esm::tmu_contract_frag_kernel", 131072),
                       ("esm::tmu_epilogue_kernel<false, true>", 121856)):
        us = bench.profiled_mean_us(name, grid)
        assert us is not None and 5.0 < us < 40.0, (name, us)
