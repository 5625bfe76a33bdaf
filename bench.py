"""Benchmark: triangle multiplicative update pair cells/s at L=238, fp16, on one MI355X.

A step is one TMU pair on the pair tensor z [1, 238, 238, 128] fp16:
z1 = z + T_out(z), z2 = z1 + T_in(z1): six kernels (a, b, c per direction), inputs
resident in HBM. value = L^2 / t_step (cells/s). The timed step is the module path a
caller runs, TriMulPair -> one tmu_pair_forward call (a and b in the MFMA-fragment
layout). The per-kernel figures come from a second pass that makes the same six launches
one entry point at a time (tmu_project_frag, tmu_contract_frag, tmu_epilogue); their
output is checked to equal TriMulPair's bit for bit.

Also reported on the same JSON line:
  roofline      for the kernel with the largest share of the step (achieved =
                algorithmic bytes or flops per launch / its mean duration over a
                second pass of the timed step, from start/stop events the runtime
                stamps with each kernel's own begin and end (the durations a
                kernel trace reports); traffic = calibrated rocprofv3
                FETCH_SIZE + WRITE_SIZE per launch from profiles/);
  kernels       the same figures for every kernel of the step, and for the
                contraction its fraction of its own roof, min(MFMA peak, AI x HBM
                peak) with AI = L/3 FLOP/B by compulsory traffic;
  q8            the 8-bit ESMC-style linears [238,2560]x[2560->10240],
                [238,10240]x[10240->2560] and [238,2560]x[2560->7680] (time, TFLOP/s,
                GB/s, the output tile's weight rows the plan picked) on the weight
                layout Q8Linear keeps (codes and scales packed once per layer), the
                time with the codes in MLX's [N, K] layout beside it, and each
                launch's own duration;
  transition    the pair transition kernel (LN -> 128->512 -> ReLU -> 512->128 + z)
                at L=238 (time, TFLOP/s, fraction of MFMA peak);
  block_stack   the pair-trunk block stack at L=238: 8 blocks of (T_out, T_in,
                transition) x 3 recycles with z carried, replayed as one HIP graph;
  recycle       the recycling step's kernels at L=238: the parcae recurrence, the
                distogram expected distance (64 bins) and the p95 exit quantile;
  esmc_block    one ESMC transformer block at 238 tokens, D=2560, 40 heads, FFN 5120
                (its wqkv, wo, w1, w2 8-bit linears and the LN / RoPE / attention /
                SwiGLU kernels) as one HIP graph: 20 back-to-back replays timed,
                replays checked against the eager output (three with eager
                launches in between, and the last timed one); the eager time,
                bound by the host launches, beside it;
  pair_c256     the same TMU pair at ESMFold2's real width, C = c = 256 (the wide path);
  cpu_baseline  the CPU oracle (torch fp32 restatement of the reference's
                _trimul_forward) on the host cores, a bounded sample of the same
                workload (rank 0, N=1 only), and each q8 linear's fp32
                dequantise-then-matmul on the host (`q8_linear`, with the GPU's
                speedup over it). This leg also verifies the GPU leg:
                the benchmarked pair output and sampled q8 rows are compared with
                the oracle's (the GPU leg itself imports nothing from oracle/).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--graph]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_F16_PEAK = 2.5e15     # FLOP/s, dense fp16/bf16 MFMA

L, C, CL = 238, 128, 128


def alg_counts(L: int, C: int, c: int):
    """Algorithmic FLOPs and compulsory fp16 bytes per launch of each kernel (one direction)."""
    N = L * L
    return {
        "project": {"flops": 2 * N * C * 4 * c, "bytes": 2 * N * C + 2 * 2 * c * N},
        "contract": {"flops": 2 * c * L ** 3, "bytes": 2 * 2 * c * N + 2 * c * N},
        "epilogue": {"flops": 2 * N * (c * C + C * C), "bytes": 2 * c * N + 2 * N * C + 2 * N * C},
    }


PROFILE_COUNTERS = os.path.join(ROOT, "profiles", "bench_L238_counters.md")
PROFILE_TRACE = os.path.join(ROOT, "profiles", "bench_L238_kernel_trace.md")


def profiled_mean_us(kernel: str, grid: int):
    """The committed rocprofv3 kernel-trace mean (microseconds) of one kernel at one grid size,
    from the trace summary's table, or None."""
    try:
        for line in open(PROFILE_TRACE):
            cells = [c.strip() for c in line.split("|")]
            if len(cells) > 6 and cells[1].strip("`").startswith(kernel) and cells[3] == str(grid):
                return float(cells[5])
    except (OSError, ValueError):
        pass
    return None


def measured_traffic():
    """HBM bytes per launch per kernel from the committed rocprofv3 counter summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by a plain-copy calibration); {} if absent."""
    out = {}
    try:
        for line in open(PROFILE_COUNTERS):
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes":
                out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-q8", action="store_true", help="skip the q8 linear figures")
    ap.add_argument("--no-stack", action="store_true", help="skip the transition and block-stack figures")
    ap.add_argument("--no-block-graph", action="store_true",
                    help="time the transition kernel but skip the HIP-graph block-stack figure")
    ap.add_argument("--no-esmc", action="store_true", help="skip the ESMC block figure")
    ap.add_argument("--no-recycle", action="store_true", help="skip the recycling-step figures")
    ap.add_argument("--no-wide", action="store_true", help="skip the 256-wide pair figure")
    ap.add_argument("--graph", action="store_true", help="replay the step as a HIP graph")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 64 MiB device copy 10 times (counter calibration under rocprofv3)")
    return ap.parse_args()


def copy_probe(dev, reps: int = 10, nbytes: int = 64 << 20):
    """A plain device-to-device copy of a known size: under rocprofv3 --pmc its FETCH_SIZE /
    WRITE_SIZE per dispatch calibrate those counters (expected: nbytes each)."""
    import torch
    src = torch.ones(nbytes // 2, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def host_threads() -> int:
    """The host cores this process may use: its CPU affinity, capped by OMP_NUM_THREADS when set
    (the share of a shared host the job is given)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        cap = 0
    return max(1, min(n, cap) if cap > 0 else n)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(z, po, pi, pair_out, q8_samples, stack_case=None, esmc_case=None):
    """The CPU oracle in fp32 on the host cores: 1 warm-up, median of 3 TMU pairs at L=238, and
    the same for each benchmarked q8 linear (fp32 dequantisation and matmul, ``q8_linear``).
    It also verifies the GPU leg: the benchmarked pair output against the oracle's
    (max|err| / RMS(update), bar 1e-2) and the sampled q8 rows (normwise, bar 1e-3)."""
    import numpy as np
    import torch
    from oracle import q8 as oq8, tmu
    threads = host_threads()
    torch.set_num_threads(threads)
    threads = torch.get_num_threads()
    zf = z.float()
    fields = ("w_bundle", "w_emit", "w_gate", "ln_in_w", "ln_in_b", "ln_mix_w", "ln_mix_b", "ln_in_eps", "ln_mix_eps",
              "outgoing")
    po, pi = (tmu.TriMulWeights(**{f: getattr(p, f) for f in fields}) for p in (po, pi))
    with torch.no_grad():
        ref = tmu.trimul_pair(zf, None, po, pi)
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            tmu.trimul_pair(zf, None, po, pi)
            ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    upd_ref = ref.double() - z.double()
    upd_got = pair_out.double() - z.double()
    pair_err = float((upd_got - upd_ref).abs().max() / upd_ref.pow(2).mean().sqrt())
    q8_err, q8_cpu = {}, {}
    for name, (rows, x, q, s, b, y) in q8_samples.items():
        yr = oq8.q8_linear(x[rows].numpy(), q.numpy(), s.numpy(), b.numpy())
        q8_err[name] = float(np.linalg.norm(y - yr) / np.linalg.norm(yr))
        # the whole linear on the host: fp32 dequantisation, then the fp32 matmul
        with torch.no_grad():
            oq8.q8_linear_f32(x, q, s, b)
            tq = []
            for _ in range(3):
                t0 = time.perf_counter()
                oq8.q8_linear_f32(x, q, s, b)
                tq.append(time.perf_counter() - t0)
        q8_cpu[name] = {"ms": statistics.median(tq) * 1e3, "kind": "port",
                        "sample": "fp32 dequantise then fp32 matmul (torch), median of 3 after 1 warm-up"}
    ok = pair_err <= 1e-2 and all(e <= 1e-3 for e in q8_err.values())
    stack_err = None
    if stack_case is not None:
        # the block stack against the oracle in fp64 (exact arithmetic, fp64 stream). The bar is
        # max 3e-2 and RMS 1e-2 of RMS(update): at this depth the reference's own fp16 scheme sits
        # at max 1.75e-2 from fp64 (oracle.transition.stack_forward_fp16ref), above 1e-2
        from oracle import transition as otr
        zs, blocks, got = stack_case
        ob = [otr.BlockWeights(tmu.TriMulWeights(**{f: getattr(a, f) for f in fields}).to(torch.float64),
                               tmu.TriMulWeights(**{f: getattr(b, f) for f in fields}).to(torch.float64),
                               otr.TransitionWeights(t.ln_w.double(), t.ln_b.double(), t.w1.double(), t.w3.double(),
                                                     None if t.w2 is None else t.w2.double(), eps=t.eps))
              for a, b, t in blocks]
        with torch.no_grad():
            ref = otr.stack_forward(zs.double(), None, ob, 3)
        u = ref - zs.double()
        d = got.double() - ref
        rms = float(u.pow(2).mean().sqrt())
        stack_err = {"max_err_over_rms": float(d.abs().max()) / rms, "rms_err_over_rms": float(d.pow(2).mean().sqrt()) / rms,
                     "reference": "fp64 oracle", "bar": {"max": 3e-2, "rms": 1e-2}}
        ok = ok and stack_err["max_err_over_rms"] <= 3e-2 and stack_err["rms_err_over_rms"] <= 1e-2
    esmc_err = None
    if esmc_case is not None:
        # the ESMC block against the oracle (fp32 on the CPU, fp16-rounded dequantised weights)
        from oracle import esmc as oe
        xe, ln, lin, rs, heads, got = esmc_case
        qw = {n: oe.Q8Weights(*(t.numpy() for t in lin[n])) for n in lin}
        pw = oe.EsmcBlockWeights(ln["ln1_w"], ln["ln1_b"], ln["q_ln"], ln["k_ln"], ln["ln2_w"], ln["ln2_b"],
                                 qw["wqkv"], qw["wo"], qw["w1"], qw["w2"])
        with torch.no_grad():
            ref = oe.block_forward(pw, xe.double(), None, n_heads=heads, res_scale=rs, weights="f16")
        u = ref - xe.double()
        esmc_err = float((got.double() - ref).abs().max()) / float(u.pow(2).mean().sqrt())
        ok = ok and esmc_err <= 1e-2
    return {"value": L * L / t, "unit": "cells/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(), "host_cpus": os.cpu_count(), "torch_threads": threads,
            "sample": f"TMU pair (out+in, residuals) at L={L}, C=c={C}, fp32 torch on CPU, median of 3 after 1 "
                      f"warm-up, {t * 1e3:.1f} ms per pair",
            "q8_linear": q8_cpu,
            "check": {"pair_max_err_over_rms": pair_err, "q8_rel_err_sample_rows": q8_err,
                      "block_stack_vs_oracle_fp64": stack_err, "esmc_block_max_err_over_rms": esmc_err,
                      "ok": ok}}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the TMU path is measured on one GPU (its sharding is not built); --gpus must be 1"}))
        sys.exit(2)
    import torch
    from __graft_entry__ import load_package
    pkg = load_package()
    W = pkg.workloads

    lib = pkg.capi.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    z, _, po, pi = W.pair_inputs(L, C, CL, seed=0, dtype=torch.float16)
    t_out = pkg.trimul.TriMul.from_weights(po, device=dev)
    t_in = pkg.trimul.TriMul.from_weights(pi, device=dev)
    K = pkg.kernels
    ld = K.leading_dim(L)
    z0 = z.to(dev)
    zbuf = z0.clone()
    # the launches TriMul / tmu_forward make at C = 128: a, b in the MFMA-fragment layout
    fp = int(lib.tmu_frag_plane_elems(L))
    a = torch.empty(CL, fp, dtype=torch.float16, device=dev)
    b = torch.empty_like(a)
    x = torch.empty(1, CL, L, ld, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream()
    scale = 1.0 / 256.0

    def launch(kind, m: "pkg.trimul.TriMul", zin, zout):
        sp = pkg.capi.stream_ptr()  # the current stream: the capture stream while a graph records
        if kind == "project":
            rc = lib.tmu_project_frag(zin.data_ptr(), None, m.ln_in_w.data_ptr(), m.ln_in_b.data_ptr(), m.ln_in_eps,
                                      m.w_bundle.data_ptr(), a.data_ptr(), b.data_ptr(), 1, L, C, CL,
                                      int(not m.outgoing), sp)
        elif kind == "contract":
            rc = lib.tmu_contract_frag(a.data_ptr(), b.data_ptr(), x.data_ptr(), CL, L, ld, scale, sp)
        else:
            rc = lib.tmu_epilogue(x.data_ptr(), ld, zin.data_ptr(), None, m.ln_in_w.data_ptr(), m.ln_in_b.data_ptr(),
                                  m.ln_in_eps, m.ln_mix_w.data_ptr(), m.ln_mix_b.data_ptr(),
                                  m.ln_mix_eps * scale * scale, m.w_emit.data_ptr(), m.w_gate.data_ptr(),
                                  zout.data_ptr(), 1, L, C, CL, 1, 0, sp)
        pkg.capi.check(rc)

    kinds = ("project", "contract", "epilogue")
    pair = pkg.trimul.TriMulPair(t_out, t_in)

    def step():
        # z1 = z + T_out(z) written into zbuf; z2 = z1 + T_in(z1) in place: one C call
        pair(z0, out=zbuf)

    def kernel_step():
        # the same six launches, one entry point at a time (for per-kernel timing)
        for d, m in enumerate((t_out, t_in)):
            src = z0 if d == 0 else zbuf
            for kind in kinds:
                launch(kind, m, src, zbuf)

    # the benchmarked configuration's output, checked against the oracle in the CPU leg
    step()
    torch.cuda.synchronize()
    pair_out = zbuf.cpu()
    if not torch.isfinite(pair_out.float()).all():
        raise SystemExit("TMU pair output is not finite")
    # the launches timed one by one below make the module's bits
    kernel_step()
    torch.cuda.synchronize()
    if not torch.equal(zbuf.cpu().view(torch.int16), pair_out.view(torch.int16)):
        raise SystemExit("the per-kernel launches differ from TriMulPair's output")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    graph = None
    if args.graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        torch.cuda.synchronize()

    # timed region: exactly `steps` steps between synchronisations
    kname = {"project": "tmu_project_kernel", "contract": "tmu_contract_frag_kernel", "epilogue": "tmu_epilogue_kernel"}
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps

    # per-kernel durations: a second pass of the same eager steps (TriMulPair, one
    # tmu_pair_forward call each) whose six launches carry start/stop events that the runtime
    # stamps with each kernel's own begin and end (capi.KernelTimes, hipExtLaunchKernelGGL), i.e.
    # the durations a profiler's kernel trace reports. Not inside the timed region: a launch that
    # carries the events costs ~7 us more of dispatch (the step went from 91 to 133 us), though
    # the kernel's own duration does not change. The events are created before the pass.
    # Two more steps run first under the events and are not counted (their first launches
    # pay for the switch to the event path).
    skip = 2
    nk = 6 * (args.steps + skip)
    with pkg.capi.KernelTimes(nk):
        pass
    kt = pkg.capi.KernelTimes(nk)
    torch.cuda.synchronize()
    with kt:
        for _ in range(args.steps + skip):
            step()
    torch.cuda.synchronize()
    kt.records = kt.records[6 * skip:]
    per_name = kt.by_kernel()

    counts = alg_counts(L, C, CL)
    kern = {}
    for k in kinds:
        ts = [t for name, v in per_name.items() if name.startswith(kname[k]) for t in v]
        if len(ts) != 2 * args.steps:
            raise SystemExit(f"expected {2 * args.steps} timed launches of {kname[k]}, got {len(ts)}")
        t = statistics.fmean(ts) * 1e-6  # the mean, as rocprofv3 --stats reports it
        kern[k] = {"us": t * 1e6, "us_median": statistics.median(ts), "launches": len(ts),
                   "tflops": counts[k]["flops"] / t / 1e12,
                   "gbs": counts[k]["bytes"] / t / 1e9,
                   "mfma_frac": counts[k]["flops"] / t / MFMA_F16_PEAK,
                   "hbm_frac": counts[k]["bytes"] / t / HBM_PEAK}
    # the contraction's own roof: by its compulsory traffic (AI = flops / bytes = L/3) it cannot
    # beat AI x HBM peak, far below the MFMA peak at this L
    ai = counts["contract"]["flops"] / counts["contract"]["bytes"]
    cap = min(MFMA_F16_PEAK, ai * HBM_PEAK)
    kern["contract"].update({"ai_flop_per_byte": ai, "cap_tflops": cap / 1e12,
                             "cap_bound": "hbm" if cap < MFMA_F16_PEAK else "mfma",
                             "cap_frac": counts["contract"]["flops"] / (kern["contract"]["us"] * 1e-6) / cap})
    traffic = measured_traffic()
    for k in kinds:
        kern[k]["traffic_bytes"] = traffic.get(kname[k])
    dom = max(kinds, key=lambda k: kern[k]["us"])
    if dom == "contract":
        roof = {"bound": "mfma", "achieved": kern[dom]["tflops"], "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": kern[dom]["mfma_frac"], "traffic": kern[dom]["traffic_bytes"], "kernel": kname[dom],
                "per_launch": f"{counts[dom]['flops'] / 1e9:.3f} GFLOP"}
    else:
        roof = {"bound": "hbm", "achieved": kern[dom]["gbs"], "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": kern[dom]["hbm_frac"], "traffic": kern[dom]["traffic_bytes"], "kernel": kname[dom],
                "per_launch": f"{counts[dom]['bytes'] / 1e6:.2f} MB"}
    roof["duration"] = (f"mean of {kern[dom]['launches']} runtime-stamped kernel durations (hipExtLaunchKernelGGL "
                        "events) over a second pass of the timed step")
    # the same kernel's mean in the committed kernel trace (another run, possibly another box:
    # runs scatter by a few per cent, boxes by up to ~10%), and the fraction at that duration
    grid = {"project": 131072, "contract": 131072, "epilogue": 121856}[dom]  # threads per launch at L=238
    prof_us = profiled_mean_us("esm::" + kname[dom], grid)
    if prof_us:
        per_launch = counts[dom]["flops"] if dom == "contract" else counts[dom]["bytes"]
        peak = MFMA_F16_PEAK if dom == "contract" else HBM_PEAK
        roof["profile_us"] = prof_us
        roof["frac_at_profile_us"] = per_launch / (prof_us * 1e-6) / peak

    pair_flops = 2 * sum(v["flops"] for v in counts.values())
    pair_bytes = 2 * sum(v["bytes"] for v in counts.values())
    out = {
        "metric": "tri-mul-update pair cells/sec at L=238 fp16 (+% MFMA peak, % HBM BW)",
        "value": L * L / (ms * 1e-3), "unit": "cells/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) pair tensor, N(0,1/fan_in) weights)",
        "config": {"workload": "TMU pair outgoing+incoming with residuals, z [1,238,238,128] fp16, c_hidden 128, "
                               "all-ones mask", "L": L, "C": C, "c_hidden": CL, "batch": 1,
                   "launch": "hip graph" if graph is not None
                   else "eager: TriMulPair, one tmu_pair_forward call (six launches) per step"},
        "pair_mfma_frac": pair_flops / (ms * 1e-3) / MFMA_F16_PEAK,
        "pair_hbm_frac": pair_bytes / (ms * 1e-3) / HBM_PEAK,
        "roofline": roof,
        "kernels": kern,
    }

    q8_samples = {}
    if not args.no_q8:
        qres = {}
        for (Kd, Nd) in ((2560, 10240), (10240, 2560), (2560, 7680)):
            xq, qq, sq, bq = W.q8_inputs(L, Kd, Nd, seed=Kd)
            xt, qt, st, bt = (t.to(dev) for t in (xq, qq, sq, bq))
            y = torch.empty(L, Nd, dtype=torch.float16, device=dev)
            ws = K.q8_workspace(L, Kd, Nd, device=dev)  # split-K partials when the tiles are too few
            sbp = K.q8_pack_scales(st, bt)              # per-layer layout caches, built once, as Q8Linear
            qpp = K.q8_pack_codes(qt)                   # does by default
            for _ in range(5):
                K.q8_linear(xt, qt, st, bt, out=y, workspace=ws, packed=sbp, codes=qpp)
            rows = [0, L // 2, L - 1]
            name = f"{L}x{Kd}->{Nd}"
            q8_samples[name] = (rows, xq, qq, sq, bq, y[rows].double().cpu().numpy())
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            reps = 50

            def timed(codes):
                torch.cuda.synchronize()
                e0.record(stream)
                for _ in range(reps):
                    K.q8_linear(xt, qt, st, bt, out=y, workspace=ws, packed=sbp, codes=codes)
                e1.record(stream)
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) * 1e-3 / reps

            t_nk = timed(None)  # the codes read in MLX's [N, K] layout (through LDS), the same bits
            t = timed(qpp)
            fl = 2 * L * Kd * Nd
            by = Nd * Kd + 2 * 2 * Nd * (Kd // 64) + 2 * L * Kd + 2 * L * Nd
            qres[name] = {"us": t * 1e6, "tflops": fl / t / 1e12, "mfma_frac": fl / t / MFMA_F16_PEAK,
                          "gbs": by / t / 1e9, "hbm_frac": by / t / HBM_PEAK, "split_k": ws is not None,
                          "layout": "packed codes and scales (Q8Linear's default)", "us_nk_codes": t_nk * 1e6,
                          "tile_rows": int(pkg.capi.lib().q8_tile_rows(L, Kd, Nd))}
            # each launch's own duration (runtime-stamped events, a pass of its own): with split-K the
            # GEMM and the reduction of its partials separately, the reduction being the launch a
            # consumer that sums the partials itself (the ESMC block's LayerNorm) does not make
            nl = 20 * (2 if ws is not None else 1)
            kq = pkg.capi.KernelTimes(nl)
            torch.cuda.synchronize()
            with kq:
                for _ in range(20):
                    K.q8_linear(xt, qt, st, bt, out=y, workspace=ws, packed=sbp, codes=qpp)
            torch.cuda.synchronize()
            qres[name]["kernels_us"] = {k.split("<")[0].split("::")[-1]: statistics.fmean(v)
                                        for k, v in kq.by_kernel().items()}
        # the quantiser (layer_params' mx.quantize) on the largest ESMC weight, w1 [10240, 2560] fp32:
        # reads 4 B per weight, writes a code per weight and an fp16 scale and bias per 64
        Nw, Kw = 10240, 2560
        wf = torch.randn(Nw, Kw, generator=torch.Generator().manual_seed(11)).mul_(0.02).to(dev)
        for _ in range(3):
            K.q8_quantize(wf)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        reps = 20
        for _ in range(reps):
            K.q8_quantize(wf)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        by = 5 * Nw * Kw + 4 * Nw * (Kw // 64)
        qres[f"quantize {Nw}x{Kw}"] = {"us": t * 1e6, "gbs": by / t / 1e9, "hbm_frac": by / t / HBM_PEAK}
        del wf
        out["q8"] = qres

    stack_case = None
    if not args.no_stack:
        # the transition kernel alone, in place on a copy of z
        zs, blocks = W.block_stack(L, n_blocks=8, C=C, c=CL, H=4 * C, seed=0)
        trunk = pkg.trunk.PairTrunk.from_weights(blocks, device=dev)
        tr = trunk.blocks[0].transition
        zt = zs.to(dev).contiguous()
        for _ in range(5):
            tr.run(zt, zt)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 50
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            tr.run(zt, zt)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        tfl = 4 * C * (4 * C) * L * L
        out["transition"] = {"us": t * 1e6, "tflops": tfl / t / 1e12, "mfma_frac": tfl / t / MFMA_F16_PEAK,
                             "gbs": 4 * C * L * L / t / 1e9}
    if not args.no_stack and not args.no_block_graph:
        # the block stack: one HIP graph of 8 blocks x 3 recycles (168 kernels), z reloaded per replay
        recycles = 3
        zbuf = torch.empty(1, L, L, C, dtype=torch.float16, device=dev)
        z0s = zs.to(dev)
        replay = trunk.graphed(zbuf, None, recycles=recycles)
        zbuf.copy_(z0s)
        replay()
        torch.cuda.synchronize()
        stack_out = zbuf.cpu()
        ts = []
        for _ in range(5):
            zbuf.copy_(z0s)
            torch.cuda.synchronize()
            e0.record(stream)
            replay()
            e1.record(stream)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e-3)
        t = statistics.median(ts)
        fl = 8 * recycles * (2 * sum(v["flops"] for v in counts.values()) + tfl)
        out["block_stack"] = {"ms": t * 1e3, "blocks": 8, "recycles": recycles, "launch": "hip graph",
                              "tflops": fl / t / 1e12, "mfma_frac": fl / t / MFMA_F16_PEAK,
                              "cells_per_s_per_block": L * L * 8 * recycles / t}
        stack_case = (zs, blocks, stack_out)

    if not args.no_recycle:
        g = torch.Generator().manual_seed(0)
        zr, zi, rf = (torch.randn(1, L, L, C, generator=g).to(dev) for _ in range(3))
        lw, lb, av = torch.ones(C, device=dev), torch.zeros(C, device=dev), torch.rand(C, generator=g).to(dev)
        bm = (torch.randn(C, C, generator=g) * C ** -0.5).half().to(dev)
        dw, db = (torch.randn(64, C, generator=g) * 0.1).half().to(dev), torch.randn(64, generator=g).to(dev)
        cen = pkg.recycle.centers_6b(dev)
        zo = torch.empty_like(zr)
        ed_prev = K.expected_distance(zr, dw, db, cen)
        ed = torch.empty_like(ed_prev)
        qo = torch.empty(1, device=dev)
        ops = {"parcae_step": lambda: K.parcae_step(zr, zi, rf, lw, lb, 1e-5, av, bm, out=zo),
               "expected_distance": lambda: K.expected_distance(zo, dw, db, cen, out=ed),
               "p95_quantile": lambda: K.abs_diff_quantile(ed, ed_prev, 0.95, out=qo)}
        rres = {}
        for name, fn in ops.items():
            for _ in range(3):
                fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(20):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            rres[name] = {"us": e0.elapsed_time(e1) * 1e3 / 20}
        pb = 4 * C * L * L * 4  # parcae: read z, z_init, refined, write z (fp32)
        rres["parcae_step"].update({"gbs": pb / rres["parcae_step"]["us"] / 1e3,
                                    "hbm_frac": pb / rres["parcae_step"]["us"] / 1e3 / (HBM_PEAK / 1e9)})
        out["recycle"] = rres

    if not args.no_wide:
        # the same pair at ESMFold2's real pair width, C = c = 256 (the wide path: five launches
        # per direction), z [1, 238, 238, 256] fp16
        zw, _, pow_, piw = W.pair_inputs(L, 256, 256, seed=0, dtype=torch.float16)
        T = pkg.trimul
        pair_w = T.TriMulPair(T.TriMul.from_weights(pow_, device=dev), T.TriMul.from_weights(piw, device=dev))
        zw0 = zw.to(dev)
        zwo = torch.empty_like(zw0)
        for _ in range(3):
            pair_w(zw0, out=zwo)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            pair_w(zw0, out=zwo)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        cw = alg_counts(L, 256, 256)
        fl = 2 * sum(v["flops"] for v in cw.values())
        by = 2 * sum(v["bytes"] for v in cw.values())  # compulsory: the three fused kernels' bytes
        tr = measured_traffic()  # counter bytes of the five launches per direction, when profiled
        wide_keys = ("ln_rows_kernel", "wide_gemm_ws_kernel_gate_cm", "tmu_contract_frag_kernel_c256",
                     "ln_cf_to_cl_kernel", "wide_gemm_ws_kernel_resgate")
        meas = 2 * sum(tr[k] for k in wide_keys) if all(k in tr for k in wide_keys) else None
        out["pair_c256"] = {"us": t * 1e6, "cells_per_s": L * L / t, "tflops": fl / t / 1e12,
                            "mfma_frac": fl / t / MFMA_F16_PEAK,
                            "compulsory_bytes": by, "gbs": by / t / 1e9, "hbm_frac": by / t / HBM_PEAK,
                            "traffic_bytes": meas, "launches": 10,
                            "workload": "TMU pair out+in with residuals, z [1,238,238,256] fp16, c_hidden 256"}

    esmc_case = None
    if not args.no_esmc:
        ED, EF, EH = 2560, 5120, 40
        xe, ln, lin = W.esmc_block_inputs(L, ED, EF, seed=0)
        blk = pkg.esmc.EsmcBlock.from_arrays(ln, lin, EH, device=dev)
        rs = (80 / 36) ** 0.5
        xed = xe.to(dev)
        for _ in range(3):
            ye = blk(xed, None, res_scale=rs)
        torch.cuda.synchronize()
        esmc_out = ye.cpu()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        e0.record(stream)
        for _ in range(reps):
            blk(xed, None, res_scale=rs)
        e1.record(stream)
        torch.cuda.synchronize()
        t_eager = e0.elapsed_time(e1) * 1e-3 / reps  # bound by the host launches (9 kernels and torch's allocations)
        # the same block replayed as one HIP graph: the GPU's own time; every replay is
        # checked against the eager output, with eager launches in between
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            yg = blk(xed, None, res_scale=rs)
        held = pkg.scratch.current(dev)  # the shared scratch the captured launches use stays alive
        replays_equal = True
        for _ in range(3):  # each replay checked against the eager output, eager launches in between
            g.replay()
            torch.cuda.synchronize()
            replays_equal &= bool(torch.equal(yg, ye))
            blk(xed, None, res_scale=rs)
        torch.cuda.synchronize()
        reps = 20  # timed: back-to-back replays, the block's steady-state time
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        replays_equal &= bool(torch.equal(yg, ye))
        fl = 2 * L * ED * (3 * ED + ED + 2 * EF + EF) + 4 * L * L * ED  # linears + attention
        wbytes = sum(q.numel() + 4 * s_.numel() for q, s_, _ in lin.values())
        out["esmc_block"] = {"us": t * 1e6, "eager_us": t_eager * 1e6, "tokens": L, "D": ED, "ffn": EF,
                             "heads": EH, "launch": "hip graph", "graph_replays_equal_eager": replays_equal,
                             "tflops": fl / t / 1e12, "mfma_frac": fl / t / MFMA_F16_PEAK,
                             "weight_gbs": wbytes / t / 1e9, "weight_hbm_frac": wbytes / t / HBM_PEAK}
        esmc_case = (xe, ln, lin, rs, EH, esmc_out)

    if args.copy_probe:
        copy_probe(dev)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(z, po, pi, pair_out, q8_samples, stack_case, esmc_case)
        out["speedup_vs_cpu"] = out["value"] / out["cpu_baseline"]["value"]
        for name, c in out["cpu_baseline"]["q8_linear"].items():
            if name in out.get("q8", {}):
                c["speedup_of_gpu"] = c["ms"] * 1e3 / out["q8"][name]["us"]
    print(json.dumps(out), flush=True)
    if not args.no_cpu and not out["cpu_baseline"]["check"]["ok"]:
        raise SystemExit("the benchmarked outputs differ from the oracle beyond the bars")


if __name__ == "__main__":
    main()
