"""Throughput of the anchored transport score, forward + backward, on one MI355X.

Workload: 1M synthetic events on a 640x480 sensor over 100 ms (50 line segments + 30% noise), a smooth random
dense flow grid 2x480x640 (max 200 px/s), AnchoredExact with h = sigma (default 1 px), tau = 20 ms (0.2 of the
window), cut = 3, 16 slices, every event an anchor, dequantisation jitter, smoothed anchors, exposure
correction; backward to the flow grid.  One step = one full loss evaluation + backward, inputs resident in
HBM.  Prints one JSON line (rank 0, N = 1) with events/s, the dominant kernel's roofline and the CPU baseline
(the oracle's OpenMP restatement of the reference CPU path on this host's cores).

    python bench.py [--steps K] [--warmup W] [--sigma S] [--no-cpu]

Other workloads (parity-test configurations, not the headline metric), same output contract:

    python bench.py --workload iwe             # 1M events 640x480, dense flow: warp to t = 0.5, bilinear IWE
                                               # (inside mask), gather of the IWE at the warped events,
                                               # loss = sum, backward to the flow grid
    python bench.py --workload iwe-plumbing    # the same on 100k events 240x180, constant flow (2, -1.25)
    python bench.py --workload anchored-reflayout  # the headline workload through the reference's own call
                                               # pattern (device plan in the reference layout + the pybind-surface
                                               # ats_pair_fwd / ats_pair_bwd), as an unchanged functional.py gets it
    python bench.py --workload anchored-blobs  # contention stress: the anchored score on 4M events, 90% in 5
                                               # Gaussian blobs (sigma 8 px), Sim2 flow (0, 0, 0.1, 0.1)
    python bench.py --workload voxel           # voxel_grid (the training input): 1M events 640x480, 15 time bins
    python bench.py --workload mpcm-lut        # MotionPriorCMax's look-up table at its DSEC configuration: 15
                                               # time bins x 19200 cells of 4 px (640x480), the 32 nearest of
                                               # 19200 tile trajectories (K = 10 B-spline) per cell and bin,
                                               # their mean displacement to t_ref, backward to the coefficients
    python bench.py --workload trajectories    # 4 windows x 500k events 640x480 (25 ms each), per-pixel cubic
                                               # B-spline trajectories with 10 control points: anchored
                                               # pair-sum score (h 1, tau 20 ms = 0.8, 16 slices) + the IWE
                                               # contrast (bilinear splat at t = 0.5), grad to the control
                                               # points

Two helpers for the rocprofv3 summaries under profiles/ (no GPU work beyond what they name):

    python bench.py --calibrate-copy MB        # a plain f32 copy of MB MiB (read MB, write MB), 5 times
    python bench.py --summarize DIR... --out FILE --title T --command C [--calibration DIR... --copy-mb MB]
        # kernel table from *_kernel_stats.csv and per-dispatch counter means from *_counter_collection.csv;
        # with a calibration, FETCH_SIZE / WRITE_SIZE are scaled by what they read for the copy of MB MiB in
        # the calibration runs, and the per-launch HBM bytes of every kernel are recorded for the roofline
        # "traffic" of bench.py
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

VALU_PEAK = 256 * 4 * 16 * 2.4e9      # fp32 lane-slots/s (non-packed): 256 CUs x 4 SIMD x 16 lanes x 2.4 GHz
FP32_PEAK = 157.3e12                   # fp32 FLOP/s (packed FMA), MI355X
SLOTS_FWD, SLOTS_BWD = 14, 16          # VALU lane-slots per contributing pair (forward, backward)
SLOTS_BWD_TRAJ = 20                    # trajectory backward: the pair recomputed (13) + k gS (1) + k gS r (2) +
                                       # position and velocity gradient sums (2 adds, 2 FMAs)
FLOPS_FWD, FLOPS_BWD = 13, 19          # fp32 flops per contributing pair (FMA = 2, exp = 1)
HBM_PEAK = 8.0e12                      # bytes/s
# compulsory HBM bytes per event of the anchored step: positions 8, dequantisation 8, smoothing 8, time 4,
# batch 8 (the flow grid and its gradient are added per call); with the splat leg: + 20 forward + 32 backward
STEP_BYTES_PER_EVENT, SPLAT_BYTES_PER_EVENT = 36, 52
KERNEL_OF = {"atl_fast_pair_fwd": "k_fast_fwd<false>", "atl_fast_pair_bwd": "k_fast_bwd", "atl_fast_pair_bwd_src": "k_fast_bwd",
             "atl_fast_pair_bwd_traj": "k_fast_bwd_traj<10>"}
COUNTERS = ROOT / "profiles" / "anchored_score_1M_640x480_counters.md"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", default="anchored",
                    choices=["anchored", "anchored-reflayout", "anchored-blobs", "iwe", "iwe-composed", "iwe-plumbing",
                             "trajectories", "mpcm-lut", "voxel"])
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--sigma", type=float, default=1.0)
    ap.add_argument("--events", type=int, default=0, help="events of the anchored workloads (default 1M; 4M blobs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="iwe, iwe-plumbing: time eager steps instead of replays of the captured step")
    ap.add_argument("--cpu-budget", type=float, default=25.0, help="seconds of CPU baseline work, at most")
    ap.add_argument("--calibrate-copy", type=float, default=0.0, metavar="MB")
    ap.add_argument("--summarize", nargs="+", metavar="DIR")
    ap.add_argument("--out")
    ap.add_argument("--title", default="rocprofv3 summary")
    ap.add_argument("--command", default="")
    ap.add_argument("--copy-mb", type=float, default=0.0)
    ap.add_argument("--calibration", nargs="*", default=[], metavar="DIR",
                    help="counter runs of --calibrate-copy (FETCH_SIZE, WRITE_SIZE)")
    ap.add_argument("--pairs", type=float, default=0.0,
                    help="--summarize: contributing pairs K per launch of the pair kernels (the bench line's "
                         "roofline.pairs), for their VALU lane-slots per pair")
    return ap.parse_args()


# ------------------------------------------------------------------------------------------- profiles
def _short(name):
    n = name.replace("(anonymous namespace)::", "").replace("void ", "")
    if n.startswith("at::native"):
        m = re.search(r"at::native::(?:\(anonymous namespace\)::)?(\w+)<[^<]*?(?:at::native::)?(\w+Functor\w*|\w+_kernel\w*)?",
                      n)
        return "torch " + n.split("<")[0].replace("at::native::", "") + (" " + m.group(2) if m and m.group(2) else "")
    return n.split("(")[0]


def _counters(dirs):
    agg = {}
    for f in sorted(sum((glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True) for d in dirs),
                        [])):
        for r in csv.DictReader(open(f)):
            agg.setdefault(_short(r["Kernel_Name"]), {}).setdefault(r["Counter_Name"], []).append(
                float(r["Counter_Value"]))
    return agg


def summarize(dirs, out, title, command, copy_mb, cal_dirs=(), pairs=0.0):
    """Markdown summary of rocprofv3 csv output (kernel stats and counters), with the per-launch HBM traffic
    of every kernel when a calibration copy of copy_mb MiB is among the counter runs, and the VALU lane-slots
    per contributing pair (SQ_INSTS_VALU x 64 / K) of the pair kernels when K is given."""
    lines = [f"# {title}", "", "Command (repo root, on the MI355X):", "", f"    {command}", ""]
    for f in sorted(sum((glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True) for d in dirs), [])):
        rows = list(csv.DictReader(open(f)))
        lines += ["| kernel | calls | avg us | total share |", "|---|---|---|---|"]
        for r in rows[:24]:
            lines.append(f"| {_short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['Percentage']):.1f}% |")
        lines.append("")
    agg = _counters(dirs)
    traffic = {}
    if agg:
        scale = {}
        if copy_mb > 0 and cal_dirs:
            want_kib = copy_mb * 1024.0
            for cs in _counters(cal_dirs).values():      # the calibration runs hold only the copy kernel
                for c in ("FETCH_SIZE", "WRITE_SIZE"):
                    if c in cs:
                        scale[c] = want_kib / (sum(cs[c]) / len(cs[c]))
            lines += [f"Calibration: a plain copy of {copy_mb:g} MiB (torch.neg, f32) reads FETCH_SIZE = "
                      f"{want_kib / scale.get('FETCH_SIZE', float('nan')):.0f} and WRITE_SIZE = "
                      f"{want_kib / scale.get('WRITE_SIZE', float('nan')):.0f} (KiB per dispatch) for "
                      f"{want_kib:.0f} KiB moved each way: scale factors {scale.get('FETCH_SIZE', float('nan')):.3f}"
                      f" and {scale.get('WRITE_SIZE', float('nan')):.3f}.", ""]
        lines += ["| kernel | counter | mean per dispatch | dispatches |", "|---|---|---|---|"]
        for k in sorted(agg):
            for c in sorted(agg[k]):
                v = agg[k][c]
                lines.append(f"| {k} | {c} | {sum(v) / len(v):.6g} | {len(v)} |")
            if "FETCH_SIZE" in agg[k] and "WRITE_SIZE" in agg[k] and len(scale) == 2:
                fetch = sum(agg[k]["FETCH_SIZE"]) / len(agg[k]["FETCH_SIZE"]) * scale["FETCH_SIZE"]
                write = sum(agg[k]["WRITE_SIZE"]) / len(agg[k]["WRITE_SIZE"]) * scale["WRITE_SIZE"]
                traffic[k] = (fetch + write) * 1024.0
        lines.append("")
    if pairs > 0:
        rows = [(k, agg[k]) for k in sorted(agg) if k.startswith("k_fast_") and "SQ_INSTS_VALU" in agg[k]]
        if rows:
            lines += [f"VALU lane-slots per contributing pair (SQ_INSTS_VALU x 64 / K, K = {pairs:.4g} pairs per "
                      f"launch):", ""]
            for k, cs in rows:
                v = sum(cs["SQ_INSTS_VALU"]) / len(cs["SQ_INSTS_VALU"])
                act = ""
                if "SQ_THREAD_CYCLES_VALU" in cs:
                    tc = sum(cs["SQ_THREAD_CYCLES_VALU"]) / len(cs["SQ_THREAD_CYCLES_VALU"])
                    act = f"; active lanes {tc / (64.0 * v):.2f} (SQ_THREAD_CYCLES_VALU / 64 SQ_INSTS_VALU)"
                lines.append(f"- {k}: {v * 64.0 / pairs:.1f}{act}")
            lines.append("")
    if traffic:
        lines += ["HBM traffic per launch (calibrated FETCH_SIZE + WRITE_SIZE):", ""]
        lines += [f"- {k}: {v / 1e6:.1f} MB" for k, v in sorted(traffic.items())]
        lines += ["", f"<!-- traffic: {json.dumps(traffic)} -->"]
    text = "\n".join(lines) + "\n"
    if out:
        Path(out).write_text(text)
    print(text)


def recorded_traffic(kernel, counters=None):
    """Calibrated HBM bytes per launch of `kernel` (or the sum over a list of kernels) from a committed counter
    summary (default: the anchored score's), or None."""
    path = counters or COUNTERS
    if not path.exists():
        return None
    m = re.search(r"<!-- traffic: (\{.*\}) -->", path.read_text())
    if not m:
        return None
    table = json.loads(m.group(1))
    if isinstance(kernel, str):
        return table.get(kernel)
    parts = [table.get(k) for k in kernel]
    return None if any(v is None for v in parts) else float(sum(parts))


def calibrate_copy(mb):
    n = int(mb * 2 ** 20 / 4)
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_mib": mb, "elements": n}), flush=True)


def workload(kind, n_events, device):
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import DenseLinearFlow, Sim2
    if kind == "anchored-blobs":
        win = synth.blob_window(seed=0, n=n_events)
        motion = Sim2(1, win.height, win.width, init=torch.as_tensor(win.motion["theta"])[None])
        desc = (f"anchored score fwd+bwd, {win.n} events, 640x480, 90% in 5 Gaussian blobs (sigma 8 px) + 10% "
                f"noise, Sim2 flow (0, 0, 0.1, 0.1) per window")
    else:
        win = synth.dense_flow_window(seed=0, n=n_events)
        grid = win.motion["grid"]
        motion = DenseLinearFlow(1, win.height, win.width, grid=grid.shape[-2:], init=torch.as_tensor(grid))
        desc = f"anchored score fwd+bwd, {win.n} events, 640x480, dense flow 2x480x640"
    return win, EventPacket.from_window(win, device), motion.to(device), desc


def _host_cpu():
    """Model name and physical cores of the host (/proc/cpuinfo), and the CPUs this process may use."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    return {"cpu_model": model, "host_physical_cores": len(cores) or None,
            "cpus_available": len(os.sched_getaffinity(0))}


def _oracle():
    """The oracle, with its OpenMP threads bound close (set before its runtime starts)."""
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")
    import oracle as O
    return O


def _baseline_line(O, n, n_all, dt, what):
    return dict({"value": n / dt, "unit": "events/s", "cores": O.num_threads(), "kind": "port",
                 "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
                 "sample": (f"{what} on the whole window, {dt:.2f} s" if n == n_all else
                            f"{what} on the first {n} events of the same window (time-sorted prefix, the largest of "
                            f"a doubling series that fits the budget; it truncates the +-tau neighbourhoods near "
                            f"its end), {dt:.2f} s")}, **_host_cpu())


def _velocity_np(win, xy, b):
    """The window's motion field at xy (NumPy, fp32 op order of the motion models) and, for a dense grid,
    the flow-lookup indices and weights."""
    O = _oracle()
    if win.motion["kind"] == "dense":
        return O.dense_velocity(win.motion["grid"], xy, b, win.height, win.width)
    th = win.motion["theta"].astype(np.float32)
    c = np.array([(win.width - 1) / 2.0, (win.height - 1) / 2.0], np.float32)
    d = (xy - c).astype(np.float32)
    vx = th[0] + (th[2] * d[:, 0] - th[3] * d[:, 1])
    vy = th[1] + (th[3] * d[:, 0] + th[2] * d[:, 1])
    return np.stack([vx, vy], 1).astype(np.float32), None, None


def _bounded_run(run, n_all, budget):
    """Time prefixes of the (time-sorted) window of 20k, 40k, 80k, ... events until one takes more than a
    quarter of the budget or covers the whole window; the work per event grows with the prefix (a short prefix
    truncates the +-tau neighbourhoods), at most quadratically, so the last run stays within the budget.
    Returns (events, seconds, events of the previous run)."""
    n, prev = min(n_all, 20_000), 0
    while True:
        t0 = time.perf_counter()
        run(n)
        dt = time.perf_counter() - t0
        if dt > budget / 4 or n >= n_all:
            return n, dt, prev
        prev, n = n, min(n_all, 2 * n)


def cpu_baseline(win, sigma, budget, splat_leg=False):
    """Oracle on the same workload: the full anchored score forward + backward, the plan built with torch CPU
    ops as the reference builds it on CPU tensors (atl/ops/functional.py:132-178), the pair sums, splat and
    gather in the OpenMP restatement of csrc/atl_cpu.cpp (with splat_leg, the IWE at t = 0.5 forward and
    backward); timed once on a bounded prefix."""
    O = _oracle()
    H, W = win.height, win.width
    rng = np.random.default_rng(0)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(np.float32)
    xa = (xs + sigma * rng.standard_normal(xs.shape)).astype(np.float32)
    dense = win.motion["kind"] == "dense"

    def run(n):
        sl = slice(0, n)
        v, idx, wts = _velocity_np(win, xs[sl], win.b[sl])
        anchors = np.arange(n)
        p = O.build_pair_plan_torch(xs[sl], win.t[sl], v, win.b[sl], 1, H, W, anchors, sigma, 0.2, 3.0, 16,
                                    anchor_xy=xa[sl])
        S = O.ats_pair_fwd(p, sigma, 0.2, 3.0)
        wc = O.window_counts(win.t[sl], win.b[sl], anchors, 0.2)
        vis = (O.visible_fraction_dense(win.motion["grid"], xa[sl], win.t[sl], win.b[sl], win.t[sl], win.b[sl], 1,
                                        H, W, 0.2) if dense else None)
        _, gS, _ = O.anchored_epilogue(S, wc, sigma, H, W, vis=vis)
        gv = O.ats_pair_bwd(gS, p, sigma, 0.2, 3.0, n)
        if dense:
            O.sample_grid_bwd(gv, idx, wts, win.motion["grid"].shape)
        if splat_leg:                              # IWE at t = 0.5: transport, inside mask, splat, variance grad
            vr, _, _ = _velocity_np(win, win.xy[sl], win.b[sl])
            y = (win.xy[sl] + vr * (np.float32(0.5) - win.t[sl])[:, None]).astype(np.float32)
            w = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(np.float32)
            img = O.splat_bilinear_fwd(y, w, win.b[sl], 1, H, W)
            gimg = ((2.0 / (H * W - 1)) * (img - img.mean())).astype(np.float32)
            O.splat_bilinear_bwd(gimg, y, w, win.b[sl])

    n, dt, _ = _bounded_run(run, win.n, budget)
    return _baseline_line(O, n, win.n, dt, "anchored score fwd+bwd")


# ----------------------------------------------------------------------------------------- IWE workloads
# Algorithmic HBM bytes of each entry point: per event (positions 8, batch 8, weights or values 4, outputs)
# plus the image or flow grid once.
IWE_COUNTERS = ROOT / "profiles" / "iwe_1M_640x480_counters.md"
# the kernels of the fused entry points whose HBM counters the IWE counter summary holds
IWE_KERNELS = {
    "atl_warp_splat_gather_fwd": ["k_flow_interleave", "k_wsg_warp<true>", "k_tile_bin<0, true, false>",
                                  "k_tile_accum_bins<0, 1>", "k_wsg_gather"],
    "atl_warp_splat_gather_bwd": ["k_wsg_pack", "k_tile_accum_bins<5, 1>", "k_wsg_grad<true>",
                                  "k_tile_accum_bins<4, 2>"],
}
IWE_BYTES = {
    "atl_splat_bilinear_fwd": lambda n, hw, g: 20 * n + 4 * hw,
    "atl_splat_bilinear_bwd": lambda n, hw, g: 32 * n + 4 * hw,
    "atl_gather_bilinear_fwd": lambda n, hw, g: 20 * n + 4 * hw,
    "atl_gather_bilinear_bwd": lambda n, hw, g: 28 * n + 8 * hw,
    "atl_sample_grid_fwd": lambda n, hw, g: 24 * n + 4 * g,
    "atl_sample_grid_bwd_planned": lambda n, hw, g: 16 * n + 8 * g,
    "atl_sample_grid_bwd_binned": lambda n, hw, g: 24 * n + 8 * g,
    # fused warp -> splat -> gather: events (xy, t, b) and values (or their gradients), the flow grid (or its
    # gradient) and the image once per direction
    "atl_warp_splat_gather_fwd": lambda n, hw, g: 24 * n + 4 * hw + 4 * g,
    "atl_warp_splat_gather_bwd": lambda n, hw, g: 24 * n + 4 * hw + 4 * g,
}


def iwe_workload(kind, dev):
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import DenseLinearFlow, Translation
    if kind in ("iwe", "iwe-composed"):
        win = synth.dense_flow_window(seed=0)
        grid = win.motion["grid"]
        motion = DenseLinearFlow(1, win.height, win.width, grid=grid.shape[-2:], init=torch.as_tensor(grid))
        desc = (f"IWE splat+gather fwd+bwd, {win.n} events, 640x480, dense flow 2x480x640 (max 20 px/window), "
                f"warp to t=0.5, bilinear, inside mask, loss = sum of gathered IWE, grad to the flow grid"
                + (" (transport, make_iwe and gather as separate ops)" if kind == "iwe-composed" else
                   " (fused warp -> splat -> gather)"))
    else:
        win = synth.plumbing_translation(seed=0)
        motion = Translation(1, win.height, win.width, init=torch.as_tensor(win.motion["theta"])[None])
        desc = (f"IWE splat+gather fwd+bwd, {win.n} events, 240x180, translation (2.0, -1.25) px/window, "
                f"warp to t=0, bilinear, inside mask, loss = sum of gathered IWE, grad to theta")
    return win, EventPacket.from_window(win, dev), motion.to(dev), desc


def iwe_cpu_baseline(win, t_ref, budget):
    """Oracle on the host: NumPy warp (+ flow lookup), OpenMP splat / gather forward and backward, flow-grid
    adjoint; same loss as the GPU step."""
    O = _oracle()
    H, W = win.height, win.width

    def run(n):
        sl = slice(0, n)
        xy, t, b = win.xy[sl], win.t[sl], win.b[sl]
        if win.motion["kind"] == "dense":
            v, idx, wts = O.dense_velocity(win.motion["grid"], xy, b, H, W)
        else:
            v = np.broadcast_to(win.motion["theta"].astype(np.float32), xy.shape)
        y = (xy + v * (np.float32(t_ref) - t)[:, None]).astype(np.float32)
        w = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(np.float32)
        img = O.splat_bilinear_fwd(y, w, b, 1, H, W)
        O.gather_bilinear_fwd(img, y, b)
        gimg, gp1 = O.gather_bilinear_bwd(np.ones(n, np.float32), img, y, b)
        gp2, _ = O.splat_bilinear_bwd(gimg, y, w, b)
        gv = (gp1 + gp2) * (np.float32(t_ref) - t)[:, None]
        if win.motion["kind"] == "dense":
            O.sample_grid_bwd(gv, idx, wts, win.motion["grid"].shape)
        else:
            gv.sum(0)

    n, dt, _ = _bounded_run(run, win.n, budget)
    return _baseline_line(O, n, win.n, dt, "IWE step")


def iwe_main(a, dev):
    from x_amd.objectives.base import IWEConfig, iwe_at_events, make_iwe
    from x_amd.ops import _ext, gather
    win, ev, motion, desc = iwe_workload(a.workload, dev)
    t_ref = 0.0 if a.workload == "iwe-plumbing" else 0.5
    cfg = IWEConfig(kernel="bilinear", sigma=0.0, mask_border=True)
    # the loss is the sum of the gathered values; its backward is seeded with its gradient, ones, made once here:
    # torch's many-block sum clears a semaphore buffer with a memset, which a captured graph must not hold
    ones = torch.ones(ev.n, device=dev)

    def body():
        if a.workload == "iwe-composed":
            y = motion.transport(ev.xy, ev.t, t_ref, ev.b)
            img = make_iwe(ev, y, t_ref, cfg)
            gather(img, y, ev.b).backward(ones)
        else:
            _, vals = iwe_at_events(ev, motion, t_ref, cfg)
            vals.backward(ones)

    def step():
        for p in motion.parameters():
            p.grad = None
        body()

    # The fused workloads are launch-bound at these sizes: their timed steps replay the whole forward + backward
    # step captured once as a HIP graph (every kernel runs again in every replay; only the host launch work is
    # gone).  The kernel times behind the roofline come from eager steps either way.
    use_graph = a.workload in ("iwe", "iwe-plumbing") and not a.no_graph
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    kernels = list(IWE_BYTES)
    rec = _ext.time_kernels(kernels, every=5)      # every bracket delays the next launch: sample the steps
    t0 = time.perf_counter()
    for _ in range(10 if use_graph else a.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = {k: float(np.mean([e0.elapsed_time(e1) for e0, e1, _ in rec[k]])) for k in kernels if rec[k]}
    _ext.time_kernels(())
    if use_graph:
        side = torch.cuda.Stream()                 # torch's capture recipe: warm the step up on a side stream
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(side)
        for p in motion.parameters():
            p.grad = None                          # the captured backward writes the gradients it allocates
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            body()
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            graph.replay()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    hw = ev.height * ev.width
    g = 0 if a.workload == "iwe-plumbing" else 2 * hw
    gbs = {k: IWE_BYTES[k](ev.n, hw, g) / (ms[k] * 1e-3) / 1e9 for k in ms}
    dom = max(ms, key=lambda k: ms[k])
    line = {
        "metric": f"events/s for IWE splat+gather fwd+bwd @{ev.n} events {ev.width}x{ev.height}; % HBM roofline",
        "value": ev.n * a.steps / dt, "unit": "events/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": 1e3 * dt / a.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": desc, "events": ev.n, "sensor": [ev.width, ev.height], "parallelism": "single GPU",
                   "timed": "HIP graph replays of the whole step" if use_graph else "eager steps"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": gbs[dom], "peak": 8000.0, "unit": "GB/s",
                     "frac": gbs[dom] / 8000.0,
                     "traffic": (recorded_traffic(IWE_KERNELS[dom], IWE_COUNTERS)
                                 if a.workload == "iwe" and dom in IWE_KERNELS else None),
                     "kernel_ms": ms[dom]},
        "kernel_ms": ms,
        "kernel_gbs": gbs,
    }
    if not a.no_cpu:
        line["cpu_baseline"] = iwe_cpu_baseline(win, t_ref, a.cpu_budget)
    print(json.dumps(line), flush=True)


# ----------------------------------------------------------------------------------- trajectories workload
TRAJ_TAU = 0.8                         # 20 ms of a 25 ms window


def trajectories_main(a, dev):
    """The continuous-time workload: AnchoredTrajectories (pair sums over per-pixel cubic B-spline trajectories,
    h = 1, tau = 0.8, 16 slices, every event an anchor) plus the IWE contrast at t = 0.5, backward to the
    (4, 20, 480, 640) control points."""
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import PixelTrajectories
    from x_amd.objectives import AnchoredTrajectories, iwe_variance
    from x_amd.ops import _ext
    from x_amd.ops import functional as F
    win = synth.bspline_windows(seed=0)
    K = win.motion["K"]
    ev = EventPacket.from_window(win, dev)
    coeff = torch.tensor(win.motion["coeffs"], device=dev, requires_grad=True)
    obj = AnchoredTrajectories(h=1.0, tau=TRAJ_TAU, cut=3.0, n_slices=16, n_anchors=None, seed=0, rng="device")

    def step():
        coeff.grad = None
        # one layout scope per step: the coefficient grid's channels-last copy is made once per step and serves
        # every look-up of both terms
        with F.layout_scope():
            m = PixelTrajectories(coeff, K, "bspline", tile=1)
            loss = obj(ev, m)["loss"] - iwe_variance(ev, m, 0.5)
        loss.backward()

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    kernels = ["atl_fast_pair_fwd", "atl_fast_pair_bwd_traj"]
    rec = _ext.time_kernels(kernels, every=4)
    first_draw = obj._philox[1]
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = {k: float(np.mean([e0.elapsed_time(e1) for e0, e1, _ in rec[k]])) for k in kernels}
    _ext.time_kernels(())
    # contributing pairs of the timed steps' own noise draws (counted outside the timed region)
    pairs = []
    with torch.no_grad():
        m = PixelTrajectories(coeff.detach(), K, "bspline", tile=1)
        tab = m.slice_tables(16, dev)
        for draw in range(first_draw, first_draw + a.steps):
            xs, xa = F.event_noise(ev.xy, 0, draw, 1.0)
            p = m.origin(xs, ev.t, ev.b)
            plan = F.FastPairPlan(p, ev.t, None, ev.b, ev.batch_size, ev.height, ev.width, None, 1.0, TRAJ_TAU, 3.0,
                                  16, xa, traj=(m.coeff_rows(p, ev.b), K, tab))
            pairs.append(int(plan.counts().sum()))
    Kp = float(np.mean(pairs))
    dom = max(kernels, key=lambda k: ms[k])
    slots = SLOTS_FWD if dom.endswith("fwd") else SLOTS_BWD_TRAJ
    achieved = Kp * slots / (ms[dom] * 1e-3)
    line = {
        "metric": f"events/s for anchored-score (pair-sum + splat) fwd+bwd @{ev.n} events ({ev.batch_size} windows) "
                  f"640x480, cubic B-spline trajectories; % VALU roofline",
        "value": ev.n * a.steps / dt, "unit": "events/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": 1e3 * dt / a.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"AnchoredTrajectories(h=1, tau={TRAJ_TAU}, cut=3, S=16, all anchors) - IWE variance "
                               f"at t=0.5 on {ev.batch_size} windows x {ev.n // ev.batch_size} events, 640x480, "
                               f"PixelTrajectories(K={K}, bspline, tile 1, 6 fixed-point steps), grad to the "
                               f"({ev.batch_size}, {2 * K}, 480, 640) control points",
                   "events": ev.n, "windows": ev.batch_size, "sensor": [640, 480], "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "kernel": dom, "achieved": achieved / 1e12, "peak": VALU_PEAK / 1e12,
                     "unit": "Tslot/s", "frac": achieved / VALU_PEAK, "traffic": recorded_traffic(KERNEL_OF[dom]),
                     "pairs": Kp, "slots_per_pair": slots, "kernel_ms": ms[dom]},
        "kernel_ms": ms,
        "pairs_per_anchor": Kp / ev.n,
    }
    if not a.no_cpu:
        line["cpu_baseline"] = trajectories_cpu_baseline(win, a.cpu_budget)
    print(json.dumps(line), flush=True)


def trajectories_cpu_baseline(win, budget):
    """Oracle on a prefix of window 0: trajectory starts (fixed point on the fp32 sampler), coefficient rows,
    the fp32 plan and OpenMP pair loops forward and backward, window counts, exposure, epilogue, the coefficient
    adjoint; the IWE leg (transport to 0.5, OpenMP splat forward and backward, coefficient adjoint).  The
    fixed-point inversion's own backward is not included (the oracle has no position gradient of the sampler),
    so the baseline does less work than the GPU step."""
    O = _oracle()
    H, W, K = win.height, win.width, win.motion["K"]
    coeffs = np.ascontiguousarray(win.motion["coeffs"][:1])
    rng = np.random.default_rng(0)
    tab = O.traj_slice_table(K, "bspline", 16)
    g_ref, _ = O.traj_basis_table(np.array([0.5]), K, "bspline")

    def run(n):
        xy, t, b = win.xy[:n], win.t[:n], win.b[:n]
        xs = (xy + rng.uniform(-0.5, 0.5, xy.shape)).astype(np.float32)
        xa = (xs + rng.standard_normal(xs.shape)).astype(np.float32)
        p = O.traj_origin(coeffs, xs, t, b, K, "bspline")
        rows, idx, wts = O.sample_grid(coeffs, p, b)
        anchors = np.arange(n)
        plan = O.build_pair_plan_traj(p, rows, tab, t, b, 1, H, W, anchors, xa, 1.0, TRAJ_TAU, 3.0, 16)
        S = O.ats_pair_fwd(plan, 1.0, TRAJ_TAU, 3.0)
        wc = O.window_counts(t, b, anchors, TRAJ_TAU)
        vis = O.traj_visible_fraction(coeffs, xa, t, b, t, b, 1, H, W, TRAJ_TAU, K, "bspline")
        _, gS, _ = O.anchored_epilogue(S, wc, 1.0, H, W, vis=vis)
        _, gc = O.ats_pair_bwd_traj(gS, plan, tab, K, 1.0, TRAJ_TAU, 3.0, n)
        O.sample_grid_bwd(gc.astype(np.float32), idx, wts, coeffs.shape)
        q = O.traj_origin(coeffs, xy, t, b, K, "bspline")
        d, _, qidx, qwts = O.traj_displacement(coeffs, q, np.full(n, 0.5, np.float32), b, K, "bspline")
        y = q + d
        w = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(np.float32)
        img = O.splat_bilinear_fwd(y, w, b, 1, H, W)
        gimg = (2.0 / (H * W - 1)) * (img - img.mean())
        gpos, _ = O.splat_bilinear_bwd(gimg.astype(np.float32), y, w, b)
        gout = np.concatenate([g_ref * gpos[:, 1:2], g_ref * gpos[:, 0:1]], 1).astype(np.float32)
        O.sample_grid_bwd(gout, qidx, qwts, coeffs.shape)

    n, dt, _ = _bounded_run(run, int((win.b == 0).sum()), budget)
    return _baseline_line(O, n, int((win.b == 0).sum()), dt, "the trajectory step (window 0)")


# ----------------------------------------------------------------------------------------------- voxel grid
def voxel_main(a, dev):
    """voxel_grid (atl/ops/functional.py:221-238, the trainer's input, atl/train/trainer.py:136) on 1M line-segment
    events at 640x480 with 15 time bins (configs/dsec_*.yaml num_bins), polarity +-1, no normalisation: the tile
    engine (atl_voxel_grid_ws), with the per-event atomic kernel (atl_voxel_grid) timed beside it."""
    from x_amd import synth
    from x_amd.ops import _ext
    from x_amd.ops import functional as F
    win = synth.dense_flow_window(seed=0)
    rng = np.random.default_rng(0)
    pol = np.where(rng.random(win.n) > 0.5, 1.0, -1.0).astype(np.float32)
    pos, t, p, b = (torch.as_tensor(v, device=dev) for v in (win.xy, win.t, pol, win.b))
    C, H, W = 15, win.height, win.width

    def step():
        F.voxel_grid(pos, t, p, b, 1, C, H, W, normalize=None)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    rec = _ext.time_kernels(["atl_voxel_grid_ws"], every=1)
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    kms = float(np.mean([e0.elapsed_time(e1) for e0, e1, _ in rec["atl_voxel_grid_ws"]]))
    # the per-event kernel (one global atomic per corner) on the same input, for comparison
    vox = torch.zeros(1, C, H, W, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(a.steps):
        _ext.call("atl_voxel_grid", _ext.ptr(pos), _ext.ptr(t), _ext.ptr(p), _ext.ptr(b), win.n, 1, C, H, W,
                  _ext.ptr(vox), s)
    e1.record()
    torch.cuda.synchronize()
    atomic_ms = e0.elapsed_time(e1) / a.steps
    _ext.time_kernels(())
    nbytes = win.n * 24 + C * H * W * 4          # pos, t, p, b per event; the grid written once
    line = {
        "metric": "events/s for voxel_grid @1M events 640x480, 15 bins; % HBM roofline",
        "value": win.n * a.steps / dt, "unit": "events/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": 1e3 * dt / a.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "voxel_grid, 1000000 line-segment events, 640x480, 15 time bins, polarity +-1, "
                               "no normalisation", "events": win.n, "sensor": [W, H], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "atl_voxel_grid_ws", "achieved": nbytes / (kms * 1e-3) / 1e9,
                     "peak": 8000.0, "unit": "GB/s", "frac": nbytes / (kms * 1e-3) / 8e12, "traffic": None,
                     "kernel_ms": kms, "algorithmic_bytes": nbytes},
        "kernel_ms": {"atl_voxel_grid_ws": kms, "atl_voxel_grid (per-event atomics)": atomic_ms},
    }
    if not a.no_cpu:
        O = _oracle()
        n, t0 = 125_000, time.perf_counter()
        while True:
            O.voxel_grid(win.xy[:n], win.t[:n], pol[:n], win.b[:n], 1, C, H, W)
            el = time.perf_counter() - t0
            if el > a.cpu_budget / 4 or n >= win.n:
                break
            n, t0 = min(win.n, 2 * n), time.perf_counter()
        line["cpu_baseline"] = _baseline_line(O, n, win.n, el, "voxel_grid")
    print(json.dumps(line), flush=True)


# ------------------------------------------------------------------------------ MotionPriorCMax look-up table
def mpcm_lut_main(a, dev):
    """MotionPriorCMaxLoss.lut_flow at the reference's DSEC configuration (atl/objectives/mpcm.py:4-7): 480x640,
    4 px cells, tile-4 trajectories (K = 10 cubic B-splines from a smooth random coefficient grid), 15 bins,
    32 neighbours; one step = the table and the backward of its sum of squares to the coefficient grid."""
    from x_amd.motion import PixelTrajectories
    from x_amd.objectives import MotionPriorCMaxLoss
    from x_amd.ops import _ext
    g = torch.Generator().manual_seed(0)
    c = torch.nn.functional.avg_pool2d(torch.randn(1, 20, 480, 640, generator=g), 31, 1, 15, count_include_pad=False)
    coef = (c / c.abs().amax() * 25.0).to(dev).requires_grad_(True)
    loss = MotionPriorCMaxLoss()
    t_ref = torch.tensor(0.37, device=dev)

    def step():
        coef.grad = None
        table, _ = loss.lut_flow(PixelTrajectories(coef, 10, "bspline", tile=4), 480, 640, t_ref)
        table.square().sum().backward()

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    rec = _ext.time_kernels(["atl_knn_indices"], every=1)
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    kms = float(np.mean([e0.elapsed_time(e1) for e0, e1, _ in rec["atl_knn_indices"]]))
    _ext.time_kernels(())
    P, Q, n, k = 15, 120 * 160, 120 * 160, 32
    # algorithmic bytes of the KNN entry point: the points (8 B each) and queries (8 B) read, the indices written
    nbytes = P * n * 8 + Q * 8 + P * Q * k * 8
    line = {
        "metric": "look-up-table queries/s for MotionPriorCMax's KNN table fwd+bwd (15 bins x 19200 cells, k=32, "
                  "19200 trajectories); % HBM roofline of the KNN pass",
        "value": P * Q * a.steps / dt, "unit": "queries/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": 1e3 * dt / a.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "MotionPriorCMaxLoss.lut_flow, 640x480, lut 4, PixelTrajectories(K=10, bspline, tile 4), "
                               "15 bins, 32 neighbours, backward to the (1, 20, 480, 640) coefficients",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "atl_knn_indices", "achieved": nbytes / (kms * 1e-3) / 1e9,
                     "peak": 8000.0, "unit": "GB/s", "frac": nbytes / (kms * 1e-3) / 8e12, "traffic": None,
                     "kernel_ms": kms, "algorithmic_bytes": nbytes},
    }
    if not a.no_cpu:
        O = _oracle()
        with torch.no_grad():
            m = PixelTrajectories(coef.detach().cpu(), 10, "bspline", tile=4)
            edges = torch.linspace(0, 1, 16)
            pts = m.tile_trajectories((edges[:-1] + edges[1:]) * 0.5)[0].numpy()
        q = loss.cell_centres(480, 640, "cpu").numpy()
        nq, t0 = 256, time.perf_counter()
        while True:
            O.knn_indices(q[:nq], pts[:1], k)
            el = time.perf_counter() - t0
            if el > a.cpu_budget / 4 or nq >= Q:
                break
            nq, t0 = min(Q, nq * 2), time.perf_counter()
        line["cpu_baseline"] = dict({"value": nq / el, "unit": "queries/s", "cores": 1, "kind": "port",
                                     "sample": f"the oracle's brute-force KNN (NumPy, one thread) of {nq} cells on "
                                               f"one bin's 19200 trajectories, {el:.2f} s (the table's gather and "
                                               f"backward not included)"}, **_host_cpu())
    print(json.dumps(line), flush=True)


def main():
    a = parse()
    if a.summarize:
        summarize(a.summarize, a.out, a.title, a.command, a.copy_mb, a.calibration, a.pairs)
        return
    if a.calibrate_copy > 0:
        calibrate_copy(a.calibrate_copy)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {a.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    if a.workload.startswith("iwe") or a.workload in ("trajectories", "mpcm-lut", "voxel"):
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        {"trajectories": trajectories_main, "mpcm-lut": mpcm_lut_main, "voxel": voxel_main}.get(a.workload, iwe_main)(a, dev)
        return
    from x_amd.objectives import AnchoredExact
    from x_amd.ops import _ext
    from x_amd.ops import functional as F
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_events = a.events if a.events else (4_000_000 if a.workload == "anchored-blobs" else 1_000_000)
    win, ev, motion, desc = workload(a.workload, n_events, dev)
    obj = AnchoredExact(h=a.sigma, tau=0.2, cut=3.0, n_slices=16, n_anchors=None, seed=0, rng="device")
    blobs = a.workload == "anchored-blobs"
    reflayout = a.workload == "anchored-reflayout"
    if reflayout:                                  # the reference's call: v from the flow, then plan + pair sums
        def ref_pair_sums(ev_, motion_, xs, xa, anchors):
            v = motion_.velocity(xs, ev_.t, ev_.b)
            return F.ats_pair_sums_reference_layout(xs, ev_.t, v, ev_.b, ev_.batch_size, ev_.height, ev_.width,
                                                    anchors, obj.h, obj.tau, obj.cut, obj.n_slices, anchor_xy=xa)
        obj._pair_sums = ref_pair_sums
    if blobs:
        from x_amd.objectives import iwe_variance

    def step():
        for prm in motion.parameters():
            prm.grad = None
        # one layout scope per step: the flow's interleaved copy is made once per step
        with F.layout_scope():
            loss = obj(ev, motion)["loss"]
            if blobs:                              # the splat leg of the contention config: IWE contrast at 0.5
                loss = loss - iwe_variance(ev, motion, 0.5)
        loss.backward()

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    # the pair kernels first (the roofline's candidates); the objective's dense flow takes the flow path, whose
    # backward is the pair backward (atl_fast_pair_bwd_src) and then the flow-grid adjoint
    kernels = (["atl_ats_pair_fwd_ws", "atl_ats_pair_bwd_ws_binned"] if reflayout else
               ["atl_fast_pair_fwd", "atl_fast_pair_bwd_src", "atl_fast_flow_adjoint"]) + (
        ["atl_splat_bilinear_fwd_ws", "atl_splat_bilinear_bwd"] if blobs else [])
    rec = _ext.time_kernels(kernels, every=4)      # every bracket delays the next launch: sample the steps
    first_draw = obj._philox[1]
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = {k: float(np.mean([e0.elapsed_time(e1) for e0, e1, _ in rec[k]])) for k in kernels}
    _ext.time_kernels(())
    kernels = kernels[:2]                          # the roofline's candidates: the pair kernels
    # contributing pairs K = sum_i n_i of the timed steps' own noise draws (counted outside the timed region)
    pairs = []
    with torch.no_grad():
        for draw in range(first_draw, first_draw + a.steps):
            xs, xa = F.event_noise(ev.xy, 0, draw, a.sigma)
            v = motion.velocity(xs, ev.t, ev.b)
            plan = F.FastPairPlan(xs, ev.t, v, ev.b, 1, ev.height, ev.width, None, a.sigma, 0.2, 3.0, 16,
                                  anchor_xy=xa)
            pairs.append(int(plan.counts().sum()))
    K = float(np.mean(pairs))
    dom = max(kernels, key=lambda k: ms[k])
    fwd = "_fwd" in dom
    slots = SLOTS_FWD if fwd else SLOTS_BWD
    achieved = K * slots / (ms[dom] * 1e-3)
    flops = K * (FLOPS_FWD if fwd else FLOPS_BWD) / (ms[dom] * 1e-3)
    value = ev.n * a.steps / dt
    # whole-step roofline: every contributing pair at its forward + backward slots on the VALU, plus the step's
    # compulsory bytes at HBM peak (flow grid read and gradient written, twice 2 x 4 x Hg x Wg bytes)
    hw = ev.height * ev.width
    step_bytes = ev.n * (STEP_BYTES_PER_EVENT + (SPLAT_BYTES_PER_EVENT if blobs else 0)) + 16 * hw \
        + (8 * hw if blobs else 0)
    step_roof_s = K * (SLOTS_FWD + SLOTS_BWD) / VALU_PEAK + step_bytes / HBM_PEAK
    line = {
        "metric": ("events/s for anchored-score fwd+bwd @1M events 640x480; % HBM/VALU roofline"
                   if a.workload == "anchored" else
                   "events/s for anchored-score fwd+bwd @1M events 640x480 through the reference-layout pair "
                   "entry points; % VALU roofline" if reflayout else
                   f"events/s for anchored-score (pair-sum + splat) fwd+bwd @{ev.n} events 640x480 blobs; "
                   f"% VALU roofline"),
        "value": value, "unit": "events/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": 1e3 * dt / a.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{desc}, h={a.sigma}, tau=0.2, cut=3, S=16, all anchors"
                               + (", pair sums through the reference layout (ats_pair_fwd/bwd)" if reflayout else "")
                               + (", minus the IWE variance at t=0.5 (bilinear splat fwd+bwd)" if blobs else ""),
                   "events": ev.n, "sensor": [640, 480], "sigma": a.sigma, "tau": 0.2, "slices": 16,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "kernel": dom, "achieved": achieved / 1e12, "peak": VALU_PEAK / 1e12,
                     "unit": "Tslot/s", "frac": achieved / VALU_PEAK,
                     # the committed counters are for this exact workload only (1M events, h = 1)
                     "traffic": (recorded_traffic(KERNEL_OF[dom]) if a.workload == "anchored" and a.sigma == 1.0
                                 and ev.n == 1_000_000 else None),
                     "pairs": K, "slots_per_pair": slots, "kernel_ms": ms[dom],
                     "step_roof_ms": step_roof_s * 1e3, "step_frac": step_roof_s / (dt / a.steps),
                     "step_bytes": step_bytes,
                     "flop_view": {"achieved": flops / 1e12, "peak": FP32_PEAK / 1e12, "unit": "TFLOP/s",
                                   "frac": flops / FP32_PEAK}},
        "kernel_ms": ms,
        "pairs_per_anchor": K / ev.n,
    }
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline(win, a.sigma, a.cpu_budget, splat_leg=blobs)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
