#!/usr/bin/env python3
"""SO3LR MD throughput on one MI355X: atom-steps/s at the 24,000-atom NaCl
solution, fp64 E + F + virial every step.

One step = velocity Verlet with a Berendsen thermostat at 300 K (0.5 fs),
ghost-row update, neighbour-list rebuild when an atom moved more than half the
1 A skin (LAMMPS `neigh_modify every 1 delay 0 check yes`), and one
so3lr_compute_device call.  Positions, velocities and forces stay in HBM
(torch tensors as plumbing); the rebuild wraps the positions and builds the
candidate lists on the GPU (so3lr_reneighbor_device).

Prints one JSON line (the driver's contract), with the dominant kernel's
roofline from HIP events recorded on its launch stream, and the CPU oracle
timed on the same host on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

MODEL = os.path.join(REPO, "models", "so3lr.so3lr")
A100_ATOM_STEPS = 69706.0  # the reference's published 24k-atom water figure on 1 A100 (examples/scaling/README.md:56-60)
HBM_PEAK_GBS = 8000.0
FP64_PEAK_TFS = 78.6
# algorithmic work of the dominant kernel, per active short-range pair and block
# (filters: 2 x (32x128 + 128x128 + 4x32 + 32x128) MAC, forward)
FILTER_FWD_FLOP_PER_PAIR = 2.0 * 2.0 * (32 * 128 + 128 * 128 + 4 * 32 + 32 * 128)
# reverse: dgrad of W1 (128x128), E1 (128x32), W0 (128x32), E0 (32x4) plus the
# layer-0 recompute (32x128 + 4x32), both filters
FILTER_BWD_FLOP_PER_PAIR = 2.0 * 2.0 * (128 * 128 + 128 * 32 + 128 * 32 + 32 * 4 + 32 * 128 + 4 * 32)
KB = 8.617333262e-5
ACC = 9648.533212  # eV / (A amu) -> A / ps^2


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def traffic_bytes(kernel, config):
    """HBM bytes per launch (read + written) of `kernel` from the committed
    PMC summary (two rocprofv3 passes, FETCH_SIZE and WRITE_SIZE, scaled by a
    plain copy of known size); None when no summary covers this workload."""
    path = os.path.join(REPO, "profiles", "pmc_traffic_config%d.json" % config)
    try:
        rec = json.load(open(path))["kernels"][kernel]
    except (OSError, KeyError, ValueError):
        return None
    return rec["read_bytes"] + rec["write_bytes"]


def cpu_baseline(z, x, box, periodic, images, seconds_budget):
    """Oracle (CPU restatement of the reference math, OpenMP) timed on the
    host cores: repeated E+F+virial calls on a bounded sample of the same
    workload until about `seconds_budget` seconds of CPU work are done;
    reports the median call as atom-steps/s."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from oracle.oracle import Oracle, lib
    import support
    orc = Oracle(MODEL)
    kw = {}
    if images is not None:
        # the first 64 molecules of the packed batch, with their own (Q, M)
        offs, qs, ms = images
        k = min(64, len(qs))
        zs, xs = z[:offs[k]], x[:offs[k]]
        kw = dict(image=np.repeat(np.arange(k), np.diff(offs[:k + 1])), image_charge=np.asarray(qs[:k], float),
                  image_multiplicity=ms[:k])
        sr, lr = support.build_graphs(xs, None)
        what = "the first %d molecules of the packed batch (open boundaries)" % k
    elif not any(periodic):
        zs, xs = z, x
        sr, lr = support.build_graphs(xs, None)
        what = "the whole molecule (open boundaries)"
    else:
        # every atom of a 40 A cube cut from the system, treated as periodic
        # with that side (wider than twice the 12 A LR cutoff)
        side = 40.0
        sel = np.all(x < side, axis=1)
        zs, xs = z[sel], x[sel]
        sr, lr = support.build_graphs(xs, np.full(3, side))
        what = "a %.0f A periodic sub-cube of the benchmark system" % side
        if int(np.sum(zs)) % 2:
            kw = dict(multiplicity=2.0)  # a cut that leaves an odd electron count
    orc.evaluate(zs, sr, lr, **kw)  # warm-up (page-in, thread pool)
    times = []
    t_start = time.time()
    while len(times) < 3 or (time.time() - t_start < seconds_budget and len(times) < 1000):
        t0 = time.time()
        orc.evaluate(zs, sr, lr, **kw)
        times.append(time.time() - t0)
    med = float(np.median(times))
    return {"value": len(zs) / med, "unit": "atom-steps/s", "cores": int(lib().orc_num_threads()),
            "kind": "port",
            "sample": "median of %d E+F+virial calls (%.1f s of CPU work) on %d atoms: %s, CPU fp64 oracle, OpenMP"
                      % (len(times), sum(times), len(zs), what)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--roofline-steps", type=int, default=10,
                    help="steps after the timed ones with per-kernel HIP events")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain device copy of this size first (HBM-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs one LAMMPS rank on one MI355X with no "
              "GPU-to-GPU exchange (--gpus %d is not supported)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch
    from so3lrxlammps_amd import Context, Lists, systems

    log("generating config %d" % args.config)
    images = None
    if args.config == 2:
        # 512 independent molecules evaluated together (packed images)
        z, x, offs, qs, ms, extent = systems.packed_molecules()
        images = (offs, qs, ms)
        box, Q, M = np.full(3, extent), None, None
        desc = "512 molecules of 12-40 atoms (H C N O S), Q in {-1,0,1}, packed images, non-periodic"
    else:
        z, x, box, Q, M, desc = systems.config(args.config)
        if box is None:  # config 0: the molecule in its 40 A box, open boundaries
            box = np.full(3, 40.0)
    periodic = (0, 0, 0) if args.config in (0, 2) else (1, 1, 1)
    n = len(z)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    # an explicit stream: handle 0 (torch's default) would leave the library on its own stream
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    if args.copy_probe_mib > 0:
        # a plain copy of known size: FETCH_SIZE / WRITE_SIZE of this kernel
        # give the counters' scale against true HBM bytes
        with torch.cuda.stream(stream):
            src = torch.ones(args.copy_probe_mib << 17, dtype=torch.float64, device=dev)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    ctx = Context(MODEL, 0)
    if images is not None:
        ctx.set_images(z, *images)
    else:
        ctx.set_system(z, Q, M)
    lo = np.zeros(3)
    v0, m = systems.maxwell_boltzmann(z, 300.0)
    xt = torch.tensor(x, dtype=torch.float64, device=dev)
    vt = torch.tensor(v0, dtype=torch.float64, device=dev)
    inv_m = torch.tensor(ACC / m, dtype=torch.float64, device=dev)[:, None]
    mt = torch.tensor(m, dtype=torch.float64, device=dev)[:, None]
    ft = torch.zeros((n, 3), dtype=torch.float64, device=dev)
    lot = torch.tensor(lo, dtype=torch.float64, device=dev)
    dt, skin, tau, T0 = 0.0005, 1.0, 0.1, 300.0
    # config 4 runs NPT: Berendsen barostat at 1 bar (water compressibility)
    npt = args.config == 4
    P0_bar, tau_p, beta_bar = 1.0, 1.0, 4.5e-5
    EV_A3_TO_BAR = 1.602176634e6
    state = {"builds": 0, "build_s": 0.0, "box": np.array(box, dtype=float), "mu_total": 1.0}

    def rebuild():
        # HBM-resident reneighbor: wraps xt in place, builds the candidate
        # lists on the GPU (no ghost rows, no host copies)
        t0 = time.time()
        ctx.reneighbor_device(xt, lo, lo + state["box"], periodic, skin, stream=stream.cuda_stream)
        state["x_build"] = xt.clone()
        state["box_build"] = state["box"].copy()
        state["builds"] += 1
        state["build_s"] += time.time() - t0

    def force():
        e, w = ctx.compute_device(xt, ft, stream=stream.cuda_stream)
        return e, w

    rebuild()
    e, w = force()

    # config 0: repeated single points; 1 and 2: NVE; 3: NVT; 4: NPT
    single_point = args.config == 0
    thermostat = args.config in (3, 4)

    def step():
        if single_point:
            return force()
        vt.addcmul_(ft, inv_m, value=0.5 * dt)
        xt.add_(vt, alpha=dt)
        disp = (xt - state["x_build"]).norm(dim=1).max().item()
        # a box change moves the far corner: LAMMPS Neighbor::check_distance
        # charges that against the skin as well
        disp += float(np.linalg.norm(state["box"] - state["box_build"]))
        if disp > 0.5 * skin:
            rebuild()
        e, w = force()
        vt.addcmul_(ft, inv_m, value=0.5 * dt)
        ke = 0.5 * (mt * vt * vt).sum() / ACC
        if thermostat:
            temp = 2.0 * ke / (3.0 * n * KB)
            lam = torch.sqrt(1.0 + dt / tau * (T0 / temp - 1.0))
            vt.mul_(lam)
        if npt:
            # P = (2 KE + tr W) / (3 V); W is the LAMMPS virial (eV)
            vol = float(np.prod(state["box"]))
            p_bar = (2.0 * ke.item() + w[0] + w[1] + w[2]) / (3.0 * vol) * EV_A3_TO_BAR
            mu = (1.0 - dt / tau_p * beta_bar * (P0_bar - p_bar)) ** (1.0 / 3.0)
            xt.sub_(lot).mul_(mu).add_(lot)
            state["box"] = state["box"] * mu
            state["mu_total"] *= mu
            state["pressure_bar"] = p_bar
            ctx.set_box(lo, lo + state["box"])
        return e, w

    log("warmup %d steps" % args.warmup)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    builds0, build_s0 = state["builds"], state["build_s"]
    log("timing %d steps" % args.steps)
    t0 = time.perf_counter()
    for k in range(args.steps):
        e, w = step()
        if (k + 1) % 25 == 0:
            log("  step %d E=%.6f eV" % (k + 1, e))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = n * args.steps / elapsed
    builds_timed, build_s_timed = state["builds"] - builds0, state["build_s"] - build_s0

    # kernel durations for the roofline: HIP events on the launch stream over
    # further steps of the same run (events keep the evaluation out of graph
    # replay, so they are not recorded during the timed steps above)
    ctx.kernel_timing(True)
    for _ in range(args.roofline_steps):
        step()
    torch.cuda.synchronize()
    ctx.kernel_timing(False)

    # dominant kernel: the pair filters (forward + reverse) carry ~90% of the
    # FLOPs; the roofline is the reverse filter of blocks 1.. (block 0 runs a
    # cheaper instantiation, ev = 0, timed under its own name)
    timing = {}
    for name in ("filter_fwd", "filter_fwd_block0", "filter_bwd", "filter_bwd_block0", "attn_fwd", "attn_bwd",
                 "attn_bwd_block0", "long_range"):
        try:
            timing[name] = ctx.kernel_timing_read(name)
        except Exception:  # kernel not launched
            pass
    free_b, total_b = torch.cuda.mem_get_info(dev)
    ms_f, launches_f, pairs_f = timing["filter_bwd"]
    avg_ms = ms_f / launches_f
    flop = FILTER_BWD_FLOP_PER_PAIR * pairs_f / launches_f
    achieved = flop / (avg_ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": "k_filter_bwd_mfma<false>", "achieved": achieved, "peak": FP64_PEAK_TFS,
                "unit": "TFLOP/s", "frac": achieved / FP64_PEAK_TFS,
                "traffic": traffic_bytes("k_filter_bwd_mfma<false>", args.config),
                "avg_launch_ms": avg_ms, "pairs_per_launch": pairs_f / launches_f,
                "flop_per_pair": FILTER_BWD_FLOP_PER_PAIR}
    kernels = {k: {"avg_ms": v[0] / v[1], "launches": v[1]} for k, v in timing.items()}

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(z, x, box, periodic, images, args.cpu_budget)

    sr_active, sr_cand, lr_cand = ctx.graph_stats()
    if npt:
        extra = {"ensemble": "NPT (Berendsen, 1 bar, 300 K)", "box_scale": state["mu_total"],
                 "pressure_bar_last": state.get("pressure_bar")}
    elif single_point:
        extra = {"ensemble": "single-point E+F+virial calls"}
    elif thermostat:
        extra = {"ensemble": "NVT (Berendsen, 300 K)"}
    else:
        extra = {"ensemble": "NVE"}
    out = {
        "metric": "atom-steps/s/GPU (fp64 E+F+virial) at 24k-atom water; max atoms per GPU",
        "value": value, "unit": "atom-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": value / A100_ATOM_STEPS, "dtype": "f64", "data": "synthetic (seeded, config %d)" % args.config,
        "config": {"workload": "config 3: " + desc, "atoms": n, "integrator": "velocity Verlet", **extra,
                   "timestep_fs": 0.5, "skin_A": skin, "sr_pairs_active": sr_active,
                   "sr_pair_candidates": sr_cand, "lr_pair_candidates": lr_cand,
                   "neighbor_rebuilds_timed": builds_timed,
                   "rebuild_seconds_timed": build_s_timed,
                   "ns_per_day": value / n * 0.5 * 86400 / 1e6,
                   "device_bytes": ctx.device_bytes(),
                   "hbm_used_bytes": int(total_b - free_b), "hbm_total_bytes": int(total_b),
                   "kernels": kernels},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
