#!/usr/bin/env python3
"""SO3LR MD throughput on one MI355X: atom-steps/s at the 24,000-atom NaCl
solution, fp64 E + F + virial every step; and the
metric's second half, max atoms per GPU, from the 150,000-atom water box
(configs[4]) run in the same process.

Headline (`value`): one step = velocity Verlet with a Berendsen thermostat at
300 K (0.5 fs), a neighbour-list rebuild when an atom moved more than half the
1 A skin (LAMMPS `neigh_modify every 1 delay 0 check yes`), and one
so3lr_compute_device call.  Positions, velocities and forces stay in HBM
(torch tensors as plumbing); the rebuild wraps the positions and builds the
candidate lists on the GPU (so3lr_reneighbor_device).

`rows_path`: the drop-in route a LAMMPS pair style takes, timed on the same
system: host positions, the LAMMPS stand-in's ghost rows and candidate lists
at every rebuild (LAMMPS's own work, reported apart), so3lr_set_topology with
those lists, then so3lr_compute with host arrays every step.

`capacity`: config 4 (150,000 atoms) NPT steps with hipMemGetInfo before and
after, the library's device bytes and bytes per atom.

`roofline`: the kernel with the most GPU time per step among the timed ones,
its algorithmic work per unit (no recompute) / its HIP-event average on the
launch stream.  `cpu_baseline`: the CPU oracle on a bounded sample.
Prints one JSON line (the driver's contract).
"""
import argparse
import json
import os
import platform
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

MODEL = os.path.join(REPO, "models", "so3lr.so3lr")
A100_ATOM_STEPS = 69706.0  # the reference's published 24k-atom water figure on 1 A100 (examples/scaling/README.md:56-60)
HBM_PEAK_GBS = 8000.0
FP64_PEAK_TFS = 78.6
KB = 8.617333262e-5
ACC = 9648.533212  # eV / (A amu) -> A / ps^2


def _mac(*shapes):
    return sum(a * b for a, b in shapes)


# Algorithmic work per unit of each timed kernel: minimal forward and
# input-gradient work, no recompute (units: active SR pairs for the filters,
# owned atoms otherwise).  "issued" is what the kernel executes when that
# differs (the reverse filters recompute the layer-0 pre-activations).
# Filters, per pair and block, both filters (F = 128, R = 32, F/4 = 32):
#   forward  radial W0 (128x32) + W1 (128x128), spherical E0 (32x4) + E1 (128x32);
#   reverse  the transposes of the same four layers (input gradients only).
_FILTER = 2 * 2 * _mac((128, 32), (128, 128), (32, 4), (128, 32))   # 98,816 flop
_FILTER_B0 = 2 * 2 * _mac((128, 32), (128, 128))                     # 81,920: ev = 0 in block 0
_FILTER_BWD_ISSUED = _FILTER + 2 * 2 * _mac((128, 32), (32, 4))      # + layer-0 recompute: 115,712
_FILTER_BWD_B0_ISSUED = _FILTER_B0 + 2 * 2 * _mac((128, 32))         # 98,304
# block 0 through element-pair tables: W0 (128x32) and 8 table rows of 128
# (4 heads x 2 directions) per filter; the reverse recomputes W0's output
_FILTER_B0_TAB = 2 * 2 * _mac((128, 32), (8, 128))                    # 20,480
_FILTER_BWD_B0_TAB_ISSUED = _FILTER_B0_TAB + 2 * 2 * _mac((128, 32))  # 36,864
# Blocks after 0 on their radial tables: the radial branch W1 silu(W0 rbf +
# b0) + ob1 of each filter is a fitted polynomial of r (32 coefficients per
# channel), so the forward is bound by its rows: per pair it must write the
# filter rows (2 x 128 doubles), the logits (16) and s (4), and read r and
# the endpoints (algorithmic bytes).  The reverse contracts df with the slope
# polynomials (14 x 128 per filter at the accuracy of degree 13; 32 x 128
# issued) and runs the spherical branch's transposes: E1^T (32x128), E0^T (4x32).
_FILTER_RT_BYTES = 8 * (256 + 16 + 4) + 8 + 8                        # 2,224 B
_FILTER_BWD_RT = 2 * 2 * _mac((14, 128), (32, 128), (4, 32))          # 24,064 flop
_FILTER_BWD_RT_ISSUED = 2 * 2 * _mac((32, 128), (32, 128), (4, 32))   # 33,280: 32 powers
KERNEL_WORK = {
    # name: (kernel symbol, bound, algorithmic per unit, issued per unit, unit)
    # (bound "hbm": bytes per unit; "mfma": flop per unit)
    "filter_fwd_radial": ("k_radial_fwd_rows", "hbm", _FILTER_RT_BYTES, _FILTER_RT_BYTES, "pair"),
    "filter_bwd_radial": ("k_filter_bwd_mfma<false, false, true>", "mfma", _FILTER_BWD_RT, _FILTER_BWD_RT_ISSUED,
                          "pair"),
    "filter_fwd": ("k_filter_fwd_mfma<false>", "mfma", _FILTER, _FILTER, "pair"),
    "filter_fwd_block0": ("k_filter_fwd_mfma<true>", "mfma", _FILTER_B0, _FILTER_B0, "pair"),
    "filter_bwd": ("k_filter_bwd_mfma<false, false>", "mfma", _FILTER, _FILTER_BWD_ISSUED, "pair"),
    "filter_bwd_block0": ("k_filter_bwd_mfma<true, false>", "mfma", _FILTER_B0, _FILTER_BWD_B0_ISSUED, "pair"),
    "filter_fwd_block0_tables": ("k_filter_fwd_class", "mfma", _FILTER_B0_TAB, _FILTER_B0_TAB, "pair"),
    "filter_bwd_block0_tables": ("k_filter_bwd_class<false>", "mfma", _FILTER_B0_TAB, _FILTER_BWD_B0_TAB_ISSUED,
                                 "pair"),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_info():
    model = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"cpu_model": model, "nproc": affinity, "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS")}


def traffic_per_launch(kernel, config, units_per_launch):
    """HBM bytes per launch of `kernel` from the committed PMC summary (two
    rocprofv3 passes, FETCH_SIZE and WRITE_SIZE, scaled by a plain copy of
    known size), rescaled to this run's units per launch; None when the
    summary does not cover this kernel and workload."""
    path = os.path.join(REPO, "profiles", "pmc_traffic_config%d.json" % config)
    try:
        doc = json.load(open(path))
        rec = doc["kernels"][kernel]
        per_unit = (rec["read_bytes"] + rec["write_bytes"]) / rec.get("units_per_launch", doc["pairs_per_launch"])
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None, None
    return per_unit * units_per_launch, "profiles/pmc_traffic_config%d.json: %.0f B per %s, x this run's count" % (
        config, per_unit, KERNEL_WORK_UNIT.get(kernel, "unit"))


KERNEL_WORK_UNIT = {v[0]: v[4] for v in KERNEL_WORK.values()}


def kernel_work(widths, elements=0):
    """KERNEL_WORK plus the generic-width filter sections of a model on the
    generic kernels: per active pair and block, both filters, algorithmic
    2 (R F + NH F/4 + (F + F/4) F) MAC each way; the reverse also issues the
    hidden row's recompute (R F + NH F/4).  Block 0 through the element-pair
    tables (`elements` > 0: g_b0_fwd, g_b0_bwd): 2 (R F + 2 NH F) MAC each
    way; the forward issues the table rows padded to 16 (16 F), the reverse
    R F more for the recompute."""
    work = dict(KERNEL_WORK)
    F, R = widths["invariant_features"], widths["radial_basis_features"]
    NH, FH = len(widths["degree_slots"]), widths["invariant_features"] // 4
    alg = 2 * 2 * (R * F + NH * FH + (F + FH) * F)
    work["generic_filter_fwd"] = ("g_filt_fwd: both filters and the logits, fused", "mfma", alg, alg, "pair")
    work["generic_filter_bwd"] = ("g_filt_bwd: both filters' reverse, fused", "mfma", alg,
                                  alg + 2 * 2 * (R * F + NH * FH), "pair")
    # the blocks after 0 on their radial tables: bound by the rows, 2 F
    # doubles written per pair with the 4 NH logits and NH invariants (the
    # invariants are read back), r and the endpoints read
    rt_bytes = 8 * (2 * F + 4 * NH + NH) + 16
    work["generic_filter_fwd_radial"] = ("g_radial_fwd_rows", "hbm", rt_bytes, rt_bytes, "pair")
    # and the reverse: df against the slope polynomials (14 powers per
    # channel at the accuracy of degree 13; 32 issued), E1^T, E0^T
    rt_bwd = 2 * 2 * (14 * F + FH * F + NH * FH)
    work["generic_filter_bwd_radial"] = ("g_radial_bwd_rows", "mfma", rt_bwd, 2 * 2 * (32 * F + FH * F + NH * FH),
                                         "pair")
    if elements:
        tab = 2 * 2 * (R * F + 2 * NH * F)
        work["generic_filter_fwd_block0_tables"] = ("g_b0_fwd: block 0's fused table filters", "mfma", tab,
                                                    2 * 2 * (R * F + 16 * F), "pair")
        work["generic_filter_bwd_block0_tables"] = ("g_b0_bwd: block 0's fused table filters, reverse", "mfma", tab,
                                                    tab + 2 * 2 * R * F, "pair")
    return work


def cpu_baseline(z, x, box, periodic, images, seconds_budget):
    """Oracle (CPU restatement of the reference math, OpenMP) timed on the
    host cores: for a periodic configuration the whole system, the median of
    5 E+F+virial calls after 2 warm-ups; otherwise repeated calls on a
    bounded sample until about `seconds_budget` seconds of CPU work are
    done.  Reports the median call as atom-steps/s."""
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
        # the whole periodic system, its graphs from the LAMMPS stand-in's
        # lists: the median of 5 calls after 2 warm-ups
        from so3lrxlammps_amd import Lists
        zs, xs = z, x
        sr, lr = support.graphs_from_lists(Lists(xs, np.zeros(3), box, periodic), xs)
        what = "the whole periodic benchmark system"
    times = []
    if any(periodic):
        for k in range(7):
            t0 = time.time()
            orc.evaluate(zs, sr, lr, **kw)
            if k >= 2:
                times.append(time.time() - t0)
    else:
        orc.evaluate(zs, sr, lr, **kw)  # warm-up (page-in, thread pool)
        t_start = time.time()
        while len(times) < 3 or (time.time() - t_start < seconds_budget and len(times) < 1000):
            t0 = time.time()
            orc.evaluate(zs, sr, lr, **kw)
            times.append(time.time() - t0)
    med = float(np.median(times))
    out = {"value": len(zs) / med, "unit": "atom-steps/s", "cores": int(lib().orc_num_threads()),
           "kind": "port",
           "sample": "median of %d E+F+virial calls (%.1f s of CPU work) on %d atoms: %s, CPU fp64 oracle, OpenMP"
                     % (len(times), sum(times), len(zs), what)}
    out.update(cpu_info())
    return out


def load_config(index):
    from so3lrxlammps_amd import systems
    images = None
    if index == 2:
        z, x, offs, qs, ms, extent = systems.packed_molecules()
        images = (offs, qs, ms)
        box, Q, M = np.full(3, extent), None, None
        desc = "512 molecules of 12-40 atoms (H C N O S), Q in {-1,0,1}, packed images, non-periodic"
    else:
        z, x, box, Q, M, desc = systems.config(index)
        if box is None:  # config 0: the molecule in its 40 A box, open boundaries
            box = np.full(3, 40.0)
    periodic = (0, 0, 0) if index in (0, 2) else (1, 1, 1)
    return z, x, np.asarray(box, float), Q, M, images, periodic, desc


class DeviceMD:
    """The HBM-resident MD loop on one context (config 0: repeated single
    points; 1 and 2: NVE; 3: NVT; 4: NPT with a Berendsen barostat)."""

    def __init__(self, index, z, x, box, Q, M, images, periodic, stream):
        import torch
        from so3lrxlammps_amd import Context, systems
        self.torch = torch
        self.index = index
        self.stream = stream
        dev = torch.device("cuda:0")
        self.ctx = Context(MODEL, 0)
        if images is not None:
            self.ctx.set_images(z, *images)
        else:
            self.ctx.set_system(z, Q, M)
        self.n = len(z)
        self.periodic = periodic
        self.lo = np.zeros(3)
        v0, m = systems.maxwell_boltzmann(z, 300.0)
        self.xt = torch.tensor(x, dtype=torch.float64, device=dev)
        self.vt = torch.tensor(v0, dtype=torch.float64, device=dev)
        self.inv_m = torch.tensor(ACC / m, dtype=torch.float64, device=dev)[:, None]
        self.mt = torch.tensor(m, dtype=torch.float64, device=dev)[:, None]
        self.ft = torch.zeros((self.n, 3), dtype=torch.float64, device=dev)
        self.lot = torch.tensor(self.lo, dtype=torch.float64, device=dev)
        self.dt, self.skin, self.tau, self.T0 = 0.0005, 1.0, 0.1, 300.0
        self.npt = index == 4
        self.single_point = index == 0
        self.thermostat = index in (3, 4)
        self.P0_bar, self.tau_p, self.beta_bar = 1.0, 1.0, 4.5e-5
        self.state = {"builds": 0, "build_s": 0.0, "box": np.array(box, dtype=float), "mu_total": 1.0}
        self.rebuild()
        self.force()

    def rebuild(self):
        # HBM-resident reneighbor: wraps xt in place, builds the candidate
        # lists on the GPU (no ghost rows, no host copies)
        st = self.state
        t0 = time.time()
        self.ctx.reneighbor_device(self.xt, self.lo, self.lo + st["box"], self.periodic, self.skin,
                                   stream=self.stream.cuda_stream)
        st["x_build"] = self.xt.clone()
        st["box_build"] = st["box"].copy()
        st["builds"] += 1
        st["build_s"] += time.time() - t0

    def force(self):
        return self.ctx.compute_device(self.xt, self.ft, stream=self.stream.cuda_stream)

    def step(self):
        torch, st, dt = self.torch, self.state, self.dt
        if self.single_point:
            return self.force()
        self.vt.addcmul_(self.ft, self.inv_m, value=0.5 * dt)
        self.xt.add_(self.vt, alpha=dt)
        disp = (self.xt - st["x_build"]).norm(dim=1).max().item()
        # a box change moves the far corner: LAMMPS Neighbor::check_distance
        # charges that against the skin as well
        disp += float(np.linalg.norm(st["box"] - st["box_build"]))
        if disp > 0.5 * self.skin:
            self.rebuild()
        e, w = self.force()
        self.vt.addcmul_(self.ft, self.inv_m, value=0.5 * dt)
        ke = 0.5 * (self.mt * self.vt * self.vt).sum() / ACC
        if self.thermostat:
            temp = 2.0 * ke / (3.0 * self.n * KB)
            self.vt.mul_(torch.sqrt(1.0 + dt / self.tau * (self.T0 / temp - 1.0)))
        if self.npt:
            # P = (2 KE + tr W) / (3 V); W is the LAMMPS virial (eV)
            vol = float(np.prod(st["box"]))
            p_bar = (2.0 * ke.item() + w[0] + w[1] + w[2]) / (3.0 * vol) * 1.602176634e6
            mu = (1.0 - dt / self.tau_p * self.beta_bar * (self.P0_bar - p_bar)) ** (1.0 / 3.0)
            self.xt.sub_(self.lot).mul_(mu).add_(self.lot)
            st["box"] = st["box"] * mu
            st["mu_total"] *= mu
            st["pressure_bar"] = p_bar
            self.ctx.set_box(self.lo, self.lo + st["box"])
        return e, w

    def run(self, warmup, steps, report_every=25):
        for _ in range(warmup):
            self.step()
        self.torch.cuda.synchronize()
        b0, s0 = self.state["builds"], self.state["build_s"]
        t0 = time.perf_counter()
        for k in range(steps):
            e, w = self.step()
            if (k + 1) % report_every == 0:
                log("  step %d E=%.6f eV" % (k + 1, e))
        self.torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        return elapsed, self.state["builds"] - b0, self.state["build_s"] - s0

    def ensemble(self):
        if self.npt:
            return {"ensemble": "NPT (Berendsen, 1 bar, 300 K)", "box_scale": self.state["mu_total"],
                    "pressure_bar_last": self.state.get("pressure_bar")}
        if self.single_point:
            return {"ensemble": "single-point E+F+virial calls"}
        return {"ensemble": "NVT (Berendsen, 300 K)" if self.thermostat else "NVE"}


def rows_path(z, x, box, Q, M, periodic, steps, warmup):
    """The LAMMPS pair-style route on host arrays: NVT velocity Verlet in
    numpy; at every rebuild the stand-in wraps the owned atoms, makes the ghost
    rows and the full SR / half LR candidate lists (LAMMPS's work, timed
    apart), then so3lr_set_topology; every step the ghost rows' positions
    (LAMMPS forward communication) and so3lr_compute with host arrays."""
    from so3lrxlammps_amd import Context, Lists, systems
    ctx = Context(MODEL, 0)
    ctx.set_system(z, Q, M)
    n = len(z)
    lo, hi = np.zeros(3), np.asarray(box, float)
    v, m = systems.maxwell_boltzmann(z, 300.0)
    inv_m = (ACC / m)[:, None]
    x = np.array(x, dtype=float)
    dt, skin, tau, T0 = 0.0005, 1.0, 0.1, 300.0
    t = {"lammps_lists": 0.0, "set_topology": 0.0, "forward_comm": 0.0, "compute": 0.0, "rebuilds": 0,
         "compute_first": 0.0, "compute_first_n": 0}
    st = {"fresh": False}

    def rebuild():
        t0 = time.perf_counter()
        np.copyto(x, lo + np.mod(x - lo, hi - lo))  # LAMMPS Domain::pbc at reneighbor
        lists = Lists(x, lo, hi, periodic)
        t1 = time.perf_counter()
        ctx.set_topology(lists)
        t2 = time.perf_counter()
        t["lammps_lists"] += t1 - t0
        t["set_topology"] += t2 - t1
        t["rebuilds"] += 1
        st["lists"], st["x_build"] = lists, x.copy()
        st["fresh"] = True  # the next compute is the topology's first

    # the output arrays persist across steps, as a pair style's do
    out = (np.zeros((n, 3)), np.zeros(n))

    def force():
        t0 = time.perf_counter()
        xr = st["lists"].rows_positions(x)
        t1 = time.perf_counter()
        e, f, _, w = ctx.compute(xr, eatom=False, out=out)  # f is out[0]: used before the next call
        t2 = time.perf_counter()
        t["forward_comm"] += t1 - t0
        t["compute"] += t2 - t1
        if st["fresh"]:
            t["compute_first"] += t2 - t1
            t["compute_first_n"] += 1
            st["fresh"] = False
        return e, f, w

    rebuild()
    e, f, w = force()

    def step(f):
        v[:] += 0.5 * dt * f * inv_m
        x[:] += dt * v
        if np.sqrt(((x - st["x_build"]) ** 2).sum(1)).max() > 0.5 * skin:
            rebuild()
        e, f, w = force()
        v[:] += 0.5 * dt * f * inv_m
        temp = (m[:, None] * v * v).sum() / ACC / (3.0 * n * KB)
        v[:] *= np.sqrt(1.0 + dt / tau * (T0 / temp - 1.0))
        return f

    for _ in range(warmup):
        f = step(f)
    for k in t:
        t[k] = 0 if k in ("rebuilds", "compute_first_n") else 0.0
    t0 = time.perf_counter()
    for _ in range(steps):
        f = step(f)
    elapsed = time.perf_counter() - t0
    lib_s = t["set_topology"] + t["compute"]
    rb = max(1, t["rebuilds"])
    out = {
        "value": n * steps / elapsed, "unit": "atom-steps/s", "steps": steps, "ms_per_step": 1e3 * elapsed / steps,
        "library_value": n * steps / lib_s,
        "library_ms_per_step": 1e3 * lib_s / steps,
        "set_topology_ms": 1e3 * t["set_topology"] / rb,
        "compute_ms": 1e3 * t["compute"] / steps,
        # the first so3lr_compute after each so3lr_set_topology also puts the
        # topology's nodes in spatial order, counts its active pairs and
        # captures a new graph; the others replay it
        "compute_ms_first_after_set_topology": 1e3 * t["compute_first"] / max(1, t["compute_first_n"]),
        "compute_ms_other_calls": 1e3 * (t["compute"] - t["compute_first"]) / max(1, steps - t["compute_first_n"]),
        "rebuilds": t["rebuilds"],
        "lammps_stand_in_lists_ms_per_rebuild": 1e3 * t["lammps_lists"] / rb,
        "forward_comm_ms_per_step": 1e3 * t["forward_comm"] / steps,
        "note": "value: whole loop on host arrays including the LAMMPS stand-in's list builds and ghost-row "
                "positions (LAMMPS's own work); library_value: so3lr_set_topology + so3lr_compute only",
    }
    ctx.close()
    return out


def tiled(z, x, box, tile):
    """The periodic cell repeated tile = (a, b, c) times along its axes: a
    larger periodic system with the same local structure."""
    a, b, c = tile
    shifts = np.array([[i, j, k] for i in range(a) for j in range(b) for k in range(c)], float) * box
    xs = (x[None, :, :] + shifts[:, None, :]).reshape(-1, 3)
    return np.tile(z, len(shifts)), xs, box * np.array(tile, float)


def capacity(steps, warmup, stream, tile=(1, 1, 1)):
    """Config 4 (150,000 atoms; with `tile`, that cell repeated) NPT on the
    device path: throughput, HBM in use (hipMemGetInfo) and the library's
    bytes per atom."""
    import torch
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free0, total = torch.cuda.mem_get_info()
    z, x, box, Q, M, images, periodic, desc = load_config(4)
    if tuple(tile) != (1, 1, 1):
        z, x, box = tiled(z, x, box, tile)
        desc = "config 4 cell repeated %dx%dx%d: %d H2O, %.1f x %.1f x %.1f A, periodic" % (
            tuple(tile) + (len(z) // 3,) + tuple(box))
    md = DeviceMD(4, z, x, box, Q, M, images, periodic, stream)
    elapsed, builds, _ = md.run(warmup, steps)
    free1, _ = torch.cuda.mem_get_info()
    n = md.n
    dev_bytes = md.ctx.device_bytes()
    used = total - free1
    used_by_run = free0 - free1
    out = {"workload": ("config 4: " if tuple(tile) == (1, 1, 1) else "") + desc, "atoms": n, "steps": steps,
           "ms_per_step": 1e3 * elapsed / steps, "atom_steps_per_s": n * steps / elapsed,
           "hbm_used_bytes": int(used), "hbm_used_by_this_run_bytes": int(used_by_run),
           "hbm_total_bytes": int(total), "device_bytes": int(dev_bytes),
           "device_bytes_per_atom": dev_bytes / n,
           "max_atoms_estimate": int((total - (used - used_by_run)) / (used_by_run / n)),
           "note": "max_atoms_estimate: HBM not in use before this run / (HBM this run took per atom); "
                   "water at 1 g/cm^3, linear in the candidate pair count"}
    out.update(md.ensemble())
    md.ctx.close()
    del md
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def model_widths(path):
    """The model's file name and widths, and which kernels evaluate it (the
    fused ones at the v1 widths, the generic ones otherwise)."""
    from so3lrxlammps_amd.model_file import read_model
    manifest, arrays = read_model(path)
    a = manifest["architecture"]
    rep = [int(v) for v in arrays["model.euclidean_transformers.0.euclidean_attention_block.degree_repeats"]]
    degrees = [(r - 1) // 2 for r in rep]
    head = int(arrays["model.atomic_energy_output_block.layers.0.weight"].shape[0])
    F, R = int(a["invariant_features"]), int(a["radial_basis_features"])
    v1 = F == 128 and R == 32 and degrees == [1, 2, 3, 4] and head == 128
    return {"file": os.path.basename(path), "invariant_features": F, "radial_basis_features": R,
            "degree_slots": degrees, "head_width": head, "blocks": int(a["interaction_blocks"]),
            "kernels": "fused v1" if v1 else "generic"}


def main():
    global MODEL
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-rows-path", action="store_true")
    ap.add_argument("--rows-steps", type=int, default=0, help="rows-path steps (default: --steps)")
    ap.add_argument("--no-capacity", action="store_true")
    ap.add_argument("--capacity-steps", type=int, default=5)
    ap.add_argument("--capacity-tiles", default="1x1x1",
                    help="comma-separated repeats of the config-4 cell for the capacity block, e.g. "
                         "1x1x1,1x2x2,2x2x2 (a memory-vs-size curve; the first is the reported block)")
    ap.add_argument("--roofline-steps", type=int, default=10,
                    help="steps after the timed ones with per-kernel HIP events")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain device copy of this size first (HBM-counter calibration)")
    ap.add_argument("--model", default=MODEL,
                    help="model file (default: the shipped v1 model; models of other widths run on the "
                         "generic kernels, whose roofline is that of their filter GEMM sections, and are "
                         "reported without a baseline ratio)")
    args = ap.parse_args()
    default_model = os.path.abspath(args.model) == os.path.abspath(MODEL)
    MODEL = args.model
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs one LAMMPS rank on one MI355X with no "
              "GPU-to-GPU exchange (--gpus %d is not supported)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch

    log("generating config %d" % args.config)
    z, x, box, Q, M, images, periodic, desc = load_config(args.config)
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

    md = DeviceMD(args.config, z, x, box, Q, M, images, periodic, stream)
    log("warmup %d steps, timing %d steps" % (args.warmup, args.steps))
    elapsed, builds_timed, build_s_timed = md.run(args.warmup, args.steps)
    value = n * args.steps / elapsed

    # kernel durations for the roofline: HIP events on the launch stream over
    # further steps of the same run (events keep the evaluation out of graph
    # replay, so they are not recorded during the timed steps above)
    md.ctx.kernel_timing(True)
    for _ in range(args.roofline_steps):
        md.step()
    torch.cuda.synchronize()
    md.ctx.kernel_timing(False)
    timing = {}
    work = kernel_work(model_widths(MODEL), elements=len(set(int(v) for v in z)))
    for name in ("filter_fwd", "filter_fwd_radial", "filter_fwd_block0", "filter_fwd_block0_tables",
                 "filter_fwd_block0_radial", "filter_bwd", "filter_bwd_radial", "filter_bwd_block0",
                 "filter_bwd_block0_tables", "filter_bwd_block0_radial",
                 "attn_fwd", "attn_bwd",
                 "attn_bwd_block0", "long_range", "generic_filter_fwd", "generic_filter_bwd",
                 "generic_attn_bwd_pairs", "generic_filter_fwd_block0_tables", "generic_filter_bwd_block0_tables",
                 "generic_filter_fwd_block0_radial", "generic_filter_bwd_block0_radial", "generic_filter_fwd_radial",
                 "generic_filter_bwd_radial"):
        try:
            timing[name] = md.ctx.kernel_timing_read(name)
        except Exception:  # kernel not launched
            pass
    steps_timed = max(1, args.roofline_steps)
    kernels = {}
    for k, (ms, launches, units) in timing.items():
        row = {"avg_ms": ms / launches, "launches": launches, "ms_per_step": ms / steps_timed}
        if k in work:
            sym, bound, alg, issued, unit = work[k]
            per_launch = units / launches
            rate = alg * per_launch / (ms / launches * 1e-3)  # flop/s or B/s
            if bound == "hbm":
                row.update({"kernel": sym, "units_per_launch": per_launch, "gbs_algorithmic": rate / 1e9,
                            "frac": rate / 1e9 / HBM_PEAK_GBS})
            else:
                row.update({"kernel": sym, "units_per_launch": per_launch, "tflops_algorithmic": rate / 1e12,
                            "frac": rate / 1e12 / FP64_PEAK_TFS})
        kernels[k] = row
    # the roofline kernel: most GPU time per step among those with a work model
    roofline = None
    timed_with_model = [k for k in kernels if k in work]
    if timed_with_model:
        dom = max(timed_with_model, key=lambda k: kernels[k]["ms_per_step"])
        sym, bound, alg, issued, unit = work[dom]
        ms, launches, units = timing[dom]
        avg_ms = ms / launches
        per_launch = units / launches
        hbm = bound == "hbm"
        scale, peak = (1e9, HBM_PEAK_GBS) if hbm else (1e12, FP64_PEAK_TFS)
        achieved = alg * per_launch / (avg_ms * 1e-3) / scale
        traffic, traffic_src = traffic_per_launch(sym, args.config, per_launch)
        roofline = {"bound": bound, "kernel": sym, "achieved": achieved, "peak": peak,
                    "unit": "GB/s" if hbm else "TFLOP/s",
                    "frac": achieved / peak, "traffic": traffic, "traffic_source": traffic_src,
                    "avg_launch_ms": avg_ms, "pairs_per_launch": per_launch,
                    ("bytes_per_pair_algorithmic" if hbm else "flop_per_pair_algorithmic"): alg,
                    ("bytes_per_pair_issued" if hbm else "flop_per_pair_issued"): issued,
                    "achieved_issued": issued * per_launch / (avg_ms * 1e-3) / scale,
                    "selection": "the timed kernel with the most GPU time per step (%.3f ms of %d steps' HIP events)"
                                 % (kernels[dom]["ms_per_step"], steps_timed)}
    free_b, total_b = torch.cuda.mem_get_info(dev)
    sr_active, sr_cand, lr_cand = md.ctx.graph_stats()
    config = {"workload": "config %d: %s" % (args.config, desc), "atoms": n, "integrator": "velocity Verlet",
              **md.ensemble(), "timestep_fs": 0.5, "skin_A": md.skin, "sr_pairs_active": sr_active,
              "sr_pair_candidates": sr_cand, "lr_pair_candidates": lr_cand,
              "neighbor_rebuilds_timed": builds_timed, "rebuild_seconds_timed": build_s_timed,
              "ns_per_day": value / n * 0.5 * 86400 / 1e6, "device_bytes": md.ctx.device_bytes(),
              "device_bytes_per_atom": md.ctx.device_bytes() / n,
              "hbm_used_bytes": int(total_b - free_b), "hbm_total_bytes": int(total_b), "kernels": kernels}
    md.ctx.close()
    del md
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    rows = None
    if not args.no_rows_path and args.config in (1, 3) and Q is not None:
        log("rows path (LAMMPS pair-style route, host arrays)")
        rows = rows_path(z, x, box, Q, M, periodic, args.rows_steps or args.steps, max(2, args.warmup // 2))
        rows["fraction_of_device_path"] = rows["value"] / value
        rows["library_fraction_of_device_path"] = rows["library_value"] / value
    cap = None
    if not args.no_capacity and args.config != 4:
        tiles = [tuple(int(v) for v in t.split("x")) for t in args.capacity_tiles.split(",")]
        curve = []
        for tile in tiles:
            log("capacity: config 4 cell x %s" % "x".join(map(str, tile)))
            curve.append(capacity(args.capacity_steps, 2, stream, tile))
        cap = curve[0]
        if len(curve) > 1:
            cap["curve"] = [{k: c[k] for k in ("workload", "atoms", "ms_per_step", "atom_steps_per_s",
                                               "hbm_used_bytes", "hbm_used_by_this_run_bytes", "device_bytes",
                                               "device_bytes_per_atom")} for c in curve]

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(z, x, box, periodic, images, args.cpu_budget)

    out = {
        "metric": "atom-steps/s/GPU (fp64 E+F+virial) at 24k-atom water; max atoms per GPU",
        "value": value, "unit": "atom-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": value / A100_ATOM_STEPS if args.config == 3 and default_model else None, "dtype": "f64",
        "data": "synthetic (seeded, config %d)" % args.config,
        "config": config,
        "roofline": roofline,
        "rows_path": rows,
        "capacity": cap,
        "cpu_baseline": cpu,
        "model": model_widths(MODEL),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
