"""Timing of the so3lr/turbo path: one image per MPI rank, rank 0 on the GPU.

    mpiexec -launcher fork -n 16 python -m so3lrxlammps_amd.turbo_bench --steps 200

Rank r runs molecule r of the config-2 generator (12-40 atoms of H, C, N, O,
S, its own charge and multiplicity; systems.packed_molecules) through the
pair-style mirror with velocity Verlet at 0.25 fs, as a one-rank LAMMPS
partition would.  Rank 0 prints one JSON line: image-steps/s and atom-steps/s
over the timed steps, and per step the coordinator's time in the gathers
(which includes waiting for the slowest image), in the packed GPU evaluation
(positions up, the kernels, forces and per-atom terms down) and in the scatter.
The ranks build their lists with one OpenMP thread each (--threads), as
one-rank partitions would.
"""
import argparse
import json
import os
import time

import numpy as np

from . import systems, turbo
from .pair_style import Atoms

MASS = {1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999, 16: 32.06}
SYMBOL = {1: "H", 6: "C", 7: "N", 8: "O", 16: "S"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--model", default=None)
    ap.add_argument("--per-rank", action="store_true", help="every rank prints its own time split")
    ap.add_argument("--threads", type=int, default=1,
                    help="OpenMP threads per rank for the list builds (a one-rank partition: 1)")
    args = ap.parse_args()
    os.environ["OMP_NUM_THREADS"] = str(args.threads)  # before the list builder's OpenMP runtime loads
    comm, rank, size = turbo.mpi_world()
    model = args.model or os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "models",
                                       "so3lr.so3lr")
    z_all, x_all, offs, qs, ms, _ = systems.packed_molecules(n_mol=size)
    z = z_all[offs[rank]:offs[rank + 1]]
    x = x_all[offs[rank]:offs[rank + 1]].copy()
    x -= x.mean(0)
    elements = sorted(set(int(v) for v in z))
    types = np.array([elements.index(int(v)) + 1 for v in z])
    pair = turbo.PairSO3LRTurbo(comm, device=args.device)
    pair.settings([model, repr(float(qs[rank])), repr(float(ms[rank]))])
    pair.coeff(["*", "*"] + [SYMBOL[e] for e in elements], len(elements))
    atoms = Atoms(x=x, types=types, lo=x.min(0) - 40.0, hi=x.max(0) + 40.0, periodic=(0, 0, 0))
    pair.init_style(atoms)
    mass = np.array([MASS[int(v)] for v in z])[:, None]
    rng = np.random.default_rng(1000 + rank)
    v = rng.normal(scale=0.02, size=x.shape)  # A/ps
    dt, conv = 0.25e-3, 9648.533212
    f = pair.compute(atoms, vflag=False)["forces"]
    phases = np.zeros(4)
    t0 = 0.0
    rebuilds = 0
    for step in range(args.warmup + args.steps):
        if step == args.warmup:
            phases[:] = 0.0
            t0 = time.perf_counter()
        v += 0.5 * dt * f / mass * conv
        atoms.x = atoms.x + dt * v
        res = pair.compute(atoms, vflag=False)
        f = res["forces"]
        if step >= args.warmup:
            rebuilds += int(res["lists_changed"])
        v += 0.5 * dt * f / mass * conv
        st = pair.broker.stats()
        phases += [st["gather_ms"], st["evaluate_ms"], st["scatter_ms"], st["total_ms"]]
    wall = time.perf_counter() - t0
    if args.per_rank:
        # this rank's own split: inside the broker call, and everything else
        print("rank %d call_ms=%.3f other_ms=%.3f reneighbours=%d" % (
            rank, phases[3] / args.steps, 1e3 * wall / args.steps - phases[3] / args.steps, rebuilds), flush=True)
    if rank == 0:
        k = args.steps
        atoms_total = int(offs[-1])
        print(json.dumps({
            "metric": "turbo image-steps/s", "value": size * k / wall, "unit": "image-steps/s",
            "atom_steps_per_s": atoms_total * k / wall, "images": size, "atoms": atoms_total, "steps": k,
            "ms_per_step": 1e3 * wall / k, "gather_ms": phases[0] / k, "evaluate_ms": phases[1] / k,
            "scatter_ms": phases[2] / k, "call_ms": phases[3] / k, "rank0_reneighbours": rebuilds,
            "dtype": "f64", "data": "synthetic",
            "config": {"workload": "config-2 molecules, one per MPI rank (so3lr/turbo)"}}), flush=True)
    pair.broker.close()
    turbo.mpi_finalize()


if __name__ == "__main__":
    main()
