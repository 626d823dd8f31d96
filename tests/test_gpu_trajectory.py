"""Trajectory-level parity: NVE molecular dynamics driven by the HIP path
against the same integrator driven by the CPU oracle's forces.

Velocity Verlet in metal units (dt = 0.5 fs), the same numpy arithmetic on
both sides, so any difference comes from the forces alone and grows with the
dynamics.  Two runs:

* the eleven images of the reference's turbo validation
  (VALIDATION.md:59-75: alanine twice and its cation doublet, a water
  molecule, ethanol, a cyclic water trimer, acetate, methylammonium, the
  methyl radical, triplet O2 and H2O+), each with its own (Q, M), packed into
  one evaluation on the LAMMPS rows path for 400 steps, against the oracle
  one image at a time: positions within 1e-9 A and total energy within
  1e-9 eV per image;
* config 1 (3,000 atoms of periodic water) for 100 steps on the HBM-resident
  path (device reneighbor when an atom has moved half the 1 A skin, graph
  replay of the evaluation in between), against the oracle on the stand-in's
  lists: positions within 1e-8 A and potential and total energy within
  1e-10 relative at steps 0, 50 and 100.

The achieved differences are printed and land in the run's parity-margin
summary.
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu

DT = 0.0005          # ps
ACC = 9648.533212    # eV / (A amu) -> A / ps^2
SKIN = 1.0

# (name, charge, multiplicity): the golden molecules, geometry from their data files
IMAGES = [("alanine", 0, 1), ("alanine", 0, 1), ("alanine_cation", 1, 2), ("water_molecule", 0, 1),
          ("ethanol", 0, 1), ("water_trimer", 0, 1), ("acetate", -1, 1), ("methylammonium", 1, 1),
          ("methyl", 0, 2), ("o2", 0, 3), ("h2o_cation", 1, 2)]


def _image(name):
    try:
        ref, z, pos, _ = support.load_golden(name)
    except FileNotFoundError:
        z, pos = support.read_molecule(name)
    return np.asarray(z, dtype=np.int64), np.asarray(pos, dtype=np.float64)


def _kinetic(v, m):
    return 0.5 * (m[:, None] * v * v).sum() / ACC


def test_eleven_images_400_nve_steps():
    from so3lrxlammps_amd import Context, Lists, systems
    orc = Oracle(support.MODEL)
    zs, xs, vs, ms_ = [], [], [], []
    for k, (name, q, mult) in enumerate(IMAGES):
        z, x = _image(name)
        v, m = systems.maxwell_boltzmann(z, 300.0, seed=systems.SEED + 17 * k)
        # images 40 A apart along x: no pair across images within reach
        zs.append(z), xs.append(x - x.mean(0) + np.array([40.0 * k, 0.0, 0.0])), vs.append(v), ms_.append(m)
    offs = np.concatenate([[0], np.cumsum([len(z) for z in zs])])
    qs = np.array([q for _, q, _ in IMAGES], float)
    mm = np.array([mult for _, _, mult in IMAGES], float)
    z_all = np.concatenate(zs)
    inv_m = [(ACC / m)[:, None] for m in ms_]

    # --- the HIP path: one packed evaluation of all eleven images per step
    ctx = Context(support.MODEL, 0)
    ctx.set_images(z_all, offs, qs, mm)
    xg = [x.copy() for x in xs]
    vg = [v.copy() for v in vs]
    state = {}

    def gpu_forces():
        x = np.concatenate(xg)
        if "lists" not in state or np.sqrt(((x - state["x_build"]) ** 2).sum(1)).max() > 0.5 * SKIN:
            state["lists"] = Lists(x, x.min(0) - 20.0, x.max(0) + 20.0, (0, 0, 0))
            ctx.set_topology(state["lists"])
            state["x_build"] = x.copy()
            state["builds"] = state.get("builds", 0) + 1
        e, f, ea, w = ctx.compute(state["lists"].rows_positions(x))
        img_e = ctx.terms()["image_energy"].copy()
        return [f[offs[k]:offs[k + 1]] for k in range(len(IMAGES))], img_e

    # --- the oracle: each image on its own
    def oracle_forces(xo):
        fs, es = [], []
        for k, (_, q, mult) in enumerate(IMAGES):
            out = orc.evaluate(zs[k], *support.build_graphs(xo[k], None), charge=q, multiplicity=mult)
            fs.append(out["forces"])
            es.append(out["energy"])
        return fs, np.array(es)

    xo = [x.copy() for x in xs]
    vo = [v.copy() for v in vs]
    fg, eg = gpu_forces()
    fo, eo = oracle_forces(xo)
    e0 = np.array([eg[k] + _kinetic(vg[k], ms_[k]) for k in range(len(IMAGES))])
    print("eleven images: %d atoms; step 0 max|dE| %.2e eV max|dF| %.2e eV/A" % (
        offs[-1], np.abs(eg - eo).max(), max(np.abs(a - b).max() for a, b in zip(fg, fo))), flush=True)
    for step in range(1, 401):
        for k in range(len(IMAGES)):
            vg[k] += 0.5 * DT * fg[k] * inv_m[k]
            xg[k] += DT * vg[k]
            vo[k] += 0.5 * DT * fo[k] * inv_m[k]
            xo[k] += DT * vo[k]
        fg, eg = gpu_forces()
        fo, eo = oracle_forces(xo)
        for k in range(len(IMAGES)):
            vg[k] += 0.5 * DT * fg[k] * inv_m[k]
            vo[k] += 0.5 * DT * fo[k] * inv_m[k]
        if step % 100 == 0:
            dx = max(np.abs(a - b).max() for a, b in zip(xg, xo))
            print("  step %d: max|dx| %.2e A, max|dE_pot| %.2e eV, list builds %d" % (
                step, dx, np.abs(eg - eo).max(), state["builds"]), flush=True)
    etot_g = np.array([eg[k] + _kinetic(vg[k], ms_[k]) for k in range(len(IMAGES))])
    etot_o = np.array([eo[k] + _kinetic(vo[k], ms_[k]) for k in range(len(IMAGES))])
    for k, (name, q, mult) in enumerate(IMAGES):
        dx = np.abs(xg[k] - xo[k]).max()
        de = abs(etot_g[k] - etot_o[k])
        print("  image %2d %-15s (Q %+d, M %d): max|dx| %.2e A  |dE_tot| %.2e eV  NVE drift %.2e eV" % (
            k, name, q, mult, dx, de, etot_g[k] - e0[k]), flush=True)
        support.TRAJECTORY.append(("400 steps, image %d %s" % (k, name), dx, de, "eV |dE_tot|"))
        assert dx <= 1e-9, (name, dx)
        assert de <= 1e-9, (name, de)
        # energy is conserved by the dynamics itself (a check of the forces'
        # consistency with the energy, not of parity)
        assert abs(etot_g[k] - e0[k]) <= 5e-3 * max(1, len(zs[k]) / 10), (name, etot_g[k] - e0[k])
    assert state["builds"] >= 1
    ctx.close()


def _wrap(x, box):
    return np.mod(x, box)


def _min_image(d, box):
    return d - np.round(d / box) * box


def test_config1_100_nve_steps_device_path():
    import torch
    from so3lrxlammps_amd import Context, Lists, systems
    z, x0, box, q, mult, desc = systems.config(1)
    box = np.asarray(box, float)
    lo, hi, per = np.zeros(3), box, (1, 1, 1)
    v0, m = systems.maxwell_boltzmann(z, 300.0)
    inv_m = (ACC / m)[:, None]
    orc = Oracle(support.MODEL)
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    ctx = Context(support.MODEL, 0)
    ctx.set_system(z, q, mult)

    # --- the HIP path: positions and forces in persistent device tensors
    # (the same pointers every step, so the evaluation is captured once and
    # replayed), integration in numpy on the host
    xg, vg = x0.copy(), v0.copy()
    st = {"builds": 0}
    with torch.cuda.stream(stream):
        xt = torch.tensor(xg, dtype=torch.float64, device=dev)
        ft = torch.zeros_like(xt)

    def gpu_forces():
        with torch.cuda.stream(stream):
            xt.copy_(torch.from_numpy(xg))
            if "x_build" not in st or np.sqrt(((xg - st["x_build"]) ** 2).sum(1)).max() > 0.5 * SKIN:
                ctx.reneighbor_device(xt, lo, hi, per, SKIN, stream=stream.cuda_stream)
                xg[:] = xt.cpu().numpy()  # wrapped into the box in place
                st["x_build"] = xg.copy()
                st["builds"] += 1
            e, w = ctx.compute_device(xt, ft, stream=stream.cuda_stream)
            stream.synchronize()
            return e, ft.cpu().numpy()

    # --- the oracle on the stand-in's lists at its own positions
    xo, vo = x0.copy(), v0.copy()

    def oracle_forces():
        xw = _wrap(xo, box)
        lists = Lists(xw, lo, hi, per)
        out = orc.evaluate(z, *support.graphs_from_lists(lists, xw))
        return out["energy"], out["forces"]

    def compare(step, eg, eo):
        dx = np.abs(_min_image(xg - xo, box)).max()
        kg, ko = _kinetic(vg, m), _kinetic(vo, m)
        de_pot = abs(eg - eo) / abs(eo)
        de_tot = abs((eg + kg) - (eo + ko)) / abs(eo + ko)
        print("  config 1 step %3d: max|dx| %.2e A  |dE_pot|/|E| %.2e  |dE_tot|/|E| %.2e  builds %d" % (
            step, dx, de_pot, de_tot, st["builds"]), flush=True)
        support.TRAJECTORY.append(("config 1, step %d" % step, dx, max(de_pot, de_tot), "rel |dE|"))
        assert dx <= 1e-8, (step, dx)
        assert de_pot <= 1e-10 and de_tot <= 1e-10, (step, de_pot, de_tot)
        return eg + kg

    print("config 1:", desc, "100 NVE steps", flush=True)
    eg, fg = gpu_forces()
    eo, fo = oracle_forces()
    e_start = compare(0, eg, eo)
    for step in range(1, 101):
        vg += 0.5 * DT * fg * inv_m
        xg += DT * vg
        vo += 0.5 * DT * fo * inv_m
        xo += DT * vo
        eg, fg = gpu_forces()
        eo, fo = oracle_forces()
        vg += 0.5 * DT * fg * inv_m
        vo += 0.5 * DT * fo * inv_m
        if step in (50, 100):
            e_now = compare(step, eg, eo)
    print("  NVE drift over 100 steps: %.2e eV (%.2e eV per atom)" % (e_now - e_start, (e_now - e_start) / len(z)),
          flush=True)
    # the integrator's own error from an unequilibrated lattice start (the
    # oracle-driven run drifts the same way, to the digits compared above);
    # a loose sanity bound, not a parity bar
    assert abs(e_now - e_start) <= 1e-3 * len(z)
    assert st["builds"] >= 1
    ctx.close()
