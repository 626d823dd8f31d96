"""The benchmark configurations on the GPU, against the CPU oracle.

Every configuration is checked directly against the oracle at its full size
(energy 1e-10 relative, forces 1e-9 eV/A, virial 1e-9 eV absolute), the
oracle's graphs built from the LAMMPS stand-in's lists.  Config 4 (150,000 atoms) is also
checked through size-independent properties: translation invariance, zero net
force of a periodic cell, bitwise determinism, and agreement of a cluster cut
from it with the oracle.
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def orc():
    return Oracle(support.MODEL)


def _device_eval(ctx, x, lo, hi, per, eatom=False):
    """HBM-resident path: device reneighbor + one evaluation."""
    import torch
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        xt = torch.tensor(x, dtype=torch.float64, device=dev)
        ft = torch.zeros_like(xt)
        ea = torch.zeros(len(x), dtype=torch.float64, device=dev) if eatom else None
        ctx.reneighbor_device(xt, lo, hi, per, 1.0, stream=stream.cuda_stream)
        e, w = ctx.compute_device(xt, ft, ea, stream=stream.cuda_stream)
        stream.synchronize()
        out = (e, ft.cpu().numpy(), w, ea.cpu().numpy() if eatom else None)
    return out


def _check(e, f, w, out):
    # the achieved margins, printed so the logs show them against the bars
    support.record_margin(e, f, w, out)
    print("  |dE|/|E| %.2e  max|dF| %.2e eV/A  max|dW| %.2e eV (max|W| %.2e)" % (
        abs(e - out["energy"]) / abs(out["energy"]), np.abs(f - out["forces"]).max(),
        np.abs(w - out["virial"]).max(), np.abs(out["virial"]).max()), flush=True)
    assert abs(e - out["energy"]) <= 1e-10 * abs(out["energy"]), (e, out["energy"])
    assert np.abs(f - out["forces"]).max() <= 1e-9
    assert np.abs(w - out["virial"]).max() <= 1e-9  # eV, absolute, at every size


def test_config0_molecule(orc):
    from so3lrxlammps_amd import Context, Lists, systems
    z, x, box, q, m, desc = systems.config(0)
    print("config 0:", desc, flush=True)
    sr, lr = support.build_graphs(x, None)
    out = orc.evaluate(z, sr, lr, charge=q, multiplicity=m)
    c = Context(support.MODEL, 0)
    c.set_system(z, q, m)
    lo, hi = np.zeros(3), np.full(3, 40.0)
    lists = Lists(x, lo, hi, (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(x))
    _check(e, f, w, out)
    e2, f2, w2, _ = _device_eval(c, x, lo, hi, (0, 0, 0))
    _check(e2, f2, w2, out)


def test_config1_water(orc):
    from so3lrxlammps_amd import Context, Lists, systems
    z, x, box, q, m, desc = systems.config(1)
    print("config 1:", desc, flush=True)
    lists = Lists(x, np.zeros(3), box, (1, 1, 1))
    sr, lr = support.graphs_from_lists(lists, x)
    out = orc.evaluate(z, sr, lr)
    c = Context(support.MODEL, 0)
    c.set_system(z, q, m)
    e, f, w, ea = _device_eval(c, x, np.zeros(3), box, (1, 1, 1), eatom=True)
    _check(e, f, w, out)
    assert np.abs(ea - out["eatom"]).max() <= 1e-10


def test_config2_packed_molecules(orc):
    """All 512 config-2 molecules (charged, open-shell) as packed images,
    through the LAMMPS rows path and the device path."""
    from so3lrxlammps_amd import Context, Lists, systems
    z, x, offs, qs, ms, extent = systems.packed_molecules()
    print("config 2: %d atoms in %d images" % (len(z), len(qs)), flush=True)
    img = np.repeat(np.arange(len(qs)), np.diff(offs))
    sr, lr = support.build_graphs(x, None)
    out = orc.evaluate(z, sr, lr, image=img, image_charge=qs, image_multiplicity=ms)
    c = Context(support.MODEL, 0)
    c.set_images(z, offs, qs, ms)
    lo, hi = np.zeros(3), np.full(3, extent)
    lists = Lists(x, lo, hi, (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(x))
    _check(e, f, w, out)
    t = c.terms()
    assert np.abs(t["image_energy"] - out["image_energy"]).max() <= 1e-10 * np.abs(out["image_energy"]).max()
    for k in range(len(qs)):
        assert abs(t["charges"][offs[k]:offs[k + 1]].sum() - qs[k]) < 1e-12
    e2, f2, w2, _ = _device_eval(c, x, lo, hi, (0, 0, 0))
    _check(e2, f2, w2, out)
    t2 = c.terms()
    assert np.abs(t2["image_energy"] - t["image_energy"]).max() <= 1e-11 * np.abs(t["image_energy"]).max()


def test_config2_images_perturbed_weights(tmp_path):
    """64 config-2 molecules as packed images on a second set of weights
    (every parameter tensor scaled elementwise by 1 +- 20 %, seeded): the
    per-image charge correction and (Q, M) embedding with other values."""
    from so3lrxlammps_amd import Context, Lists, systems
    path = support.perturbed_model(tmp_path / "perturbed.so3lr")
    z, x, offs, qs, ms, extent = systems.packed_molecules(n_mol=64)
    print("config 2, perturbed weights: %d atoms in %d images" % (len(z), len(qs)), flush=True)
    img = np.repeat(np.arange(len(qs)), np.diff(offs))
    sr, lr = support.build_graphs(x, None)
    out = Oracle(path).evaluate(z, sr, lr, image=img, image_charge=qs, image_multiplicity=ms)
    c = Context(path, 0)
    c.set_images(z, offs, qs, ms)
    lists = Lists(x, np.zeros(3), np.full(3, extent), (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(x))
    _check(e, f, w, out)
    t = c.terms()
    assert np.abs(t["image_energy"] - out["image_energy"]).max() <= 1e-10 * np.abs(out["image_energy"]).max()
    for k in range(len(qs)):
        assert abs(t["charges"][offs[k]:offs[k + 1]].sum() - qs[k]) < 1e-12


def test_config3_full_size(orc):
    """The headline system, all 24,000 atoms, device path against the oracle."""
    from so3lrxlammps_amd import Context, Lists, systems
    z, x, box, q, m, desc = systems.config(3)
    print("config 3:", desc, flush=True)
    lists = Lists(x, np.zeros(3), box, (1, 1, 1))
    sr, lr = support.graphs_from_lists(lists, x)
    del lists
    out = orc.evaluate(z, sr, lr)
    c = Context(support.MODEL, 0)
    c.set_system(z, q, m)
    e, f, w, ea = _device_eval(c, x, np.zeros(3), box, (1, 1, 1), eatom=True)
    _check(e, f, w, out)
    assert np.abs(ea - out["eatom"]).max() <= 1e-10
    t = c.terms()
    assert np.abs(t["charges"] - out["charges"]).max() <= 1e-12
    assert abs(t["charges"].sum()) < 1e-9


def test_config4_memory_ceiling_properties(orc):
    """150,000 atoms: translation invariance, zero net force, bitwise
    determinism, and a cluster of its molecules against the oracle."""
    from so3lrxlammps_amd import Context, Lists, systems
    z, x, box, q, m, desc = systems.config(4)
    print("config 4:", desc, flush=True)
    c = Context(support.MODEL, 0)
    c.set_system(z, q, m)
    e1, f1, w1, _ = _device_eval(c, x, np.zeros(3), box, (1, 1, 1))
    e2, f2, w2, _ = _device_eval(c, x, np.zeros(3), box, (1, 1, 1))
    assert e1 == e2 and np.array_equal(f1, f2) and np.array_equal(w1, w2)
    assert np.all(np.isfinite(f1))
    # a periodic cell has no net force (pair terms cancel up to rounding)
    assert np.abs(f1.sum(0)).max() <= 1e-8 * np.sqrt(len(z))
    shift = np.array([0.37, -1.21, 2.93])
    e3, f3, w3, _ = _device_eval(c, np.mod(x + shift, box), np.zeros(3), box, (1, 1, 1))
    assert abs(e3 - e1) <= 1e-10 * abs(e1)
    assert np.abs(f3 - f1).max() <= 1e-9
    assert np.abs(w3 - w1).max() <= 1e-9 * np.abs(w1).max()
    print("config 4 device bytes:", c.device_bytes(), flush=True)
    # whole molecules of the same water inside a 30 A cube away from the cell
    # faces, as an open cluster, against the oracle
    o = x[0::3]
    keep = np.all((o >= 10.0) & (o < 40.0), axis=1)
    idx = (3 * np.nonzero(keep)[0][:, None] + np.arange(3)[None, :]).ravel()
    zs, xs = z[idx], x[idx]
    assert np.all(xs > 5.0) and np.all(xs < 45.0)  # no molecule split by the periodic wrap
    cs = Context(support.MODEL, 0)
    cs.set_system(zs, 0.0, 1.0)
    lo, hi = np.zeros(3), np.full(3, 50.0)
    sr, lr = support.build_graphs(xs, None)
    out = orc.evaluate(zs, sr, lr, charge=0.0, multiplicity=1.0)
    e4, f4, w4, _ = _device_eval(cs, xs, lo, hi, (0, 0, 0))
    _check(e4, f4, w4, out)


def test_config4_full_size(orc):
    """The 150,000-atom memory-ceiling water, all atoms, device path against
    the oracle (about 60 GB of host memory for the oracle's per-edge
    buffers and a few tens of seconds on the GPU box's cores)."""
    import resource
    import time
    from so3lrxlammps_amd import Context, Lists, systems
    z, x, box, q, m, desc = systems.config(4)
    t0 = time.time()
    lists = Lists(x, np.zeros(3), box, (1, 1, 1))
    sr, lr = support.graphs_from_lists(lists, x)
    del lists
    out = orc.evaluate(z, sr, lr)
    del sr, lr
    print("config 4 oracle: %.0f s, peak host memory %.1f GB" %
          (time.time() - t0, resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1e6), flush=True)
    c = Context(support.MODEL, 0)
    c.set_system(z, q, m)
    e, f, w, ea = _device_eval(c, x, np.zeros(3), box, (1, 1, 1), eatom=True)
    _check(e, f, w, out)
    assert np.abs(ea - out["eatom"]).max() <= 1e-10


def test_device_reneighbor_refuses_lists_past_int_range():
    """The device reneighbor counts each atom's candidates, scans the counts
    into int offsets and carries the total in 64 bits; past 2^31 - 2 entries
    (short and long range together) it refuses before any int offset is
    read.  40,000 hydrogen atoms in an 8 A cube: every pair is a long-range
    candidate (1.6e9 entries, both directions) and most are short-range ones,
    together above 2^31."""
    import torch
    from so3lrxlammps_amd import Context, _lib
    n = 40000
    rng = np.random.default_rng(7)
    x = rng.uniform(0.0, 8.0, (n, 3))
    c = Context(support.MODEL, 0)
    c.set_system(np.ones(n, dtype=np.int64), 0, 1)
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    print("capacity: %d atoms in an 8 A cube, expect a refusal" % n, flush=True)
    with torch.cuda.stream(stream):
        xt = torch.tensor(x, dtype=torch.float64, device=dev)
        with pytest.raises(_lib.SO3LRError) as err:
            c.reneighbor_device(xt, np.full(3, -10.0), np.full(3, 20.0), (0, 0, 0), 1.0, stream=stream.cuda_stream)
        stream.synchronize()
    print("  refused:", err.value, flush=True)
    assert err.value.code == _lib.ERR_TOPOLOGY and "the limit is 2147483646" in str(err.value)
    c.close()
