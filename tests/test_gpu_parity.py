"""HIP path vs the CPU oracle, through the C ABI (libso3lr_hip.so).

Tolerances are the ones BASELINE.json states for this path: energies within
1e-10 relative, forces within 1e-9 eV/A and the virial within 1e-9 eV
(absolute: the oracle sums its totals with compensation, so its own rounding
stays far below that at every size).  The oracle's graph is built by
brute force with the minimum-image convention (tests/support.py), the HIP
path's by the LAMMPS stand-in (ghost rows, full SR + half LR lists with a
1 A skin), so the neighbour handling is checked too.
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu

MOLECULES = ["o2", "h2o_cation", "methyl", "methylammonium", "acetate", "alanine_cation", "alanine"]


@pytest.fixture(scope="module")
def orc():
    return Oracle(support.MODEL)


@pytest.fixture(scope="module")
def ctx():
    from so3lrxlammps_amd import Context
    return Context(support.MODEL, 0)


def _hip_single_point(ctx, z, pos, box, charge, mult):
    from so3lrxlammps_amd import Lists
    ctx.set_system(z, charge, mult)
    if box is None:
        lo, hi, per = pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0)
    else:
        lo, hi, per = np.zeros(3), box, (1, 1, 1)
    lists = Lists(pos, lo, hi, per)
    ctx.set_topology(lists)
    e, f, ea, w = ctx.compute(lists.rows_positions(pos))
    return e, f, ea, w, ctx.terms()


def _check(out, e, f, ea, w, terms, ftol=1e-9):
    # the achieved margins, printed so the logs show them against the bars
    support.record_margin(e, f, w, out)
    print("  |dE|/|E| %.2e  max|dF| %.2e eV/A  max|dW| %.2e eV (max|W| %.2e)" % (
        abs(e - out["energy"]) / abs(out["energy"]), np.abs(f - out["forces"]).max(),
        np.abs(w - out["virial"]).max(), np.abs(out["virial"]).max()), flush=True)
    assert abs(e - out["energy"]) <= 1e-10 * abs(out["energy"]), (e, out["energy"])
    assert np.abs(f - out["forces"]).max() <= ftol
    assert np.abs(w - out["virial"]).max() <= 1e-9  # eV, absolute
    assert np.abs(ea - out["eatom"]).max() <= 1e-10 * max(1.0, np.abs(out["eatom"]).max())
    assert np.abs(terms["charges"] - out["charges"]).max() <= 1e-12
    assert np.abs(terms["hirshfeld"] - out["hirshfeld"]).max() <= 1e-12
    assert np.abs(terms["learned"] - out["e_learned"]).max() <= 1e-9
    assert np.abs(terms["zbl"] - out["e_zbl"]).max() <= 1e-11
    assert np.abs(terms["long_range"] - out["e_lr"]).max() <= 1e-11


@pytest.mark.parametrize("name", MOLECULES)
def test_molecule_matches_oracle(ctx, orc, name):
    ref, z, pos, box = support.load_golden(name)
    q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
    print("case", name, flush=True)
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, q, m)
    sr, lr = support.build_graphs(pos, box)
    out = orc.evaluate(z, sr, lr, charge=q, multiplicity=m)
    _check(out, e, f, ea, w, terms)


def test_molecules_mfma_filters_match_oracle(orc, monkeypatch):
    """Molecules this small run the scalar filter kernels by default (at most
    SO3LR_SCALAR_FILTER_PAIRS active pairs); the same molecules with the fused
    MFMA filters forced, against the oracle at the same bars."""
    from so3lrxlammps_amd import Context
    monkeypatch.setenv("SO3LR_SCALAR_FILTER_PAIRS", "0")
    c = Context(support.MODEL, 0)
    for name in MOLECULES:
        ref, z, pos, box = support.load_golden(name)
        q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
        print("case", name, "(MFMA filters)", flush=True)
        e, f, ea, w, terms = _hip_single_point(c, z, pos, box, q, m)
        out = orc.evaluate(z, *support.build_graphs(pos, box), charge=q, multiplicity=m)
        _check(out, e, f, ea, w, terms)
    c.close()


def test_small_system_filter_paths_agree(monkeypatch):
    """The filter path switches with the active-pair count; both paths on the
    same molecule agree to rounding (the scalar kernels use the library exp
    and division, the MFMA ones the lean activations)."""
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden("alanine_cation")
    res = []
    for limit in ("0", "1000000"):
        monkeypatch.setenv("SO3LR_SCALAR_FILTER_PAIRS", limit)
        c = Context(support.MODEL, 0)
        res.append(_hip_single_point(c, z, pos, box, 1, 2))
        c.close()
    (e0, f0, _, w0, _), (e1, f1, _, w1, _) = res
    assert abs(e1 - e0) <= 1e-12 * abs(e0)
    assert np.abs(f1 - f0).max() <= 1e-10
    assert np.abs(w1 - w0).max() <= 1e-10 * max(1.0, np.abs(w0).max())


def test_molecule_matches_golden_reference(ctx):
    """The HIP path against the reference's JAX vectors directly (float64 refs)."""
    for name in ["acetate", "alanine_cation", "methylammonium"]:
        ref, z, pos, box = support.load_golden(name)
        e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, ref["charge"], ref["multiplicity"])
        assert np.abs(f - np.asarray(ref["forces"])).max() <= 3e-10
        assert abs(e - ref["energy_native_convention"]) <= 1e-11 * abs(ref["energy_native_convention"])


def test_water3000_periodic(ctx, orc):
    ref, z, pos, box = support.load_golden("water3000")
    print("case water3000", flush=True)
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, 0, 1)
    sr, lr = support.build_graphs(pos, box)
    out = orc.evaluate(z, sr, lr)
    _check(out, e, f, ea, w, terms)
    # the reference's own float32-parameter floor against JAX
    assert np.abs(f - np.asarray(ref["forces"])).max() <= 3e-6


@pytest.fixture(scope="module")
def perturbed(tmp_path_factory):
    return support.perturbed_model(tmp_path_factory.mktemp("model") / "perturbed.so3lr")


@pytest.mark.parametrize("name,q,m", [("acetate", -1, 1), ("water3000", 0, 1)])
def test_perturbed_weights_match_oracle(perturbed, name, q, m):
    """A second set of weights (every parameter tensor scaled elementwise by
    1 +- 20 %, seeded), so that parity does not rest on the shipped
    checkpoint's values alone."""
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden(name)
    print("case perturbed", name, flush=True)
    e, f, ea, w, terms = _hip_single_point(Context(perturbed, 0), z, pos, box, q, m)
    sr, lr = support.build_graphs(pos, box)
    out = Oracle(perturbed).evaluate(z, sr, lr, charge=q, multiplicity=m)
    _check(out, e, f, ea, w, terms)


def test_deterministic_bitwise(ctx):
    ref, z, pos, box = support.load_golden("alanine_cation")
    a = _hip_single_point(ctx, z, pos, box, 1, 2)
    b = _hip_single_point(ctx, z, pos, box, 1, 2)
    assert a[0] == b[0]
    assert np.array_equal(a[1], b[1])
    assert np.array_equal(a[3], b[3])


_ELEMENTS17 = [1, 6, 7, 8, 9, 11, 12, 13, 14, 15, 16, 17, 19, 20, 35, 53, 3]


def _cluster(elements, n=240, seed=5):
    """n atoms of the given elements (each at least once) at random sites of
    a sphere, no two closer than 1.8 A; multiplicity by electron parity."""
    rng = np.random.default_rng(seed)
    pts = []
    while len(pts) < n:
        p = rng.uniform(-13.0, 13.0, 3)
        if np.linalg.norm(p) < 13.0 and all(np.linalg.norm(p - q) >= 1.8 for q in pts):
            pts.append(p)
    z = np.array(list(elements) + list(rng.choice(elements, n - len(elements))), dtype=np.int64)
    return z, np.array(pts), 1 + int(z.sum()) % 2


@pytest.mark.parametrize("count", [16, 17])
def test_element_table_limit(monkeypatch, orc, count):
    """At the table path's limit: 16 elements run block 0 through the tables
    (equal to the full kernels to rounding), 17 fall back to the full kernels
    (bit for bit the SO3LR_NO_CLASS_TABLES=1 result); both against the oracle."""
    from so3lrxlammps_amd import Context, Lists
    z, pos, mult = _cluster(_ELEMENTS17[:count])
    monkeypatch.setenv("SO3LR_SCALAR_FILTER_PAIRS", "0")
    lists = Lists(pos, pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0))
    res = []
    for off in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_CLASS_TABLES", off)
        c = Context(support.MODEL, 0)
        c.set_system(z, 0, mult)
        c.set_topology(lists)
        e, f, ea, w = c.compute(lists.rows_positions(pos))
        res.append((e, f.copy(), w.copy()))
        c.close()
    (e1, f1, w1), (e2, f2, w2) = res
    print("%d elements: |dE| %.2e max|dF| %.2e" % (count, abs(e1 - e2), np.abs(f1 - f2).max()), flush=True)
    if count == 17:
        assert e1 == e2 and np.array_equal(f1, f2) and np.array_equal(w1, w2)
    else:
        assert abs(e1 - e2) <= 1e-13 * abs(e2)
        assert np.abs(f1 - f2).max() <= 1e-11
    out = orc.evaluate(z, *support.build_graphs(pos, None), charge=0, multiplicity=mult)
    assert abs(e2 - out["energy"]) <= 1e-10 * abs(out["energy"])
    assert np.abs(f2 - out["forces"]).max() <= 1e-9
    assert np.abs(w2 - out["virial"]).max() <= 1e-9


@pytest.mark.parametrize("radial_off", ["0", "1"])
def test_deterministic_bitwise_table_path(monkeypatch, radial_off):
    """Periodic water on block 0's table paths: the radial tables (built by
    the first call) and the element-pair kernels, whose element-pair sort
    places pairs with integer atomics (SO3LR_NO_RADIAL_TABLES=1).  Two
    contexts (one eager, one replaying a graph), three calls each, all bit
    for bit equal."""
    from so3lrxlammps_amd import Context, Lists
    monkeypatch.setenv("SO3LR_NO_RADIAL_TABLES", radial_off)
    ref, z, pos, box = support.load_golden("water3000")
    lists = Lists(pos, np.zeros(3), box, (1, 1, 1))
    xr = lists.rows_positions(pos)
    outs = []
    for no_graph in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_GRAPH", no_graph)
        c = Context(support.MODEL, 0)
        c.set_system(z, 0, 1)
        c.set_topology(lists)
        for _ in range(3):
            e, f, ea, w = c.compute(xr)
            outs.append((e, f.copy(), w.copy()))
        c.close()
    for e, f, w in outs[1:]:
        assert e == outs[0][0]
        assert np.array_equal(f, outs[0][1])
        assert np.array_equal(w, outs[0][2])


def test_packed_images_match_oracle(orc):
    from so3lrxlammps_amd import Context, Lists
    names = [("acetate", -1, 1), ("methyl", 0, 2), ("h2o_cation", 1, 2), ("alanine", 0, 1)]
    zs, ps, qs, ms, offs = [], [], [], [], [0]
    for k, (name, q, m) in enumerate(names):
        ref, z, pos, box = support.load_golden(name)
        zs.append(z); ps.append(pos + np.array([40.0 * k, 0, 0])); qs.append(q); ms.append(m)
        offs.append(offs[-1] + len(z))
    z = np.concatenate(zs); pos = np.concatenate(ps)
    c = Context(support.MODEL, 0)
    c.set_images(z, offs, qs, ms)
    lists = Lists(pos, pos.min(0) - 20, pos.max(0) + 20, (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(pos))
    t = c.terms()
    img = np.repeat(np.arange(len(names)), np.diff(offs))
    sr, lr = support.build_graphs(pos, None)
    out = orc.evaluate(z, sr, lr, image=img, image_charge=np.array(qs, float), image_multiplicity=ms)
    assert np.abs(f - out["forces"]).max() <= 1e-9
    assert np.abs(t["image_energy"] - out["image_energy"]).max() <= 1e-10 * np.abs(out["image_energy"]).max()
    for k in range(len(names)):
        assert abs(t["charges"][offs[k]:offs[k + 1]].sum() - qs[k]) < 1e-12


def test_refusals(ctx):
    from so3lrxlammps_amd import _lib
    ref, z, pos, box = support.load_golden("o2")
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, 0, 3)
    x = np.zeros(6)
    fbuf = np.zeros(6)
    rc = ctx.raw_compute(_lib.ptr(x), 16, _lib.ptr(fbuf), None, None, None)  # an unknown flag bit
    assert rc == _lib.ERR_ARGUMENT
    with pytest.raises(_lib.SO3LRError) as err:
        ctx.set_system(z, 0, 2)  # O2 has 16 electrons: an even count needs an odd multiplicity
    assert err.value.code == _lib.ERR_SYSTEM
    # a rank that owns no atoms, and a packed image with none, are refused
    # (src/rank_local_half_pair_graph.cpp:43)
    with pytest.raises(_lib.SO3LRError) as err:
        ctx.set_system(np.zeros(0, dtype=np.int32), 0, 1)
    assert err.value.code == _lib.ERR_ARGUMENT
    with pytest.raises(_lib.SO3LRError) as err:
        ctx.set_images(np.array([8, 8], dtype=np.int32), [0, 2, 2], [0.0, 0.0], [3.0, 1.0])
    assert err.value.code == _lib.ERR_ARGUMENT
    # offsets that overshoot the atom count and come back down: refused before
    # any of them is used as an index (host-side check, no kernel runs)
    z3 = np.array([8, 1, 1], dtype=np.int32)
    off = np.array([0, 5, 3], dtype=np.int64)
    qm = np.zeros(2)
    rc = ctx._lib.so3lr_set_images(ctx._h, 3, _lib.ptr(z3), 2, _lib.ptr(off), _lib.ptr(qm), _lib.ptr(qm + 1.0))
    assert rc == _lib.ERR_ARGUMENT, ctx._lib.so3lr_last_error(ctx._h)
    # the context stays usable after the refusals
    e2, f2, _, _, _ = _hip_single_point(ctx, z, pos, box, 0, 3)
    assert e2 == e and np.array_equal(f2, f)


def test_rows_path_atom_order(ctx):
    """The LAMMPS-list path puts its nodes in a spatial order of its own at
    the first evaluation of a topology, so the caller's atom order must not
    matter: water3000 with its atoms shuffled gives the same energy, virial,
    forces, per-atom energies, per-atom virials and per-atom terms, each in
    the shuffled order (to rounding: the node-major sums meet the pairs in
    another order)."""
    ref, z, pos, box = support.load_golden("water3000")
    p = np.random.default_rng(7).permutation(len(z))
    runs = []
    for zz, xx in ((z, pos), (z[p], pos[p])):
        e, f, ea, w, terms = _hip_single_point(ctx, zz, xx, box, 0, 1)
        runs.append((e, f, ea, w, terms, ctx.vatom()))
    (e0, f0, ea0, w0, t0, v0), (e1, f1, ea1, w1, t1, v1) = runs
    print("  |dE| %.2e  max|dF| %.2e" % (abs(e1 - e0), np.abs(f1 - f0[p]).max()), flush=True)
    assert abs(e1 - e0) <= 1e-12 * abs(e0)
    assert np.abs(w1 - w0).max() <= 1e-11 * np.abs(w0).max()
    assert np.abs(f1 - f0[p]).max() <= 1e-11
    assert np.abs(ea1 - ea0[p]).max() <= 1e-12 * np.abs(ea0).max()
    assert np.abs(v1 - v0[p]).max() <= 1e-11 * np.abs(v0).max()
    for k in ("charges", "hirshfeld", "learned", "zbl", "long_range"):
        assert np.abs(t1[k] - t0[k][p]).max() <= 1e-11 * max(1.0, np.abs(t0[k]).max()), k


def test_per_atom_virial_matches_oracle(ctx, orc):
    """so3lr_last_vatom (no counterpart in the reference) against the oracle's
    per-atom virial, at the virial's bar (1e-9 of its scale), on a dimer, a
    molecule, periodic water (rows path, and the device path into device
    memory) and packed images; the atoms' sum is the returned global virial."""
    import torch
    from so3lrxlammps_amd import Context, Lists, _lib
    for name, q, m in (("o2", 0, 3), ("acetate", -1, 1)):
        ref, z, pos, box = support.load_golden(name)
        e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, q, m)
        va = ctx.vatom()
        out = orc.evaluate(z, *support.build_graphs(pos, box), charge=q, multiplicity=m)
        scale = max(1.0, np.abs(out["vatom"]).max())
        assert np.abs(va - out["vatom"]).max() <= 1e-9 * scale, name
        assert np.abs(va.sum(0) - w).max() <= 1e-12 * max(1.0, np.abs(w).max()), name
    ref, z, pos, box = support.load_golden("water3000")
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, 0, 1)
    va = ctx.vatom()
    out = orc.evaluate(z, *support.build_graphs(pos, box))
    scale = max(1.0, np.abs(out["vatom"]).max())
    assert np.abs(va - out["vatom"]).max() <= 1e-9 * scale
    assert np.abs(va.sum(0) - w).max() <= 1e-10 * np.abs(w).max()
    # the device path: spatial node order inside, atom order out, device memory
    c = Context(support.MODEL, 0)
    c.set_system(z, 0, 1)
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        xt = torch.tensor(pos, dtype=torch.float64, device=dev)
        ft = torch.zeros_like(xt)
        vt = torch.zeros((len(z), 6), dtype=torch.float64, device=dev)
        c.reneighbor_device(xt, np.zeros(3), box, (1, 1, 1), 1.0, stream=stream.cuda_stream)
        e2, w2 = c.compute_device(xt, ft, stream=stream.cuda_stream)
        c.vatom(vt)
        stream.synchronize()
        va2 = vt.cpu().numpy()
    assert np.abs(va2 - out["vatom"]).max() <= 1e-9 * scale
    c.close()
    # packed images
    names = [("acetate", -1, 1), ("methyl", 0, 2), ("h2o_cation", 1, 2)]
    zs, ps, qs, ms, offs = [], [], [], [], [0]
    for k, (name, q, m) in enumerate(names):
        ref, zk, pk, _ = support.load_golden(name)
        zs.append(zk); ps.append(pk + np.array([40.0 * k, 0, 0])); qs.append(q); ms.append(m)
        offs.append(offs[-1] + len(zk))
    zp = np.concatenate(zs); pp = np.concatenate(ps)
    cp = Context(support.MODEL, 0)
    cp.set_images(zp, offs, qs, ms)
    lists = Lists(pp, pp.min(0) - 20, pp.max(0) + 20, (0, 0, 0))
    cp.set_topology(lists)
    # the buffers stay referenced for the whole call
    xr = np.ascontiguousarray(lists.rows_positions(pp))
    fr, er = np.zeros((len(zp), 3)), np.zeros(1)
    rc = cp.raw_compute(_lib.ptr(xr), _lib.ENERGY | _lib.VATOM, _lib.ptr(fr), None, _lib.ptr(er), None)
    assert rc == _lib.OK
    vap = cp.vatom()
    img = np.repeat(np.arange(len(names)), np.diff(offs))
    outp = orc.evaluate(zp, *support.build_graphs(pp, None), image=img, image_charge=np.array(qs, float),
                        image_multiplicity=ms)
    assert np.abs(vap - outp["vatom"]).max() <= 1e-9 * max(1.0, np.abs(outp["vatom"]).max())
    cp.close()


def test_device_reneighbor_matches_rows_path(orc):
    """HBM-resident reneighbor (owned positions + image codes) against the
    LAMMPS-rows path and the oracle, with atoms displaced outside the box."""
    import torch
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden("water3000")
    rng = np.random.default_rng(3)
    moved = pos + rng.normal(scale=0.05, size=pos.shape)
    moved[:50] += box  # some atoms one period away: the reneighbor wraps them
    c = Context(support.MODEL, 0)
    c.set_system(z, 0, 1)
    lists = Lists(np.mod(moved, box), np.zeros(3), box, (1, 1, 1))
    c.set_topology(lists)
    e1, f1, ea1, w1 = c.compute(lists.rows_positions(np.mod(moved, box)))
    t1 = c.terms()
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        xt = torch.tensor(moved, dtype=torch.float64, device=dev)
        ft = torch.zeros_like(xt)
        eat = torch.zeros(len(z), dtype=torch.float64, device=dev)
        c.reneighbor_device(xt, np.zeros(3), box, (1, 1, 1), 1.0, stream=stream.cuda_stream)
        e2, w2 = c.compute_device(xt, ft, eat, stream=stream.cuda_stream)
        stream.synchronize()
        wrapped = xt.cpu().numpy()
        f2 = ft.cpu().numpy()
        ea2 = eat.cpu().numpy()
    t2 = c.terms()
    assert np.all(wrapped >= 0) and np.all(wrapped < box)
    assert np.abs(wrapped - np.mod(moved, box)).max() < 1e-12
    assert abs(e1 - e2) <= 1e-12 * abs(e1)
    assert np.abs(f1 - f2).max() <= 1e-11
    assert np.abs(w1 - w2).max() <= 1e-10 * max(1.0, np.abs(w1).max())
    # per-atom outputs come back in the caller's atom order (the device path
    # evaluates in its own spatial node order)
    assert np.abs(ea1 - ea2).max() <= 1e-12
    for key in ("learned", "zbl", "long_range", "charges", "hirshfeld"):
        assert np.abs(t1[key] - t2[key]).max() <= 1e-12, key
    sr_active, sr_cand, lr_cand = c.graph_stats()
    assert sr_cand == len(lists.lists[0][2]) // 2 and lr_cand == len(lists.lists[1][2])
    sr, lr = support.build_graphs(np.mod(moved, box), box)
    out = orc.evaluate(z, sr, lr)
    assert abs(e2 - out["energy"]) <= 1e-10 * abs(out["energy"])
    assert np.abs(f2 - out["forces"]).max() <= 1e-9


def test_scalar_filter_path_matches_mfma(monkeypatch):
    """The scalar (one pair per workgroup) filter kernels, selected with
    SO3LR_NAIVE_FILTERS=1 at context creation, against the fp64 MFMA ones: two
    independent implementations of the filter networks and their reverse."""
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden("water3000")
    results = []
    for naive in ("1", "0"):
        monkeypatch.setenv("SO3LR_NAIVE_FILTERS", naive)
        c = Context(support.MODEL, 0)
        c.set_system(z, 0, 1)
        lists = Lists(pos, np.zeros(3), box, (1, 1, 1))
        c.set_topology(lists)
        results.append(c.compute(lists.rows_positions(pos)))
        c.close()
    (e1, f1, ea1, w1), (e2, f2, ea2, w2) = results
    assert abs(e1 - e2) <= 1e-12 * abs(e2)
    assert np.abs(f1 - f2).max() <= 1e-10
    assert np.abs(w1 - w2).max() <= 1e-10 * np.abs(w2).max()


@pytest.mark.parametrize("name,q,m", [("water3000", 0, 1), ("alanine", 0, 1), ("acetate", -1, 1)])
def test_block0_element_tables_match_full_kernels(monkeypatch, name, q, m):
    """Block 0 through element-pair tables (the default for a one-image
    system) against the full block-0 filter kernels (SO3LR_NO_CLASS_TABLES=1):
    the same algebra summed in another order, so equal to rounding.  The
    molecules take the MFMA path too (SO3LR_SCALAR_FILTER_PAIRS=0): 2, 4 and
    3 elements."""
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden(name)
    monkeypatch.setenv("SO3LR_SCALAR_FILTER_PAIRS", "0")
    if box is None:
        lo, hi, per = pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0)
    else:
        lo, hi, per = np.zeros(3), box, (1, 1, 1)
    results = []
    for off in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_CLASS_TABLES", off)
        c = Context(support.MODEL, 0)
        c.set_system(z, q, m)
        lists = Lists(pos, lo, hi, per)
        c.set_topology(lists)
        e, f, ea, w = c.compute(lists.rows_positions(pos))
        results.append((e, f.copy(), ea.copy(), w.copy(), c.vatom()))
        c.close()
    (e1, f1, ea1, w1, va1), (e2, f2, ea2, w2, va2) = results
    print("%s: |dE| %.2e max|dF| %.2e max|dW| %.2e" % (name, abs(e1 - e2), np.abs(f1 - f2).max(),
                                                       np.abs(w1 - w2).max()), flush=True)
    assert abs(e1 - e2) <= 1e-13 * abs(e2)
    assert np.abs(f1 - f2).max() <= 1e-11
    assert np.abs(w1 - w2).max() <= 1e-11 * max(1.0, np.abs(w2).max())
    assert np.abs(ea1 - ea2).max() <= 1e-12 * max(1.0, np.abs(ea2).max())
    assert np.abs(va1 - va2).max() <= 1e-11 * max(1.0, np.abs(va2).max())


def _launches(ctx, kernel):
    """Launches of a timed kernel name (0 when it never ran)."""
    from so3lrxlammps_amd import SO3LRError
    try:
        return ctx.kernel_timing_read(kernel)[1]
    except SO3LRError:
        return 0


@pytest.mark.parametrize("name,q,m", [("water3000", 0, 1), ("alanine", 0, 1), ("acetate", -1, 1)])
def test_block0_radial_tables_match_element_tables(monkeypatch, name, q, m):
    """Every block on its radial tables (the default): block 0's logits as
    piecewise polynomials of r per element pair, the later blocks' radial
    branches as fitted polynomials evaluated in bucket order; against the
    element-pair MFMA kernels and the full filter chains
    (SO3LR_NO_RADIAL_TABLES=1).  The fits hold to about 1e-16 (values) and
    4e-15 (slopes) of their largest magnitudes, so the two agree to
    rounding; the kernel timings show which path ran."""
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden(name)
    monkeypatch.setenv("SO3LR_SCALAR_FILTER_PAIRS", "0")
    if box is None:
        lo, hi, per = pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0)
    else:
        lo, hi, per = np.zeros(3), box, (1, 1, 1)
    results = []
    for off in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_RADIAL_TABLES", off)
        c = Context(support.MODEL, 0)
        c.kernel_timing(True)
        c.set_system(z, q, m)
        lists = Lists(pos, lo, hi, per)
        c.set_topology(lists)
        e, f, ea, w = c.compute(lists.rows_positions(pos))
        ran = {k: _launches(c, k) for k in ("filter_fwd_block0_radial", "filter_bwd_block0_radial",
                                             "filter_fwd_block0_tables", "filter_bwd_block0_tables",
                                             "filter_fwd_radial", "filter_bwd_radial", "filter_fwd", "filter_bwd")}
        results.append((e, f.copy(), ea.copy(), w.copy(), ran))
        c.close()
    (e1, f1, ea1, w1, ran1), (e2, f2, ea2, w2, ran2) = results
    print("%s: |dE| %.2e max|dF| %.2e max|dW| %.2e" % (name, abs(e1 - e2), np.abs(f1 - f2).max(),
                                                       np.abs(w1 - w2).max()), flush=True)
    assert ran1["filter_fwd_block0_tables"] == 1 and ran1["filter_fwd_block0_radial"] == 0
    assert ran2["filter_fwd_block0_radial"] == 1 and ran2["filter_bwd_block0_radial"] == 1
    assert ran2["filter_fwd_block0_tables"] == 0 and ran2["filter_bwd_block0_tables"] == 0
    # the blocks after 0: their radial tables (two blocks), or the full chains
    assert ran2["filter_fwd_radial"] == 2 and ran2["filter_bwd_radial"] == 2 and ran2["filter_fwd"] == 0
    assert ran1["filter_fwd"] == 2 and ran1["filter_bwd"] == 2 and ran1["filter_fwd_radial"] == 0
    assert abs(e1 - e2) <= 1e-13 * abs(e2)
    assert np.abs(f1 - f2).max() <= 1e-11
    assert np.abs(w1 - w2).max() <= 1e-11 * max(1.0, np.abs(w2).max())
    assert np.abs(ea1 - ea2).max() <= 1e-12 * max(1.0, np.abs(ea2).max())


def test_graph_replay_matches_eager(monkeypatch):
    """Identical repeated calls replay a captured graph of the evaluation.
    Every replay -- with torch work, an evaluation under a different key, moved
    positions and a reneighbor in between -- matches an eager-only context bit
    for bit."""
    import torch
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden("water3000")
    monkeypatch.setenv("SO3LR_NO_GRAPH", "1")
    eager = Context(support.MODEL, 0)
    monkeypatch.delenv("SO3LR_NO_GRAPH")
    graph = Context(support.MODEL, 0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    rng = np.random.default_rng(11)
    with torch.cuda.stream(stream):
        xt = torch.tensor(pos, dtype=torch.float64, device=dev)
        fe = torch.zeros_like(xt)
        fg = torch.zeros_like(xt)
        other = torch.zeros_like(xt)
        for c in (eager, graph):
            c.set_system(z, 0, 1)
            c.reneighbor_device(xt, np.zeros(3), box, (1, 1, 1), 1.0, stream=stream.cuda_stream)
        for k in range(8):
            if k == 5:  # new topology: the graph is dropped and captured again
                for c in (eager, graph):
                    c.reneighbor_device(xt, np.zeros(3), box, (1, 1, 1), 1.0, stream=stream.cuda_stream)
            e1, w1 = eager.compute_device(xt, fe, stream=stream.cuda_stream)
            e2, w2 = graph.compute_device(xt, fg, stream=stream.cuda_stream)
            stream.synchronize()
            assert e1 == e2, k
            assert np.array_equal(w1, w2), k
            assert torch.equal(fe, fg), k
            # eager work between replays: torch kernels, another key, moved atoms
            other.copy_(fg).mul_(0.5)
            graph.compute_device(xt, other, stream=stream.cuda_stream)
            xt.add_(torch.tensor(rng.normal(scale=1e-3, size=pos.shape), dtype=torch.float64, device=dev))
            stream.synchronize()


def test_topology_faults_are_refused():
    """so3lr_set_topology builds the pair tables on the GPU; malformed LAMMPS
    lists come back as SO3LR_ERR_TOPOLOGY (owner map, a row out of range, an
    atom paired with its own image, a full list missing a reverse edge), and
    the context stays usable."""
    from so3lrxlammps_amd import Context, Lists, _lib
    ref, z, pos, box = support.load_golden("water3000")
    c = Context(support.MODEL, 0)
    c.set_system(z, 0, 1)
    lists = Lists(pos, np.zeros(3), box, (1, 1, 1))
    (si, so, sn), (li, lo_, ln) = lists.lists
    n = len(z)

    def submit(owner=lists.owner, sneigh=sn, lneigh=ln):
        owner = np.ascontiguousarray(owner, dtype=np.int32)
        sneigh = np.ascontiguousarray(sneigh, dtype=np.int32)
        lneigh = np.ascontiguousarray(lneigh, dtype=np.int32)
        rc = c._lib.so3lr_set_topology(c._h, lists.rows, _lib.ptr(owner), _lib.LIST_FULL, len(si), _lib.ptr(si),
                                       _lib.ptr(so), _lib.ptr(sneigh), len(li), _lib.ptr(li), _lib.ptr(lo_),
                                       _lib.ptr(lneigh))
        return rc, c._lib.so3lr_last_error(c._h).decode()

    bad_owner = lists.owner.copy()
    bad_owner[n + 3] = n + 7  # a ghost mapped outside the owned atoms
    rc, msg = submit(owner=bad_owner)
    assert rc == _lib.ERR_TOPOLOGY and "owner_of_row" in msg, msg
    bad = sn.copy()
    bad[5] = lists.rows + 2  # a row that does not exist
    rc, msg = submit(sneigh=bad)
    assert rc == _lib.ERR_TOPOLOGY and "out of range" in msg, msg
    ghost = n + 10
    i = int(lists.owner[ghost])
    bad = ln.copy()
    bad[lo_[i]] = ghost  # atom i paired with its own image
    rc, msg = submit(lneigh=bad)
    assert rc == _lib.ERR_TOPOLOGY and "own periodic image" in msg, msg
    bad = sn.copy()
    bad[so[0]] = si[0]  # the receiver itself (skipped): its partner's reverse edge is now unmatched
    rc, msg = submit(sneigh=bad)
    assert rc == _lib.ERR_TOPOLOGY and "not symmetric" in msg, msg
    # still usable: the good lists give the rows-path result of a fresh context
    c.set_topology(lists)
    e1, f1, _, w1 = c.compute(lists.rows_positions(pos))
    c2 = Context(support.MODEL, 0)
    c2.set_system(z, 0, 1)
    c2.set_topology(lists)
    e2, f2, _, w2 = c2.compute(lists.rows_positions(pos))
    assert e1 == e2 and np.array_equal(f1, f2) and np.array_equal(w1, w2)
    c.close()
    c2.close()


def test_active_pair_capacity_overflow_reevaluates():
    """The per-pair buffers hold the active pairs counted at the first
    evaluation of a topology plus 1/8; a geometry with more pairs inside the
    cutoff (here the positions compressed by 6 %) makes the evaluation grow
    them and run again.  Its result must be bit-identical to a context that
    counted at that geometry in the first place."""
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden("water3000")
    lists = Lists(pos, np.zeros(3), box, (1, 1, 1))
    rows0 = lists.rows_positions(pos)
    rows1 = np.ascontiguousarray(rows0 * 0.94)
    a = Context(support.MODEL, 0)
    a.set_system(z, 0, 1)
    a.set_topology(lists)
    a.compute(rows0)
    n0 = a.graph_stats()[0]
    e1, f1, ea1, w1 = a.compute(rows1)
    assert a.graph_stats()[0] > n0 + n0 // 8 + 256  # the compressed geometry overflowed the capacity
    b = Context(support.MODEL, 0)
    b.set_system(z, 0, 1)
    b.set_topology(lists)
    e2, f2, ea2, w2 = b.compute(rows1)
    assert e1 == e2 and np.array_equal(f1, f2) and np.array_equal(ea1, ea2) and np.array_equal(w1, w2)
    a.close()
    b.close()


def test_refused_first_evaluation_leaves_context_usable():
    """The first evaluation of a single system's LAMMPS-list topology puts its
    nodes in spatial order and sorts the incidence there.  A first evaluation
    with a non-finite owned position is refused before any of that; the next
    finite evaluation on the same context must order the topology itself and
    equal, bit for bit, a fresh context's first evaluation."""
    from so3lrxlammps_amd import Context, Lists, _lib
    ref, z, pos, box = support.load_golden("alanine")
    lists = Lists(pos, pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0))
    rows = lists.rows_positions(pos)
    bad = rows.copy()
    bad[3, 1] = np.nan
    a = Context(support.MODEL, 0)
    a.set_system(z, 0, 1)
    a.set_topology(lists)
    print("case alanine, NaN first evaluation", flush=True)
    with pytest.raises(_lib.SO3LRError) as err:
        a.compute(bad)
    assert err.value.code == _lib.ERR_ARGUMENT and "non-finite" in str(err.value)
    got = a.compute(rows)
    b = Context(support.MODEL, 0)
    b.set_system(z, 0, 1)
    b.set_topology(lists)
    want = b.compute(rows)
    assert got[0] == want[0]
    for g, w in zip(got[1:], want[1:]):
        assert np.array_equal(g, w)
    a.close()
    b.close()
