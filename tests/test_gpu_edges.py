"""Edge cases of the HIP path against the CPU oracle, through the C ABI.

Systems with no short-range pair at all (one atom; two ions 8 A apart, so
only the long-range pair is active), a pair just inside and one just outside
the 4.5 A cutoff, and packed images down to one atom each, with their own
charge and multiplicity (a bare proton, an open-shell H atom, triplet O).
Both the LAMMPS-rows path and the HBM-resident device path are checked at the
bars of the other parity tests: energy 1e-10 relative, forces and virial
1e-9 eV/A; each case runs on the shipped model (with the filter kernels
the library picks for these sizes, and with the fused MFMA ones forced) and
on an F = 256 model (generic kernels).
"""
import os

import numpy as np
import pytest

import support
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["v1", "v1_mfma", "generic"])
def model(request, tmp_path_factory):
    """The shipped model (v1 kernels: these systems are small enough for the
    scalar filter kernels), the same with the fused MFMA filters forced
    (SO3LR_SCALAR_FILTER_PAIRS=0 while its tests create their contexts), and
    a perturbed F = 256, R = 64 lift with duplicated degrees (generic
    kernels)."""
    if request.param == "v1":
        yield support.MODEL
    elif request.param == "v1_mfma":
        old = os.environ.get("SO3LR_SCALAR_FILTER_PAIRS")
        os.environ["SO3LR_SCALAR_FILTER_PAIRS"] = "0"
        yield support.MODEL
        if old is None:
            del os.environ["SO3LR_SCALAR_FILTER_PAIRS"]
        else:
            os.environ["SO3LR_SCALAR_FILTER_PAIRS"] = old
    else:
        d = tmp_path_factory.mktemp("edges")
        yield support.perturbed_model(d / "wide_p.so3lr", seed=23, scale=0.2,
                                      base=support.lifted_model(d / "wide.so3lr"))


@pytest.fixture(scope="module")
def orc(model):
    return Oracle(model)


def _check(e, f, w, out):
    support.record_margin(e, f, w, out)
    assert abs(e - out["energy"]) <= 1e-10 * max(1.0, abs(out["energy"])), (e, out["energy"])
    assert np.abs(f - out["forces"]).max() <= 1e-9
    assert np.abs(w - out["virial"]).max() <= 1e-9  # eV, absolute


def _both_paths(z, x, q, m, orc, model):
    """Rows path and device path of one open (non-periodic) system vs the oracle."""
    import torch
    from so3lrxlammps_amd import Context, Lists
    sr, lr = support.build_graphs(x, None)
    out = orc.evaluate(z, sr, lr, charge=q, multiplicity=m)
    lo, hi = x.min(0) - 20.0, x.max(0) + 20.0
    c = Context(model, 0)
    c.set_system(z, q, m)
    lists = Lists(x, lo, hi, (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(x))
    _check(e, f, w, out)
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        xt = torch.tensor(x, dtype=torch.float64, device=dev)
        ft = torch.zeros_like(xt)
        c.reneighbor_device(xt, lo, hi, (0, 0, 0), 1.0, stream=stream.cuda_stream)
        e2, w2 = c.compute_device(xt, ft, stream=stream.cuda_stream)
        stream.synchronize()
        f2 = ft.cpu().numpy()
    _check(e2, f2, w2, out)
    c.close()
    return out


def test_single_atom(orc, model):
    """One O atom (triplet): no pair of any kind, energy from the heads alone."""
    z = np.array([8])
    x = np.array([[1.0, 2.0, 3.0]])
    out = _both_paths(z, x, 0.0, 3.0, orc, model)
    assert np.abs(out["forces"]).max() == 0.0


def test_long_range_pair_only(orc, model):
    """Na+ and Cl- 8 A apart: no short-range candidate, one long-range pair."""
    z = np.array([11, 17])
    x = np.array([[0.0, 0.0, 0.0], [8.0, 0.0, 0.0]])
    out = _both_paths(z, x, 0.0, 1.0, orc, model)
    assert np.abs(out["forces"]).max() > 0.0


@pytest.mark.parametrize("r", [4.5 - 1e-7, 4.5 + 1e-7])
def test_pair_at_short_range_cutoff(orc, model, r):
    """Two water molecules with one O-O distance just inside / just outside
    the 4.5 A short-range cutoff."""
    oh, ang = 0.9572, np.deg2rad(104.52)
    w1 = np.array([[0.0, 0.0, 0.0], [oh, 0.0, 0.0], [oh * np.cos(ang), oh * np.sin(ang), 0.0]])
    w2 = w1 @ np.diag([-1.0, 1.0, -1.0]) + np.array([r, 0.0, 0.0])
    z = np.array([8, 1, 1, 8, 1, 1])
    x = np.vstack([w1, w2])
    d = np.linalg.norm(x[:, None] - x[None], axis=-1)
    assert abs(d[0, 3] - r) < 1e-12
    _both_paths(z, x, 0.0, 1.0, orc, model)


def test_packed_tiny_images(orc, model):
    """Packed images of 1-3 atoms, each with its own (Q, M), through the rows
    path: H2, a bare proton, an H atom (doublet), a triplet O atom, OH-."""
    from so3lrxlammps_amd import Context, Lists
    mols = [([1, 1], [[0, 0, 0], [0.74, 0, 0]], 0.0, 1.0),
            ([1], [[0, 0, 0]], 1.0, 1.0),
            ([1], [[0, 0, 0]], 0.0, 2.0),
            ([8], [[0, 0, 0]], 0.0, 3.0),
            ([8, 1], [[0, 0, 0], [0.97, 0, 0]], -1.0, 1.0)]
    z, x, offs, qs, ms = [], [], [0], [], []
    for k, (zz, xx, q, m) in enumerate(mols):
        z += zz
        x += [np.array(p, float) + np.array([40.0 * k, 0.0, 0.0]) for p in xx]  # images 40 A apart
        offs.append(len(z))
        qs.append(q)
        ms.append(m)
    z, x, offs = np.array(z), np.array(x), np.array(offs)
    img = np.repeat(np.arange(len(qs)), np.diff(offs))
    sr, lr = support.build_graphs(x, None)
    out = orc.evaluate(z, sr, lr, image=img, image_charge=np.array(qs), image_multiplicity=np.array(ms))
    c = Context(model, 0)
    c.set_images(z, offs, qs, ms)
    lo, hi = x.min(0) - 20.0, x.max(0) + 20.0
    lists = Lists(x, lo, hi, (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(x))
    _check(e, f, w, out)
    t = c.terms()
    assert np.abs(t["image_energy"] - out["image_energy"]).max() <= 1e-10 * np.abs(out["image_energy"]).max()
    for k in range(len(qs)):
        assert abs(t["charges"][offs[k]:offs[k + 1]].sum() - qs[k]) < 1e-12
    c.close()
