"""Pins of the oracle that the golden vectors leave open: closed forms,
finite differences of the energy and symmetry invariants.

* spherical harmonics: orthonormality on an exact product quadrature (pins
  every constant and index of the 24 polynomials);
* forces: central finite differences of E (pins every hand-derived reverse
  step: SH VJP, Bernstein/cutoff derivatives, LayerNorm/MLP/attention adjoints,
  LR radial and dE/dq, dE/dh seeds);
* virial: finite differences of E under homogeneous strain of every edge and
  pair vector (pins the sign, the symmetrisation and the LR half-pair term);
* rotation / translation invariance and zero net torque (pins equivariance);
* charge/spin: the table is exactly zero for Q=0, M=1, and (Q, M) parity rules;
* per-atom virial: sum rule against the virial, dimer symmetry, permutation,
  shift, and the f.r identity of an isolated molecule;
* Na and Cl rows (no golden vector holds an ion): relabelling H -> Na and
  N -> Cl together with a model whose element tables trade those rows leaves
  every term but ZBL unchanged (ZBL reads no table: it is one function of
  the nuclear charges for every element, pinned by the molecules' goldens).
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle, spherical_harmonics


@pytest.fixture(scope="module")
def orc():
    return Oracle(support.MODEL)


def test_sh_orthonormal():
    # Gauss-Legendre in cos(theta) x uniform phi: exact for degree <= 8 products
    xg, wg = np.polynomial.legendre.leggauss(12)
    phis = np.arange(24) * (2 * np.pi / 24)
    ct, ph = np.meshgrid(xg, phis, indexing="ij")
    w = np.meshgrid(wg, np.full(24, 2 * np.pi / 24), indexing="ij")
    w = (w[0] * w[1]).ravel()
    st = np.sqrt(1 - ct ** 2)
    u = np.stack([st * np.cos(ph), st * np.sin(ph), ct], -1).reshape(-1, 3)
    Y = spherical_harmonics(u)
    G = (Y * w[:, None]).T @ Y
    assert np.abs(G - np.eye(24)).max() < 1e-13


def test_sh_known_values():
    # l=1 is sqrt(3/4pi) (y, z, x); Y_{2,0}(z-axis) = sqrt(5/(4pi)); Y_{4,0}(z) = 3/sqrt(4pi)
    Y = spherical_harmonics(np.array([[0.0, 0.0, 1.0], [1.0, 0.0, 0.0]]))
    c1 = np.sqrt(3 / (4 * np.pi))
    assert np.allclose(Y[0, :3], [0, c1, 0], atol=1e-15)
    assert np.allclose(Y[1, :3], [0, 0, c1], atol=1e-15)
    assert abs(Y[0, 5] - np.sqrt(5 / (4 * np.pi))) < 1e-15
    assert abs(Y[0, 19] - 3 / np.sqrt(4 * np.pi)) < 1e-15


def _molecule(name):
    ref, z, pos, box = support.load_golden(name)
    return ref, z, pos


def _energy(orc, z, pos, q=0, m=1, box=None):
    sr, lr = support.build_graphs(pos, box)
    return orc.evaluate(z, sr, lr, charge=q, multiplicity=m)


@pytest.mark.parametrize("name", ["acetate", "methyl"])
def test_forces_finite_difference(orc, name):
    ref, z, pos = _molecule(name)
    q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
    out = _energy(orc, z, pos, q, m)
    h = 1e-4
    rng = np.random.default_rng(7)
    for i in rng.choice(len(z), size=min(4, len(z)), replace=False):
        for a in range(3):
            p1 = pos.copy(); p1[i, a] += h
            p2 = pos.copy(); p2[i, a] -= h
            fd = -(_energy(orc, z, p1, q, m)["energy"] - _energy(orc, z, p2, q, m)["energy"]) / (2 * h)
            assert abs(fd - out["forces"][i, a]) < 2e-6, (i, a, fd, out["forces"][i, a])


def _small_periodic(seed=3, n_mol=24, box=25.0):
    """Sparse periodic water gas in a 25 A box (box > 2 x 12 A LR cutoff)."""
    rng = np.random.default_rng(seed)
    pos, z = [], []
    tmpl = np.array([[0.0, 0.0, 0.0], [0.9572, 0.0, 0.0],
                     [0.9572 * np.cos(np.radians(104.52)), 0.9572 * np.sin(np.radians(104.52)), 0.0]])
    centers = []
    while len(centers) < n_mol:
        c = rng.uniform(0, box, 3)
        if all(np.linalg.norm((c - o) - box * np.round((c - o) / box)) > 3.2 for o in centers):
            centers.append(c)
    for c in centers:
        q_, _ = np.linalg.qr(rng.normal(size=(3, 3)))
        for k, zz in enumerate((8, 1, 1)):
            pos.append(c + tmpl[k] @ q_.T)
            z.append(zz)
    pos = np.mod(np.array(pos), box)
    return np.array(z), pos, np.full(3, box)


def test_virial_finite_difference(orc):
    z, pos, box = _small_periodic()
    sr, lr = support.build_graphs(pos, box)
    out = orc.evaluate(z, sr, lr)
    h = 1e-5
    comps = [(0, 0), (1, 1), (2, 2), (0, 1), (0, 2), (1, 2)]
    for k, (a, b) in enumerate(comps):
        S = np.zeros((3, 3)); S[a, b] += 0.5; S[b, a] += 0.5
        es = []
        for t in (h, -h):
            M = np.eye(3) + t * S
            sr2 = (sr[0], sr[1], sr[2] @ M.T)
            lr2 = (lr[0], lr[1], lr[2] @ M.T)
            es.append(orc.evaluate(z, sr2, lr2)["energy"])
        dEdt = (es[0] - es[1]) / (2 * h)
        assert abs(-dEdt - out["virial"][k]) < 2e-6 * max(1.0, abs(out["virial"][k])), (k, -dEdt, out["virial"][k])


def test_rotation_translation_invariance(orc):
    ref, z, pos = _molecule("alanine_cation")
    base = _energy(orc, z, pos, 1, 2)
    rng = np.random.default_rng(11)
    Q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    if np.linalg.det(Q) < 0:
        Q[:, 0] = -Q[:, 0]
    rot = _energy(orc, z, pos @ Q.T + np.array([3.0, -1.5, 7.25]), 1, 2)
    assert abs(rot["energy"] - base["energy"]) < 1e-9
    assert np.abs(rot["forces"] - base["forces"] @ Q.T).max() < 1e-9
    # net force and net torque vanish for an isolated molecule
    assert np.abs(base["forces"].sum(0)).max() < 1e-10
    torque = np.cross(pos, base["forces"]).sum(0)
    assert np.abs(torque).max() < 1e-9


def test_permutation_invariance(orc):
    ref, z, pos = _molecule("acetate")
    base = _energy(orc, z, pos, -1, 1)
    perm = np.random.default_rng(5).permutation(len(z))
    out = _energy(orc, z[perm], pos[perm], -1, 1)
    assert abs(out["energy"] - base["energy"]) < 1e-10
    assert np.abs(out["forces"] - base["forces"][perm]).max() < 1e-11


def test_charge_spin_table_rules(orc):
    counts = np.zeros(119, dtype=np.int64)
    counts[1], counts[8] = 2, 1
    assert np.all(orc.charge_spin_table(counts, 0, 1) == 0.0)
    assert np.any(orc.charge_spin_table(counts, 1, 2) != 0.0)
    # (Q, M) rules: H2O has 10 electrons
    assert Oracle.charge_multiplicity_problem(counts, 0, 1) == 0
    assert Oracle.charge_multiplicity_problem(counts, 0, 2) != 0     # parity
    assert Oracle.charge_multiplicity_problem(counts, 0.5, 1) != 0   # non-integer Q
    assert Oracle.charge_multiplicity_problem(counts, 0, 0) != 0     # M < 1
    assert Oracle.charge_multiplicity_problem(counts, 11, 1) != 0    # negative electrons
    assert Oracle.charge_multiplicity_problem(counts, 1, 2) == 0


def test_packed_images_match_single(orc):
    """Per-image charge correction: a pack equals each image alone."""
    names = [("acetate", -1, 1), ("methyl", 0, 2), ("h2o_cation", 1, 2)]
    zs, ps, imgs, qs, ms, singles = [], [], [], [], [], []
    offset = np.zeros(3)
    for k, (name, q, m) in enumerate(names):
        ref, z, pos = _molecule(name)
        singles.append(_energy(orc, z, pos, q, m))
        zs.append(z); ps.append(pos + offset); imgs.append(np.full(len(z), k))
        qs.append(q); ms.append(m)
        offset = offset + np.array([40.0, 0, 0])
    z = np.concatenate(zs); pos = np.concatenate(ps)
    sr, lr = support.build_graphs(pos, None)
    # images are > 12 A apart: no inter-image pair exists
    out = orc.evaluate(z, sr, lr, image=np.concatenate(imgs), image_charge=np.array(qs, float),
                       image_multiplicity=ms)
    start = 0
    for k, s in enumerate(singles):
        n = len(s["charges"])
        assert abs(out["image_energy"][k] - s["energy"]) < 1e-10
        assert np.abs(out["forces"][start:start + n] - s["forces"]).max() < 1e-12
        start += n


def test_per_atom_virial(orc):
    """Per-atom virial (an addition: the reference refuses vflag_atom).  Each
    edge's and LR pair's -v (x) dE/dv goes half to each endpoint.  Pins: the
    atoms' sum is the global virial, itself pinned by the strain finite
    differences above (a dropped term, a wrong weight or a missing LR part
    breaks it); the two atoms of a dimer get equal shares (a term given to one
    endpoint only breaks it, since the two directed edges carry different
    gradients); permuting the atoms permutes the rows; a rigid shift changes
    nothing; for an isolated molecule the sum equals sym(sum_i x_i (x) f_i)."""
    z, pos, box = _small_periodic()
    sr, lr = support.build_graphs(pos, box)
    out = orc.evaluate(z, sr, lr)
    assert np.abs(out["vatom"].sum(0) - out["virial"]).max() < 1e-12 * np.abs(out["virial"]).max()

    ref, z2, p2 = _molecule("o2")
    o2 = _energy(orc, z2, p2, 0, 3)
    assert np.abs(o2["vatom"][0] - o2["vatom"][1]).max() <= 1e-15 * np.abs(o2["vatom"]).max()
    assert np.abs(o2["vatom"].sum(0) - o2["virial"]).max() < 1e-13 * max(1.0, np.abs(o2["virial"]).max())

    ref, z3, p3 = _molecule("acetate")
    base = _energy(orc, z3, p3, -1, 1)
    perm = np.random.default_rng(6).permutation(len(z3))
    out3 = _energy(orc, z3[perm], p3[perm], -1, 1)
    assert np.abs(out3["vatom"] - base["vatom"][perm]).max() < 1e-11
    shifted = _energy(orc, z3, p3 + np.array([5.0, -3.0, 2.5]), -1, 1)
    assert np.abs(shifted["vatom"] - base["vatom"]).max() < 1e-11
    x, f = p3, base["forces"]
    fdotr = np.array([(x[:, 0] * f[:, 0]).sum(), (x[:, 1] * f[:, 1]).sum(), (x[:, 2] * f[:, 2]).sum(),
                      0.5 * (x[:, 0] * f[:, 1] + x[:, 1] * f[:, 0]).sum(),
                      0.5 * (x[:, 0] * f[:, 2] + x[:, 2] * f[:, 0]).sum(),
                      0.5 * (x[:, 1] * f[:, 2] + x[:, 2] * f[:, 1]).sum()])
    assert np.abs(base["vatom"].sum(0) - fdotr).max() < 1e-9


def test_ion_rows_by_relabelling(orc, tmp_path):
    """Na (Z = 11) and Cl (Z = 17) through every per-element table: alanine
    with H relabelled Na and N relabelled Cl, evaluated with a model whose
    tables trade the rows of those elements (support.relabelled_model, at
    the reference's own indexing of each table), gives the original learned
    energies, charges, Hirshfeld ratios and long-range energies atom by atom.
    A table read at the wrong row for Z > 10 only (an 8- or 10-element table,
    an index off by one past neon) changes one of them.  The electron parity
    is unchanged (+10 per relabelled atom), so (Q, M) stays valid."""
    ref, z, pos, box = support.load_golden("alanine_cation")
    q, m = ref["charge"], ref["multiplicity"]
    sr, lr = support.build_graphs(pos, box)
    base = orc.evaluate(z, sr, lr, charge=q, multiplicity=m)
    z2 = np.asarray(z).copy()
    z2[z2 == 1] = 11
    z2[z2 == 7] = 17
    assert (z2 == 11).any() and (z2 == 17).any()
    relab = Oracle(support.relabelled_model(tmp_path / "relabelled.so3lr")).evaluate(
        z2, sr, lr, charge=q, multiplicity=m)
    for key in ("e_learned", "charges", "hirshfeld", "e_lr"):
        np.testing.assert_allclose(relab[key], base[key], rtol=1e-13, atol=1e-14, err_msg=key)
    assert not np.allclose(relab["e_zbl"], base["e_zbl"])
