"""The oracle at the widths the reference runs beyond F = 128, R = 32 and
degrees 1,2,3,4 (so3lr_capabilities.cpp:54-85): F = 256 (8 heads, 8 degree
slots), R = 64, energy/charge heads narrower than F, and duplicated degrees.

No reference fixture exists at these widths, so they are pinned by what the
mathematics fixes:

* the two-copy lift (support.lifted_model): an F = 256, R = 64 model with the
  degree slots 1,1,2,2,3,3,4,4 and head width 128 that computes the same
  function as the F = 128 model it lifts gives that model's energies,
  charges, Hirshfeld ratios, forces and virial; the lift splits every summed
  weight unevenly between the copies, so the copies' adjoints differ;
* on a lift whose weights are then perturbed (the copies no longer agree),
  forces and virial are central finite differences of the energy;
* duplicated and missing degrees at F = 128 (slots 1,1,2,3 and 1,2,3,3): the
  energy is invariant under rotations (which fails if a slot's channels are
  not the harmonics of its degree) and the forces are finite differences of
  the energy;
* the other width combinations (F = 128 with R = 64, F = 256 with R = 32,
  heads 192 wide at F = 128), each built to equal the shipped model; heads
  whose new units feed the outputs, by finite differences.
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle
from test_oracle_math import _small_periodic


@pytest.fixture(scope="module")
def tmp(tmp_path_factory):
    return tmp_path_factory.mktemp("wide")


@pytest.fixture(scope="module")
def v1():
    return Oracle(support.MODEL)


@pytest.fixture(scope="module")
def wide(tmp):
    return Oracle(support.lifted_model(tmp / "wide.so3lr"))


def _golden(name):
    ref, z, pos, box = support.load_golden(name)
    return z, pos, ref.get("charge", 0), ref.get("multiplicity", 1)


def _run(orc, z, pos, q=0, m=1, box=None):
    return orc.evaluate(z, *support.build_graphs(pos, box), charge=q, multiplicity=m)


def _same(a, b):
    assert abs(a["energy"] - b["energy"]) <= 1e-12 * abs(b["energy"])
    for k in ("charges", "hirshfeld", "e_learned", "e_lr"):
        assert np.abs(a[k] - b[k]).max() <= 1e-11, k
    assert np.abs(a["forces"] - b["forces"]).max() <= 1e-10
    assert np.abs(a["virial"] - b["virial"]).max() <= 1e-10 * max(1.0, np.abs(b["virial"]).max())


def test_lift_widths(wide):
    arch = wide.model.arch
    assert (arch["invariant_features"], arch["attention_heads"], arch["euclidean_degree_channels"],
            arch["radial_basis_features"]) == (256, 8, 8, 64)
    st = wide._st
    assert (st.F, st.R, st.n_slots, st.head_hidden) == (256, 64, 8, 128)
    assert list(st.degrees) == [1, 1, 2, 2, 3, 3, 4, 4]


@pytest.mark.parametrize("name", ["acetate", "alanine_cation"])
def test_lift_equals_base_molecules(wide, v1, name):
    z, pos, q, m = _golden(name)
    _same(_run(wide, z, pos, q, m), _run(v1, z, pos, q, m))


def test_lift_equals_base_periodic(wide, v1):
    z, pos, box = _small_periodic(n_mol=16)
    _same(_run(wide, z, pos, box=box), _run(v1, z, pos, box=box))


def test_lift_of_option_model_equals_it(tmp, v1):
    """The lift of a model with RMSNorm, QK normalisation, residual scalars,
    NLH repulsion and the C6 head (4 blocks)."""
    from test_oracle_arch import _all_options_a
    base = _all_options_a(tmp, v1)
    lifted = Oracle(support.lifted_model(tmp / "wide_options.so3lr", base=base))
    z, pos, q, m = _golden("acetate")
    a, b = _run(lifted, z, pos, q, m), _run(Oracle(base), z, pos, q, m)
    _same(a, b)
    assert np.abs(a["c6_ratios"] - b["c6_ratios"]).max() <= 1e-11


@pytest.fixture(scope="module")
def wide_perturbed(tmp):
    lift = support.lifted_model(tmp / "wide_b.so3lr")
    return Oracle(support.perturbed_model(tmp / "wide_p.so3lr", seed=23, scale=0.2, base=lift))


def test_perturbed_lift_is_another_function(wide_perturbed, v1):
    z, pos, q, m = _golden("acetate")
    assert abs(_run(wide_perturbed, z, pos, q, m)["energy"] - _run(v1, z, pos, q, m)["energy"]) > 1e-2


def _fd_forces(orc, z, pos, q, m, atoms, tol=2e-6):
    out = _run(orc, z, pos, q, m)
    h = 1e-4
    for i in atoms:
        for a in range(3):
            p1 = pos.copy(); p1[i, a] += h
            p2 = pos.copy(); p2[i, a] -= h
            fd = -(_run(orc, z, p1, q, m)["energy"] - _run(orc, z, p2, q, m)["energy"]) / (2 * h)
            assert abs(fd - out["forces"][i, a]) < tol, (i, a, fd, out["forces"][i, a])


def test_wide_forces_finite_difference(wide_perturbed):
    z, pos, q, m = _golden("acetate")
    _fd_forces(wide_perturbed, z, pos, q, m, (0, 3, 6))


def test_wide_virial_finite_difference(wide_perturbed):
    z, pos, box = _small_periodic(n_mol=12)
    sr, lr = support.build_graphs(pos, box)
    out = wide_perturbed.evaluate(z, sr, lr)
    h = 1e-5
    for k, (a, b) in enumerate([(0, 0), (1, 1), (2, 2), (0, 1), (0, 2), (1, 2)]):
        S = np.zeros((3, 3)); S[a, b] += 0.5; S[b, a] += 0.5
        es = []
        for t in (h, -h):
            M = np.eye(3) + t * S
            es.append(wide_perturbed.evaluate(z, (sr[0], sr[1], sr[2] @ M.T), (lr[0], lr[1], lr[2] @ M.T))["energy"])
        dEdt = (es[0] - es[1]) / (2 * h)
        assert abs(-dEdt - out["virial"][k]) < 2e-6 * max(1.0, abs(out["virial"][k])), (k, -dEdt, out["virial"][k])


@pytest.mark.parametrize("kind", ["f128_r64", "f256_r32", "head_width_192"])
def test_other_width_combinations_equal_base(tmp, v1, kind):
    """The other combinations of the accepted widths, each built to compute
    the shipped model's function: F = 128 with R = 64 (degree elevation
    only), F = 256 with R = 32 (the lift without elevation), and energy/charge
    heads 192 wide at F = 128 (64 new units with zero output weights)."""
    path = {"f128_r64": lambda: support.lifted_model(tmp / "r64.so3lr", copies=1, R=64),
            "f256_r32": lambda: support.lifted_model(tmp / "f256r32.so3lr", copies=2, R=32),
            "head_width_192": lambda: support.head_width_model(tmp / "hk192.so3lr", 192)}[kind]()
    orc = Oracle(path)
    widths = {"f128_r64": (128, 64, 128), "f256_r32": (256, 32, 128), "head_width_192": (128, 32, 192)}[kind]
    assert (orc._st.F, orc._st.R, orc._st.head_hidden) == widths
    for name in ("acetate", "alanine_cation"):
        z, pos, q, m = _golden(name)
        _same(_run(orc, z, pos, q, m), _run(v1, z, pos, q, m))


def test_live_head_width_forces_finite_difference(tmp, v1):
    """Heads 192 wide whose new units feed the outputs: another function
    (checked), forces = -dE/dx."""
    orc = Oracle(support.head_width_model(tmp / "hk192_live.so3lr", 192, live=True))
    z, pos, q, m = _golden("acetate")
    assert abs(_run(orc, z, pos, q, m)["energy"] - _run(v1, z, pos, q, m)["energy"]) > 1e-3
    _fd_forces(orc, z, pos, q, m, (1, 5))


@pytest.mark.parametrize("degrees", [(1, 1, 2, 3), (1, 2, 3, 3)])
def test_duplicated_degrees(tmp, v1, degrees):
    orc = Oracle(support.degrees_model(tmp / ("deg_%s.so3lr" % "".join(map(str, degrees))), degrees))
    assert list(orc._st.degrees)[:4] == list(degrees)
    z, pos, q, m = _golden("alanine_cation")
    base = _run(orc, z, pos, q, m)
    assert abs(base["energy"] - _run(v1, z, pos, q, m)["energy"]) > 1e-3
    rng = np.random.default_rng(17)
    Q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    if np.linalg.det(Q) < 0:
        Q[:, 0] = -Q[:, 0]
    rot = _run(orc, z, pos @ Q.T + np.array([1.0, -2.5, 4.0]), q, m)
    assert abs(rot["energy"] - base["energy"]) < 1e-9
    assert np.abs(rot["forces"] - base["forces"] @ Q.T).max() < 1e-9
    _fd_forces(orc, z, pos, q, m, (0, 4))
