"""The pair-style mirror (so3lrxlammps_amd/pair_style.py) driving the HIP
library as LAMMPS drives PairSO3LRNativeMPI: settings / coeff / init_style /
compute on a charged molecule and on the periodic 3,000-atom water, with
moves inside and beyond half the skin (list reuse and rebuild), against the
CPU oracle at the parity bars (energy 1e-10 relative; forces 1e-9 eV/A;
the virial 1e-9 eV absolute; per-atom virial 1e-9 and per-atom energy 1e-10
of their scale), and the (Q, M) refusal of init_style."""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle
from so3lrxlammps_amd.pair_style import Atoms, LammpsError, PairSO3LRNativeMPI

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["v1", "generic"])
def model(request, tmp_path_factory):
    """The shipped model and a perturbed F = 256, R = 64 lift (generic kernels)."""
    if request.param == "v1":
        return support.MODEL
    d = tmp_path_factory.mktemp("pair_style")
    return support.perturbed_model(d / "wide_p.so3lr", seed=23, scale=0.2,
                                   base=support.lifted_model(d / "wide.so3lr"))


@pytest.fixture(scope="module")
def orc(model):
    return Oracle(model)


def _setup(name, q, m, model=support.MODEL):
    ref, z, pos, box = support.load_golden(name)
    symbols = ref["types"]
    types = np.array([symbols.index(support.SYMBOLS[int(zz)]) + 1 for zz in z])
    p = PairSO3LRNativeMPI()
    p.settings([model, repr(float(q)), repr(float(m))])
    p.coeff(["*", "*"] + list(symbols), len(symbols))
    assert p.init_one(1, 1) == p.short_range_cutoff
    if box is None:
        atoms = Atoms(x=pos.copy(), types=types, lo=pos.min(0) - 20.0, hi=pos.max(0) + 20.0, periodic=(0, 0, 0))
    else:
        atoms = Atoms(x=pos.copy(), types=types, lo=np.zeros(3), hi=box, periodic=(1, 1, 1))
    p.init_style(atoms)
    return p, atoms, z, box


def _check(res, out):
    support.record_margin(res["energy"], res["forces"], res["virial"], out)
    assert abs(res["energy"] - out["energy"]) <= 1e-10 * abs(out["energy"])
    assert np.abs(res["forces"] - out["forces"]).max() <= 1e-9
    assert np.abs(res["virial"] - out["virial"]).max() <= 1e-9  # eV, absolute
    assert np.abs(res["eatom"] - out["eatom"]).max() <= 1e-10 * max(1.0, np.abs(out["eatom"]).max())
    assert np.abs(res["vatom"] - out["vatom"]).max() <= 1e-9 * max(1.0, np.abs(out["vatom"]).max())


@pytest.mark.parametrize("name,q,m", [("acetate", -1, 1), ("water3000", 0, 1)])
def test_pair_style_matches_oracle(orc, model, name, q, m):
    p, atoms, z, box = _setup(name, q, m, model)
    rng = np.random.default_rng(4)
    for step in range(3):
        if step == 1:  # within half the 1 A skin: the lists are reused
            atoms.x = atoms.x + rng.uniform(-0.05, 0.05, atoms.x.shape)
        if step == 2:  # one atom 0.6 A outward: the lists are rebuilt
            atoms.x = atoms.x + rng.uniform(-0.05, 0.05, atoms.x.shape)
            out = atoms.x[0] - atoms.x.mean(0)
            atoms.x[0] += 0.6 * out / np.linalg.norm(out)
        res = p.compute(atoms, eflag_atom=True, vflag_atom=True)
        x = np.asarray(atoms.x)
        out = orc.evaluate(z, *support.build_graphs(x, box), charge=q, multiplicity=m)
        _check(res, out)
    assert p.topology_rebuilds == 2 and p.topology_hits == 1


def test_init_style_refuses_an_impossible_multiplicity():
    with pytest.raises(LammpsError, match="Pair style so3lr/native/mpi: charge 0"):
        _setup("o2", 0, 2)  # 16 electrons: an even count needs an odd multiplicity
