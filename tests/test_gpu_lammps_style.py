"""The C++ pair style of lammps/pair_so3lr_hip.cpp on the GPU.

PairSO3LRHip, compiled against the LAMMPS API subset of tests/lammps_api/,
is driven the way LAMMPS drives a pair style (settings, coeff, init_style,
init_list, then compute with neighbor->ago), with the rows and lists the
Python mirror (so3lrxlammps_amd/pair_style.py) hands the library at the same
steps.  Both end in the same C-ABI calls, so the C++ style must equal the
mirror bit for bit, and the CPU oracle at the parity bars (energy 1e-10
relative, forces 1e-9 eV/A, virial 1e-9 eV absolute, per-atom energy and
virial 1e-10 and 1e-9 relative to their scale).
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle
from so3lrxlammps_amd.pair_style import Atoms, LammpsError, PairSO3LRNativeMPI

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def orc():
    return Oracle(support.MODEL)


def _setup(name, q, m):
    ref, z, pos, box = support.load_golden(name)
    symbols = ref["types"]
    types = np.array([symbols.index(support.SYMBOLS[int(zz)]) + 1 for zz in z], dtype=np.int32)
    if box is None:
        atoms = Atoms(x=pos.copy(), types=types, lo=pos.min(0) - 20.0, hi=pos.max(0) + 20.0, periodic=(0, 0, 0))
    else:
        atoms = Atoms(x=pos.copy(), types=types, lo=np.zeros(3), hi=box, periodic=(1, 1, 1))
    return symbols, types, atoms, z, box


@pytest.mark.parametrize("name,q,m", [("acetate", -1, 1), ("water3000", 0, 1)])
def test_cxx_style_matches_mirror_and_oracle(orc, name, q, m):
    import lammps_style
    symbols, types, atoms, z, box = _setup(name, q, m)
    py = PairSO3LRNativeMPI(device=0)
    py.settings([support.MODEL, str(q), str(m)])
    py.coeff(["*", "*"] + symbols, ntypes=len(symbols))
    py.init_style(atoms)
    cxx = lammps_style.CxxPairStyle(len(symbols), periodic=atoms.periodic)
    cxx.settings([support.MODEL, str(q), str(m)])
    cxx.coeff(["*", "*"] + symbols)
    assert cxx.init_one(1, 1) == py.init_one(1, 1) == 4.5
    rng = np.random.default_rng(4)
    rebuilds = 0
    for step in range(3):
        if step == 1:  # within half the 1 A skin: the lists are reused
            atoms.x = atoms.x + rng.uniform(-0.05, 0.05, atoms.x.shape)
        if step == 2:  # one atom 0.6 A outward: the lists are rebuilt
            atoms.x = atoms.x + rng.uniform(-0.05, 0.05, atoms.x.shape)
            out = atoms.x[0] - atoms.x.mean(0)
            atoms.x[0] += 0.6 * out / np.linalg.norm(out)
        before = py.topology_rebuilds
        want = py.compute(atoms, eflag_atom=True, vflag_atom=True)
        ago = 0 if py.topology_rebuilds > before else step
        if ago == 0:
            rebuilds += 1
            cxx.set_atoms(py._lists, types)
            if step == 0:
                cxx.init_style()
                req = sorted(cxx.requests())
                assert req == [(0, 1, py.short_range_cutoff), (1, 0, py.long_range_cutoff)]
        print("case %s step %d ago %d" % (name, step, ago), flush=True)
        got = cxx.compute(py._lists.rows_positions(np.asarray(atoms.x)), ago, eflag_atom=True, vflag_atom=True)
        assert got["energy"] == want["energy"]
        for k in ("forces", "virial", "eatom", "vatom"):
            assert np.array_equal(got[k], want[k]), (name, step, k)
        x = np.asarray(atoms.x)
        ref = orc.evaluate(z, *support.build_graphs(x, box), charge=q, multiplicity=m)
        support.record_margin(got["energy"], got["forces"], got["virial"], ref, "C++ style step %d" % step)
        assert abs(got["energy"] - ref["energy"]) <= 1e-10 * abs(ref["energy"])
        assert np.abs(got["forces"] - ref["forces"]).max() <= 1e-9
        assert np.abs(got["virial"] - ref["virial"]).max() <= 1e-9  # eV, absolute
        assert np.abs(got["eatom"] - ref["eatom"]).max() <= 1e-10 * max(1.0, np.abs(ref["eatom"]).max())
        assert np.abs(got["vatom"] - ref["vatom"]).max() <= 1e-9 * max(1.0, np.abs(ref["vatom"]).max())
    assert rebuilds == 2
    cxx.close()


def test_cxx_style_refusals_match_mirror():
    """(Q, M) refused against the composition, the comm cutoff and the rank
    count: the C++ style and the mirror stop with the same message; a charged
    periodic cell gets the same warning."""
    import lammps_style
    symbols, types, atoms, z, box = _setup("water3000", 0, 1)
    lists = None
    for args, kw, py_kw in (
            (["0", "2"], {}, {}),                                   # even electron count, even multiplicity
            (["0", "1"], {"comm_cutoff": 12.5}, {"comm_cutoff": 12.5}),
            (["0", "1"], {"nprocs": 2}, {"nprocs": 2})):
        py = PairSO3LRNativeMPI(device=0, **py_kw)
        py.settings([support.MODEL] + args)
        py.coeff(["*", "*"] + symbols, ntypes=len(symbols))
        cxx = lammps_style.CxxPairStyle(len(symbols), periodic=atoms.periodic, **kw)
        cxx.settings([support.MODEL] + args)
        cxx.coeff(["*", "*"] + symbols)
        if lists is None:
            from so3lrxlammps_amd import Lists
            lists = Lists(atoms.x, atoms.lo, atoms.hi, atoms.periodic)
        cxx.set_atoms(lists, types)
        with pytest.raises(LammpsError) as a:
            cxx.init_style()
        with pytest.raises(LammpsError) as b:
            py.init_style(atoms)
        print("refusal:", a.value, flush=True)
        assert str(a.value) == str(b.value)
        cxx.close()
    # 3,000 atoms of water minus one electron: an odd count, so an even multiplicity
    py = PairSO3LRNativeMPI(device=0)
    py.settings([support.MODEL, "1", "2"])
    py.coeff(["*", "*"] + symbols, ntypes=len(symbols))
    py.init_style(atoms)
    cxx = lammps_style.CxxPairStyle(len(symbols), periodic=atoms.periodic)
    cxx.settings([support.MODEL, "1", "2"])
    cxx.coeff(["*", "*"] + symbols)
    cxx.set_atoms(lists, types)
    cxx.init_style()
    assert cxx.warnings() == py.warnings and len(py.warnings) == 1
    cxx.close()
