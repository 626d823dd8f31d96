"""The thin LAMMPS styles of lammps/ against their Python mirrors, on the CPU.

lammps/pair_so3lr_hip.cpp (so3lr/native/mpi) and
lammps/turbo/pair_so3lr_turbo_hip.cpp (so3lr/turbo) are compiled against the
LAMMPS API subset of tests/lammps_api/ (a missing include or a call the
subset does not declare fails the build), and the native style is run
through tests/lammps_api/pair_driver.cpp for every command that needs no
GPU.  Its messages must be the ones so3lrxlammps_amd/pair_style.py raises for
the same input, and every message either C++ style can raise must be one its
mirror raises too (apart from the LAMMPS-side conditions listed below, which
the stand-in cannot produce), so the tested mirror and the shipped C++
cannot drift apart.
"""
import ast
import os
import re
import subprocess

import numpy as np
import pytest

import support
from so3lrxlammps_amd.pair_style import Atoms, LammpsError, PairSO3LRNativeMPI

REPO = support.REPO
NATIVE_CPP = os.path.join(REPO, "lammps", "pair_so3lr_hip.cpp")
TURBO_CPP = os.path.join(REPO, "lammps", "turbo", "pair_so3lr_turbo_hip.cpp")
SOURCES = ["lammps/pair_so3lr_hip.h", "lammps/pair_so3lr_hip.cpp", "lammps/so3lrhipplugin.cpp",
           "lammps/turbo/pair_so3lr_turbo_hip.h", "lammps/turbo/pair_so3lr_turbo_hip.cpp",
           "lammps/turbo/so3lrturbohipplugin.cpp", "lammps/SO3LR_HIP.cmake", "lammps/Makefile"]

# messages of the C++ styles that only a real LAMMPS can trigger: list IDs
# other than 0 and 1, compute before the lists exist, and atom tags that
# LAMMPS itself keeps unique and owned
LAMMPS_SIDE = [
    "Unexpected so3lr/native/mpi neighbor-list ID",
    "SO3LR MPI neighbor lists were not initialized",
    "duplicate locally owned atom tag",
    "ghost tag has no owner",
    "periodic image element differs from owner",
    "Unexpected so3lr/turbo neighbor-list ID",
    "SO3LR turbo neighbor lists were not initialized",
]


@pytest.fixture(scope="module")
def built():
    """The driver and the syntax checks (idempotent; make decides)."""
    subprocess.run(["make", "-C", os.path.join(REPO, "tests", "lammps_api")], check=True,
                   stdout=subprocess.DEVNULL)
    import lammps_style
    return lammps_style


def test_sources_exist_and_integration_points_at_them():
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    for rel in SOURCES:
        assert os.path.exists(os.path.join(REPO, rel)), rel
        assert rel in text, "INTEGRATION.md does not name %s" % rel
    # the styles live in files now, not as code blocks of the document
    assert "PairSO3LRHip::compute" not in text


def test_styles_compile_against_the_api_subset(built):
    assert os.path.exists(built.DRIVER)
    assert os.path.exists(built.SYNTAX_OK)  # plugins and the turbo style compiled


def _cxx_messages(path):
    """String literals (adjacent ones joined) of every error->...() call."""
    src = open(path).read()
    msgs = []
    for m in re.finditer(r"error->(?:all|one|universe_all|universe_one|warning)\(FLERR,(.*?)\);", src, re.S):
        lits = re.findall(r'"((?:[^"\\]|\\.)*)"', m.group(1))
        if lits:
            msgs.append("".join(lits))
    return msgs


def _python_messages(path):
    """Every string constant of a Python module (joined literals included)."""
    tree = ast.parse(open(path).read())
    return [n.value for n in ast.walk(tree) if isinstance(n, ast.Constant) and isinstance(n.value, str)]


def _as_pattern(msg):
    """A C++ {}-format message as a regular expression over Python's %-format."""
    parts = re.split(r"\{[^}]*\}", msg)
    return ".*".join(re.escape(p) for p in parts)


@pytest.mark.parametrize("cpp,mirror", [
    (NATIVE_CPP, os.path.join(REPO, "so3lrxlammps_amd", "pair_style.py")),
    (TURBO_CPP, os.path.join(REPO, "so3lrxlammps_amd", "turbo.py")),
])
def test_every_cxx_message_is_raised_by_the_mirror(cpp, mirror):
    py = [re.sub(r"%[-0-9.]*[sdgf]", "X", s) for s in _python_messages(mirror)]
    checked = 0
    for msg in _cxx_messages(cpp):
        if msg in ("{}",) or any(side in msg for side in LAMMPS_SIDE):
            continue
        pat = re.compile(_as_pattern(msg).replace(r"\%", "%"))
        fixed = max(re.split(r"\{[^}]*\}", msg), key=len)
        assert any(pat.fullmatch(s) or (fixed and fixed in s) for s in py), (
            "%s raises %r, which %s never does" % (os.path.basename(cpp), msg, os.path.basename(mirror)))
        checked += 1
    assert checked >= 6


def _both(built, action_cxx, action_py):
    """Run one command on the C++ style and on the mirror; both must refuse
    it with the same message."""
    with pytest.raises(LammpsError) as a:
        action_cxx()
    with pytest.raises(LammpsError) as b:
        action_py()
    assert str(a.value) == str(b.value)
    return str(a.value)


def test_settings_argument_count_matches_mirror(built):
    for args in ([], [support.MODEL, "0", "1", "extra"]):
        msg = _both(built, lambda: built.CxxPairStyle(2).settings(args), lambda: PairSO3LRNativeMPI().settings(args))
        assert msg.startswith("Illegal pair_style so3lr/native/mpi command")


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU driver is present")
def test_model_load_failure_matches_mirror(built):
    msg = _both(built, lambda: built.CxxPairStyle(2).settings([support.MODEL, "0", "1"]),
                lambda: PairSO3LRNativeMPI().settings([support.MODEL, "0", "1"]))
    assert msg.startswith("Cannot initialize MPI-native SO3LR model: ")


def test_coeff_rules_match_mirror(built):
    for args in (["*", "*", "O"], ["1", "*", "O", "H"], ["*", "2", "O", "H"], ["*", "*", "O", "Xx"]):
        _both(built, lambda: built.CxxPairStyle(2).coeff(args), lambda: PairSO3LRNativeMPI().coeff(args, ntypes=2))
    # accepted: symbols in any case and atomic numbers
    built.CxxPairStyle(4).coeff(["*", "*", "o", "1", "NA", "17"])


def test_init_one_after_a_refused_coeff(built):
    cxx = built.CxxPairStyle(2)
    with pytest.raises(LammpsError):
        cxx.coeff(["*", "*", "O", "Xx"])
    msg = _both(built, lambda: cxx.init_one(1, 1), lambda: PairSO3LRNativeMPI().init_one(1, 1))
    assert msg == "All so3lr/native/mpi coefficients are not set"


def test_init_style_order_matches_mirror(built):
    lists_atoms = Atoms(x=np.zeros((1, 3)), types=np.array([1]), newton_pair=False)
    _both(built, lambda: built.CxxPairStyle(1, newton_pair=False).init_style(),
          lambda: PairSO3LRNativeMPI().init_style(lists_atoms))
    lists_atoms.newton_pair = True
    msg = _both(built, lambda: built.CxxPairStyle(1).init_style(), lambda: PairSO3LRNativeMPI().init_style(lists_atoms))
    assert msg == "Pair style so3lr/native/mpi model was not initialized"
