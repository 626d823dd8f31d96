"""The pair-style mirror (so3lrxlammps_amd/pair_style.py) on the CPU: the
command checks and messages of PairSO3LRNativeMPI that need no device
(plugins/lammps/pair_so3lr_native_mpi.cpp:1097-1192), and the model-load
failure as LAMMPS would report it when no GPU is present."""
import os

import numpy as np
import pytest

import support
from so3lrxlammps_amd.pair_style import Atoms, LammpsError, PairSO3LRNativeMPI


def test_settings_argument_count():
    p = PairSO3LRNativeMPI()
    for args in ([], [support.MODEL, "0", "1", "extra"]):
        with pytest.raises(LammpsError, match="Illegal pair_style so3lr/native/mpi command"):
            p.settings(args)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU driver is present")
def test_settings_reports_the_model_load_failure():
    with pytest.raises(LammpsError, match="Cannot initialize MPI-native SO3LR model"):
        PairSO3LRNativeMPI().settings([support.MODEL, "0", "1"])


def test_coeff_rules():
    p = PairSO3LRNativeMPI()
    for args in (["*", "*", "O"], ["1", "*", "O", "H"], ["*", "2", "O", "H"]):
        with pytest.raises(LammpsError, match=r"Pair coeff for so3lr/native/mpi must be '\* \* E1 ... Entypes'"):
            p.coeff(args, ntypes=2)
    with pytest.raises(LammpsError, match="Unknown SO3LR element 'Xx'"):
        p.coeff(["*", "*", "O", "Xx"], ntypes=2)
    # symbols in any case and atomic numbers, as so3lr_element_map.h reads them
    p.coeff(["*", "*", "o", "1", "NA", "17"], ntypes=4)
    assert list(p.type_to_z) == [0, 8, 1, 11, 17]


def test_init_one_and_init_style_order():
    p = PairSO3LRNativeMPI()
    with pytest.raises(LammpsError, match="All so3lr/native/mpi coefficients are not set"):
        p.init_one(1, 1)
    atoms = Atoms(x=np.zeros((1, 3)), types=np.array([1]), newton_pair=False)
    with pytest.raises(LammpsError, match="requires newton pair on"):
        p.init_style(atoms)
    atoms.newton_pair = True
    with pytest.raises(LammpsError, match="model was not initialized"):
        p.init_style(atoms)
