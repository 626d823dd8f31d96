"""MI355X-native SO3LR force evaluator (pair_style so3lr/native/mpi drop-in).

The compute path is libso3lr_hip.so (hand-written gfx950 HIP, fp64) behind the
C ABI in include/so3lr_hip.h; this package holds its sources (csrc/), ctypes
bindings (_lib) and a host-side mirror of the LAMMPS pair style (pair_style).
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))
MODEL_PATH = os.path.join(os.path.dirname(HERE), "models", "so3lr.so3lr")

from ._lib import Context, Lists, SO3LRError  # noqa: E402,F401
from .pair_style import Atoms, LammpsError, PairSO3LRNativeMPI  # noqa: E402,F401
