"""Host-side mirror of `pair_style so3lr/turbo` over libso3lr_turbo.so.

Same commands, argument meaning and error behaviour as PairSO3LRTurbo
(source/so3lr-lammps-native/plugins/lammps/pair_so3lr_turbo.{h,cpp}).  Every
MPI rank is a one-rank partition with one non-periodic image; rank 0 (the
coordinator) evaluates all images on its GPU through include/so3lr_turbo.h:

    pair = PairSO3LRTurbo()                    # MPI_COMM_WORLD is the universe
    pair.settings(["so3lr.so3lr", "-1", "1"])  # pair_style so3lr/turbo MODEL [Q [M]]
    pair.coeff(["*", "*", "C", "H", "O"], ntypes=3)
    pair.init_style(atoms)                     # collective (Q, M) check
    result = pair.compute(atoms)               # collective

Workers never load a model and make no HIP call.  Ranks that have not
imported torch bind libso3lr_hip to the system HIP runtime; MPICH's libmpi is
loaded after it, so MPICH's older copies of the GCC runtime libraries never
shadow the ones libso3lr_hip was built against.
"""
import ctypes
import os
import shutil
import sys

import numpy as np

from . import _lib
from .pair_style import LammpsError

TURBO_LIB = os.path.join(_lib.HERE, "libso3lr_turbo.so")

# every symbol include/so3lr_turbo.h declares
TURBO_SYMBOLS = ["so3lr_turbo_mpi_world", "so3lr_turbo_mpi_finalize", "so3lr_turbo_check_images",
                 "so3lr_turbo_create", "so3lr_turbo_destroy", "so3lr_turbo_last_error", "so3lr_turbo_info",
                 "so3lr_turbo_evaluate", "so3lr_turbo_stats"]

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_D = ctypes.c_double
_I = ctypes.c_int

_turbo = None
_hip_direct = None


def mpi_library():
    """MPICH's libmpi.so.12: $SO3LR_MPI_LIB, else beside the mpiexec on PATH,
    else the image's /opt/conda installation."""
    env = os.environ.get("SO3LR_MPI_LIB")
    if env:
        return env
    cands = []
    exe = shutil.which("mpiexec")
    if exe:
        cands.append(os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(exe))), "lib", "libmpi.so.12"))
    cands.append("/opt/conda/lib/libmpi.so.12")
    for c in cands:
        if os.path.exists(c):
            return c
    raise ImportError("MPICH's libmpi.so.12 not found; set SO3LR_MPI_LIB")


def hip_lib():
    """libso3lr_hip, bound to torch's HIP runtime when torch is loaded and to
    the system runtime otherwise (no torch import here)."""
    global _hip_direct
    if "torch" in sys.modules:
        return _lib.hip()
    if _hip_direct is None:
        lib = _lib._load(_lib.HIP_LIB, "libso3lr_hip")
        lib.so3lr_atomic_number.argtypes = [ctypes.c_char_p]
        lib.so3lr_check_system.argtypes = [_I64, _P, _D, _D]
        lib.so3lr_last_error.argtypes = [_P]
        lib.so3lr_last_error.restype = ctypes.c_char_p
        _hip_direct = lib
    return _hip_direct


def turbo():
    global _turbo
    if _turbo is None:
        hip_lib()
        _lib.emu()
        ctypes.CDLL(mpi_library(), mode=ctypes.RTLD_GLOBAL)
        lib = _lib._load(TURBO_LIB, "libso3lr_turbo")
        lib.so3lr_turbo_mpi_world.argtypes = [_P, _P, _P]
        lib.so3lr_turbo_check_images.argtypes = [_I64, _I64, _P, _D, _D]
        lib.so3lr_turbo_create.argtypes = [_I64, _I, ctypes.c_char_p, _I, ctypes.POINTER(_P)]
        lib.so3lr_turbo_destroy.argtypes = [_P]
        lib.so3lr_turbo_destroy.restype = None
        lib.so3lr_turbo_last_error.argtypes = [_P]
        lib.so3lr_turbo_last_error.restype = ctypes.c_char_p
        lib.so3lr_turbo_info.argtypes = [_P, _P, _P, _P, _P, _P]
        lib.so3lr_turbo_evaluate.argtypes = [_P, _I64, _P, _P, _D, _D, _I, _I, _I64, _P, _P, _P, _I64, _P, _P, _P,
                                             _P, _P, _P, _P, _P]
        lib.so3lr_turbo_stats.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P]
        _turbo = lib
    return _turbo


def mpi_world():
    """(Fortran handle of MPI_COMM_WORLD, rank, size), initialising MPI."""
    lib = turbo()
    comm, rank, size = _I64(), _I(), _I()
    rc = lib.so3lr_turbo_mpi_world(ctypes.byref(comm), ctypes.byref(rank), ctypes.byref(size))
    if rc != _lib.OK:
        raise _lib.SO3LRError(rc, lib.so3lr_turbo_last_error(None).decode())
    return comm.value, rank.value, size.value


def mpi_finalize():
    turbo().so3lr_turbo_mpi_finalize()


def check_images(comm, z, charge, multiplicity):
    """Collective (Q, M) check; raises the same SO3LRError on every rank."""
    lib = turbo()
    z = np.ascontiguousarray(z, dtype=np.int32)
    rc = lib.so3lr_turbo_check_images(comm, len(z), _lib.ptr(z), float(charge), float(multiplicity))
    if rc != _lib.OK:
        raise _lib.SO3LRError(rc, lib.so3lr_turbo_last_error(None).decode())


class Broker:
    """One so3lr_turbo broker (collective create)."""

    def __init__(self, comm, model_path, coordinator=0, device=0):
        lib = turbo()
        h = _P()
        rc = lib.so3lr_turbo_create(comm, int(coordinator), model_path.encode(), int(device), ctypes.byref(h))
        if rc != _lib.OK:
            raise _lib.SO3LRError(rc, lib.so3lr_turbo_last_error(None).decode())
        self._h = h
        self._lib = lib
        rank, size, coord = _I(), _I(), _I()
        sr, lr = _D(), _D()
        lib.so3lr_turbo_info(h, ctypes.byref(rank), ctypes.byref(size), ctypes.byref(coord), ctypes.byref(sr),
                             ctypes.byref(lr))
        self.rank, self.size, self.coordinator = rank.value, size.value, coord.value
        self.sr_cutoff, self.lr_cutoff = sr.value, lr.value

    def close(self):
        if getattr(self, "_h", None):
            self._lib.so3lr_turbo_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def evaluate(self, z, x, charge, multiplicity, lists, lists_changed):
        """This image's (energy, forces, eatom, charges, hirshfeld); collective."""
        z = np.ascontiguousarray(z, dtype=np.int32)
        x = np.ascontiguousarray(x, dtype=np.float64)
        n = len(z)
        (si, so, sn), (li, lo_, ln) = lists.lists
        f = np.zeros((n, 3))
        ea, q, h = np.zeros(n), np.zeros(n), np.zeros(n)
        e = _D()
        rc = self._lib.so3lr_turbo_evaluate(
            self._h, n, _lib.ptr(z), _lib.ptr(x), float(charge), float(multiplicity), 1 if lists_changed else 0,
            _lib.LIST_FULL if lists.sr_full else _lib.LIST_HALF, len(si), _lib.ptr(si), _lib.ptr(so),
            _lib.ptr(sn), len(li), _lib.ptr(li), _lib.ptr(lo_), _lib.ptr(ln), _lib.ptr(f), _lib.ptr(ea),
            _lib.ptr(q), _lib.ptr(h), ctypes.byref(e))
        if rc != _lib.OK:
            raise _lib.SO3LRError(rc, self._lib.so3lr_turbo_last_error(self._h).decode())
        return e.value, f, ea, q, h

    def raw_evaluate(self, *args):
        """so3lr_turbo_evaluate with caller-built arguments (returns the status)."""
        return self._lib.so3lr_turbo_evaluate(self._h, *args)

    def last_error(self):
        return self._lib.so3lr_turbo_last_error(self._h).decode()

    def stats(self):
        packed, images, gathered = _I64(), _I64(), _I()
        g, ev, sc, tot = _D(), _D(), _D(), _D()
        self._lib.so3lr_turbo_stats(self._h, ctypes.byref(packed), ctypes.byref(images), ctypes.byref(gathered),
                                    ctypes.byref(g), ctypes.byref(ev), ctypes.byref(sc), ctypes.byref(tot))
        return {"packed_atoms": packed.value, "images": images.value, "lists_gathered": gathered.value,
                "gather_ms": g.value, "evaluate_ms": ev.value, "scatter_ms": sc.value, "total_ms": tot.value}


class PairSO3LRTurbo:
    # constructor flags of the reference (pair_so3lr_turbo.cpp:77-89)
    manybody_flag = 1
    one_coeff = 1
    restartinfo = 0
    single_enable = 0

    def __init__(self, comm=None, device=0, skin=1.0, nprocs=1):
        if comm is None:
            comm, _, _ = mpi_world()
        self.comm = comm
        self.device = device
        self.skin = skin
        self.nprocs = nprocs  # ranks in this image's partition
        self.broker = None
        self.type_to_z = None
        self.total_charge = 0.0
        self.multiplicity = 1.0
        self._lists = None
        self._x_at_build = None
        self.evaluation_count = 0

    # -- pair_style so3lr/turbo MODEL [charge [multiplicity]] (:112-154)
    def settings(self, args):
        if len(args) < 1 or len(args) > 3:
            raise LammpsError("Illegal pair_style so3lr/turbo command: expected "
                              "'pair_style so3lr/turbo MODEL [charge [multiplicity]]'")
        self.model_path = args[0]
        self.total_charge = float(args[1]) if len(args) > 1 else 0.0
        self.multiplicity = float(args[2]) if len(args) > 2 else 1.0
        try:
            self.broker = Broker(self.comm, self.model_path, 0, self.device)
        except _lib.SO3LRError as exc:
            raise LammpsError(str(exc)) from exc
        self.short_range_cutoff = self.broker.sr_cutoff
        self.long_range_cutoff = self.broker.lr_cutoff

    # -- pair_coeff * * E1 ... Entypes (:156-173)
    def coeff(self, args, ntypes):
        if len(args) != ntypes + 2 or args[0] != "*" or args[1] != "*":
            raise LammpsError("Pair coeff for so3lr/turbo must be '* * E1 ... Entypes'")
        lib = hip_lib()
        t2z = [0] * (ntypes + 1)
        for t in range(1, ntypes + 1):
            z = lib.so3lr_atomic_number(args[t + 1].encode())
            if z == 0:
                raise LammpsError("Unknown SO3LR element '%s'" % args[t + 1])
            t2z[t] = z
        self.type_to_z = np.array(t2z, dtype=np.int32)

    def init_one(self, i, j):
        if self.type_to_z is None:
            raise LammpsError("All so3lr/turbo coefficients are not set")
        return self.long_range_cutoff

    # -- init_style (:182-223)
    def init_style(self, atoms):
        if self.nprocs != 1:
            raise LammpsError("so3lr/turbo requires one MPI rank per LAMMPS partition")
        if self.broker is None:
            raise LammpsError("SO3LR turbo broker was not initialized")
        if self.broker.size < 2:
            raise LammpsError("so3lr/turbo requires multiple one-rank partitions")
        if any(atoms.periodic):
            raise LammpsError("so3lr/turbo requires non-periodic boundaries")
        if not atoms.newton_pair:
            raise LammpsError("Pair style so3lr/turbo requires newton pair on")
        if self.type_to_z is None:
            raise LammpsError("Pair style so3lr/turbo coefficients are missing")
        z = self.type_to_z[np.asarray(atoms.types)]
        try:
            check_images(self.comm, z, self.total_charge, self.multiplicity)
        except _lib.SO3LRError as exc:
            raise LammpsError(str(exc)) from exc
        self._lists = None

    def _neighbor(self, atoms):
        """Rebuild the lists when an atom moved more than half the skin;
        returns whether they changed (LAMMPS neighbor->ago == 0)."""
        x = np.asarray(atoms.x, dtype=np.float64)
        if self._lists is not None:
            disp = np.sqrt(((x - self._x_at_build) ** 2).sum(1)).max()
            if disp <= 0.5 * self.skin:
                return False
        lo, hi = np.asarray(atoms.lo, float), np.asarray(atoms.hi, float)
        self._lists = _lib.Lists(x, lo, hi, (0, 0, 0), self.short_range_cutoff, self.long_range_cutoff,
                                 self.skin, self.long_range_cutoff + self.skin, sr_full=True)
        self._x_at_build = x.copy()
        return True

    # -- compute(eflag, vflag) (:235-319)
    def compute(self, atoms, eflag=True, vflag=True, eflag_atom=False, vflag_atom=False):
        if vflag_atom:
            raise LammpsError("so3lr/turbo does not provide per-atom virial")
        changed = self._neighbor(atoms)
        x = np.asarray(atoms.x, dtype=np.float64)
        z = self.type_to_z[np.asarray(atoms.types)]
        try:
            e, f, ea, q, h = self.broker.evaluate(z, x, self.total_charge, self.multiplicity, self._lists,
                                                  changed)
        except _lib.SO3LRError as exc:
            raise LammpsError("SO3LR turbo LAMMPS evaluation failed: %s" % exc) from exc
        self.evaluation_count += 1
        virial = None
        if vflag:
            # virial_fdotr_compute over the owned rows (a turbo image has no ghosts)
            virial = np.array([(f[:, 0] * x[:, 0]).sum(), (f[:, 1] * x[:, 1]).sum(), (f[:, 2] * x[:, 2]).sum(),
                               (f[:, 1] * x[:, 0]).sum(), (f[:, 2] * x[:, 0]).sum(), (f[:, 2] * x[:, 1]).sum()])
        return {"energy": e if eflag else None, "forces": f, "eatom": ea if eflag_atom else None,
                "virial": virial, "charges": q, "hirshfeld": h, "lists_changed": changed}
