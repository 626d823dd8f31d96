"""ctypes binding of tests/lammps_api/_build/libpair_driver.so: the C++ pair
style of lammps/pair_so3lr_hip.cpp (so3lr/native/mpi on libso3lr_hip),
compiled against the LAMMPS API subset of tests/lammps_api/, driven the way
LAMMPS drives a pair style.  Test infrastructure only.

    cxx = CxxPairStyle(ntypes=2, periodic=(1, 1, 1))
    cxx.settings([model, "0", "1"]); cxx.coeff(["*", "*", "O", "H"])
    cxx.set_atoms(lists, types)           # at a reneighbor: rows, tags, types, lists
    cxx.init_style()
    out = cxx.compute(rows_positions, ago=0, eflag_atom=True, vflag_atom=True)
"""
import ctypes
import os

import numpy as np

from so3lrxlammps_amd.pair_style import LammpsError

HERE = os.path.dirname(os.path.abspath(__file__))
DRIVER = os.path.join(HERE, "lammps_api", "_build", "libpair_driver.so")
SYNTAX_OK = os.path.join(HERE, "lammps_api", "_build", "syntax.ok")

_P = ctypes.c_void_p
_lib = None


def lib():
    global _lib
    if _lib is None:
        from so3lrxlammps_amd import _lib as hip
        hip.hip()  # libso3lr_hip first (bound to torch's HIP runtime when torch is loaded)
        if not os.path.exists(DRIVER):
            raise ImportError("%s not built (make -C tests/lammps_api, or __graft_entry__.build())" % DRIVER)
        d = ctypes.CDLL(DRIVER)
        d.pd_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double, _P]
        d.pd_create.restype = _P
        d.pd_destroy.argtypes = [_P]
        d.pd_destroy.restype = None
        d.pd_message.argtypes = [_P]
        d.pd_message.restype = ctypes.c_char_p
        d.pd_warnings.argtypes = [_P]
        d.pd_warning.argtypes = [_P, ctypes.c_int]
        d.pd_warning.restype = ctypes.c_char_p
        d.pd_log.restype = ctypes.c_char_p
        d.pd_settings.argtypes = [_P, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
        d.pd_coeff.argtypes = [_P, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
        d.pd_init_one.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
        d.pd_set_atoms.argtypes = [_P, ctypes.c_int, ctypes.c_int, _P, _P]
        d.pd_positions.argtypes = [_P, _P]
        d.pd_init_style.argtypes = [_P]
        d.pd_request.argtypes = [_P, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                 ctypes.POINTER(ctypes.c_double)]
        d.pd_set_list.argtypes = [_P, ctypes.c_int, ctypes.c_int, _P, _P, _P]
        d.pd_compute.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, _P, _P, _P, _P]
        _lib = d
    return _lib


def _argv(args):
    arr = (ctypes.c_char_p * max(1, len(args)))(*[a.encode() for a in args])
    return len(args), arr


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


class CxxPairStyle:
    """One PairSO3LRHip inside the driver's LAMMPS stand-in objects."""

    def __init__(self, ntypes, newton_pair=True, nprocs=1, comm_cutoff=13.0, skin=1.0, periodic=(0, 0, 0)):
        self._d = lib()
        per = np.ascontiguousarray(periodic, dtype=np.int32)
        self._h = self._d.pd_create(int(ntypes), 1 if newton_pair else 0, int(nprocs), float(comm_cutoff),
                                    float(skin), _ptr(per))
        self.n = 0

    def close(self):
        if getattr(self, "_h", None):
            self._d.pd_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def _check(self, rc):
        if rc != 0:
            raise LammpsError(self._d.pd_message(self._h).decode())

    def settings(self, args):
        self._check(self._d.pd_settings(self._h, *_argv(args)))

    def coeff(self, args):
        self._check(self._d.pd_coeff(self._h, *_argv(args)))

    def init_one(self, i, j):
        cut = ctypes.c_double()
        self._check(self._d.pd_init_one(self._h, i, j, ctypes.byref(cut)))
        return cut.value

    def set_atoms(self, lists, types_owned):
        """What LAMMPS holds after a reneighbor: owned rows then ghost rows
        (tag = owner + 1, the owner's type) and both lists."""
        owner = np.asarray(lists.owner, dtype=np.int32)
        self.n = lists.n
        self._tag = np.ascontiguousarray(owner + 1, dtype=np.int32)
        self._type = np.ascontiguousarray(np.asarray(types_owned, dtype=np.int32)[owner])
        self._d.pd_set_atoms(self._h, lists.n, lists.rows - lists.n, _ptr(self._tag), _ptr(self._type))
        self._lists = []
        for which, (il, off, nb) in enumerate(lists.lists):
            il = np.ascontiguousarray(il, dtype=np.int32)
            off = np.ascontiguousarray(off, dtype=np.int64)
            nb = np.ascontiguousarray(nb, dtype=np.int32)
            self._lists.append((il, off, nb))
            self._d.pd_set_list(self._h, which, len(il), _ptr(il), _ptr(off), _ptr(nb))

    def init_style(self):
        self._check(self._d.pd_init_style(self._h))

    def requests(self):
        out, k = [], 0
        while True:
            i, f, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
            if self._d.pd_request(self._h, k, ctypes.byref(i), ctypes.byref(f), ctypes.byref(c)) != 0:
                return out
            out.append((i.value, f.value, c.value))
            k += 1

    def warnings(self):
        return [self._d.pd_warning(self._h, k).decode() for k in range(self._d.pd_warnings(self._h))]

    def compute(self, x_rows, ago, eflag_atom=False, vflag_atom=False):
        x_rows = np.ascontiguousarray(x_rows, dtype=np.float64)
        self._d.pd_positions(self._h, _ptr(x_rows))
        n = self.n
        f = np.zeros((n, 3))
        ea = np.zeros(n)
        va = np.zeros((n, 6))
        e = ctypes.c_double()
        w = np.zeros(6)
        eflag = 1 | (2 if eflag_atom else 0)
        vflag = 1 | (4 if vflag_atom else 0)
        self._check(self._d.pd_compute(self._h, int(ago), eflag, vflag, _ptr(f), _ptr(ea), _ptr(va),
                                       ctypes.byref(e), _ptr(w)))
        return {"energy": e.value, "forces": f, "eatom": ea if eflag_atom else None, "virial": w,
                "vatom": va if vflag_atom else None}
