"""ctypes bindings of libso3lr_hip.so (include/so3lr_hip.h) and of the LAMMPS
stand-in libso3lr_lammps_emu.so (include/so3lr_lammps_emu.h).

The product path is the HIP library; there is no CPU fallback.  Importing the
bindings without a built library raises immediately.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(HERE, "libso3lr_hip.so")
EMU_LIB = os.path.join(HERE, "libso3lr_lammps_emu.so")

OK, ERR_ARGUMENT, ERR_MODEL, ERR_SYSTEM, ERR_TOPOLOGY, ERR_DEVICE, ERR_STATE, ERR_UNSUPPORTED = range(8)
ENERGY, EATOM, VIRIAL, VATOM = 1, 2, 4, 8
LIST_FULL, LIST_HALF = 0, 1

# every symbol include/so3lr_hip.h declares
HIP_SYMBOLS = ["so3lr_create", "so3lr_destroy", "so3lr_last_error", "so3lr_cutoff",
               "so3lr_atomic_number", "so3lr_check_system", "so3lr_set_system", "so3lr_set_images",
               "so3lr_set_topology", "so3lr_compute", "so3lr_compute_device", "so3lr_compute_device_noalloc",
               "so3lr_reneighbor_device", "so3lr_set_box",
               "so3lr_set_stream", "so3lr_last_terms", "so3lr_last_vatom", "so3lr_graph_stats",
               "so3lr_kernel_timing", "so3lr_kernel_timing_read", "so3lr_device_bytes"]
EMU_SYMBOLS = ["so3lr_emu_build", "so3lr_emu_error", "so3lr_emu_free", "so3lr_emu_rows",
               "so3lr_emu_owner", "so3lr_emu_image", "so3lr_emu_inum", "so3lr_emu_ilist",
               "so3lr_emu_offsets", "so3lr_emu_neigh"]

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_D = ctypes.c_double


class SO3LRError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


def _load(path, what):
    if not os.path.exists(path):
        raise ImportError("%s not built: %s missing (run __graft_entry__.build())" % (what, path))
    return ctypes.CDLL(path)


_hip = None
_emu = None


def _bind_one_hip_runtime():
    """Load torch's HIP runtime first when torch is installed.

    torch ships its own libamdhip64 (SONAME libamdhip64.so.7) and reaches it by
    file name; libso3lr_hip.so needs libamdhip64.so.7.  Loaded after torch, the
    library binds to torch's already-loaded runtime; loaded before it, torch
    would bring a second HIP runtime into the process and fail to initialise.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def hip():
    global _hip
    if _hip is None:
        _bind_one_hip_runtime()
        lib = _load(HIP_LIB, "libso3lr_hip")
        lib.so3lr_create.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_P)]
        lib.so3lr_destroy.argtypes = [_P]
        lib.so3lr_destroy.restype = None
        lib.so3lr_last_error.argtypes = [_P]
        lib.so3lr_last_error.restype = ctypes.c_char_p
        lib.so3lr_cutoff.argtypes = [_P, ctypes.c_int]
        lib.so3lr_cutoff.restype = _D
        lib.so3lr_atomic_number.argtypes = [ctypes.c_char_p]
        lib.so3lr_check_system.argtypes = [_I64, _P, _D, _D]
        lib.so3lr_set_system.argtypes = [_P, _I64, _P, _D, _D]
        lib.so3lr_set_images.argtypes = [_P, _I64, _P, _I64, _P, _P, _P]
        lib.so3lr_set_topology.argtypes = [_P, _I64, _P, ctypes.c_int, _I64, _P, _P, _P, _I64, _P, _P, _P]
        lib.so3lr_compute.argtypes = [_P, _P, ctypes.c_int, _P, _P, _P, _P]
        lib.so3lr_compute_device.argtypes = [_P, _P, ctypes.c_int, _P, _P, _P, _P]
        lib.so3lr_compute_device_noalloc.argtypes = [_P, _P, ctypes.c_int, _P, _P, _P, _P]
        lib.so3lr_set_stream.argtypes = [_P, _P]
        lib.so3lr_reneighbor_device.argtypes = [_P, _P, _P, _P, _P, _D]
        lib.so3lr_set_box.argtypes = [_P, _P, _P]
        lib.so3lr_last_terms.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P]
        lib.so3lr_last_vatom.argtypes = [_P, _P, ctypes.c_int]
        lib.so3lr_graph_stats.argtypes = [_P, _P, _P, _P]
        lib.so3lr_kernel_timing.argtypes = [_P, ctypes.c_int]
        lib.so3lr_kernel_timing_read.argtypes = [_P, ctypes.c_char_p, _P, _P, _P]
        lib.so3lr_device_bytes.argtypes = [_P]
        lib.so3lr_device_bytes.restype = _I64
        _hip = lib
    return _hip


def emu():
    global _emu
    if _emu is None:
        lib = _load(EMU_LIB, "libso3lr_lammps_emu")
        lib.so3lr_emu_build.argtypes = [_I64, _P, _P, _P, _P, _D, _D, _D, _D, ctypes.c_int, ctypes.POINTER(_P)]
        lib.so3lr_emu_error.restype = ctypes.c_char_p
        lib.so3lr_emu_free.argtypes = [_P]
        lib.so3lr_emu_free.restype = None
        lib.so3lr_emu_rows.argtypes = [_P]
        lib.so3lr_emu_rows.restype = _I64
        for name in ("so3lr_emu_owner", "so3lr_emu_image"):
            getattr(lib, name).argtypes = [_P]
            getattr(lib, name).restype = ctypes.POINTER(ctypes.c_int32)
        lib.so3lr_emu_inum.argtypes = [_P, ctypes.c_int]
        lib.so3lr_emu_inum.restype = _I64
        for name, t in (("so3lr_emu_ilist", ctypes.c_int32), ("so3lr_emu_offsets", ctypes.c_int64),
                        ("so3lr_emu_neigh", ctypes.c_int32)):
            getattr(lib, name).argtypes = [_P, ctypes.c_int]
            getattr(lib, name).restype = ctypes.POINTER(t)
        _emu = lib
    return _emu


def ptr(a):
    """Data pointer of a numpy array or a torch tensor (None stays None)."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return ctypes.c_void_p(a.data_ptr())
    return ctypes.c_void_p(a.ctypes.data)


def device_f64(t, count, what):
    """Check that `t` is a contiguous float64 tensor on a GPU holding exactly
    `count` values, and return its pointer.  The C ABI takes raw device
    pointers and cannot see sizes, so a float32 tensor, a strided view or a
    short buffer would become an out-of-bounds access on the device; the
    binding refuses them here with a ValueError instead."""
    if t is None:
        raise ValueError("%s: a device tensor is required" % what)
    if not getattr(t, "is_cuda", False):
        raise ValueError("%s must be a GPU tensor (got %s)" % (what, getattr(t, "device", type(t).__name__)))
    import torch
    if t.dtype != torch.float64:
        raise ValueError("%s must be float64 (got %s)" % (what, t.dtype))
    if not t.is_contiguous():
        raise ValueError("%s must be contiguous" % what)
    if t.numel() != count:
        raise ValueError("%s must hold %d values (got %d)" % (what, count, t.numel()))
    return ptr(t)


def _copy(p, count, dtype):
    if count == 0:
        return np.zeros(0, dtype=dtype)
    return np.ctypeslib.as_array(p, shape=(count,)).astype(dtype, copy=True)


class Lists:
    """LAMMPS-like rows and candidate lists for one reneighbor."""

    def __init__(self, x, lo, hi, periodic, sr_cut=4.5, lr_cut=12.0, skin=1.0, comm_cut=13.0,
                 sr_full=True):
        lib = emu()
        x = np.ascontiguousarray(x, dtype=np.float64)
        lo = np.ascontiguousarray(lo, dtype=np.float64)
        hi = np.ascontiguousarray(hi, dtype=np.float64)
        per = np.ascontiguousarray(periodic, dtype=np.int32)
        h = _P()
        rc = lib.so3lr_emu_build(len(x), ptr(x), ptr(lo), ptr(hi), ptr(per), sr_cut, lr_cut, skin,
                                 comm_cut, 1 if sr_full else 0, ctypes.byref(h))
        if rc != 0:
            raise ValueError("LAMMPS list emulation failed: " + lib.so3lr_emu_error().decode())
        try:
            self.n = len(x)
            self.rows = int(lib.so3lr_emu_rows(h))
            self.owner = _copy(lib.so3lr_emu_owner(h), self.rows, np.int32)
            self.image = _copy(lib.so3lr_emu_image(h), 3 * self.rows, np.int32).reshape(-1, 3)
            self.lists = []
            for which in (0, 1):
                inum = int(lib.so3lr_emu_inum(h, which))
                ilist = _copy(lib.so3lr_emu_ilist(h, which), inum, np.int32)
                off = _copy(lib.so3lr_emu_offsets(h, which), inum + 1, np.int64)
                neigh = _copy(lib.so3lr_emu_neigh(h, which), int(off[-1]), np.int32)
                self.lists.append((ilist, off, neigh))
        finally:
            lib.so3lr_emu_free(h)
        self.box = np.asarray(hi, float) - np.asarray(lo, float)
        self.sr_full = sr_full

    def rows_positions(self, x):
        """x_row = x_owner + image * box (LAMMPS forward communication)."""
        return x[self.owner] + self.image * self.box


class Context:
    """One so3lr_hip context (one LAMMPS rank on one GPU)."""

    def __init__(self, model_path, device=0):
        lib = hip()
        h = _P()
        rc = lib.so3lr_create(model_path.encode(), int(device), ctypes.byref(h))
        if rc != OK:
            raise SO3LRError(rc, lib.so3lr_last_error(None).decode())
        self._h = h
        self._lib = lib

    def close(self):
        if getattr(self, "_h", None):
            self._lib.so3lr_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def _check(self, rc):
        if rc != OK:
            raise SO3LRError(rc, self._lib.so3lr_last_error(self._h).decode())

    def cutoff(self, which):
        return self._lib.so3lr_cutoff(self._h, which)

    def set_system(self, z, charge=0.0, multiplicity=1.0):
        z = np.ascontiguousarray(z, dtype=np.int32)
        self._check(self._lib.so3lr_set_system(self._h, len(z), ptr(z), float(charge), float(multiplicity)))
        self.n = len(z)
        self.rows = None  # a new system needs a new topology

    def set_images(self, z, image_offsets, charges, multiplicities):
        z = np.ascontiguousarray(z, dtype=np.int32)
        off = np.ascontiguousarray(image_offsets, dtype=np.int64)
        q = np.ascontiguousarray(charges, dtype=np.float64)
        m = np.ascontiguousarray(multiplicities, dtype=np.float64)
        if not (len(off) == len(q) + 1 == len(m) + 1):
            raise ValueError("image_offsets needs one entry more than charges and multiplicities "
                             "(%d offsets, %d charges, %d multiplicities)" % (len(off), len(q), len(m)))
        self._check(self._lib.so3lr_set_images(self._h, len(z), ptr(z), len(q), ptr(off), ptr(q), ptr(m)))
        self.n = len(z)
        self.n_images = len(q)
        self.rows = None  # a new system needs a new topology

    def set_topology(self, lists):
        (si, so, sn), (li, lo_, ln) = lists.lists
        self._keep = (lists.owner, si, so, sn, li, lo_, ln)
        self._check(self._lib.so3lr_set_topology(
            self._h, lists.rows, ptr(lists.owner), LIST_FULL if lists.sr_full else LIST_HALF,
            len(si), ptr(si), ptr(so), ptr(sn), len(li), ptr(li), ptr(lo_), ptr(ln)))
        self.rows = lists.rows

    def compute(self, x_rows, eatom=True, out=None):
        """so3lr_compute on host arrays: (energy, forces, eatom, virial).
        `out` = (forces (n, 3), eatom (n,)) reuses the caller's arrays, as a
        pair style reuses its own from step to step."""
        x_rows = np.ascontiguousarray(x_rows, dtype=np.float64)
        if out is None:
            f = np.zeros((self.n, 3))
            ea = np.zeros(self.n)
        else:
            f, ea = out
            if f.shape != (self.n, 3) or ea.shape != (self.n,) or f.dtype != np.float64 or ea.dtype != np.float64 \
                    or not (f.flags.c_contiguous and ea.flags.c_contiguous):
                raise ValueError("out must be C-contiguous float64 arrays of shape (%d, 3) and (%d,)" % (self.n, self.n))
        e = ctypes.c_double()
        w = np.zeros(6)
        flags = ENERGY | VIRIAL | (EATOM if eatom else 0)
        self._check(self._lib.so3lr_compute(self._h, ptr(x_rows), flags, ptr(f), ptr(ea),
                                            ctypes.byref(e), ptr(w)))
        return e.value, f, ea, w

    def _rows(self):
        """Rows the positions must cover; refused like the library's own
        ERR_STATE when no topology follows the current system."""
        rows = getattr(self, "rows", None)
        if rows is None:
            raise SO3LRError(ERR_STATE, "SO3LR: compute called before set_topology")
        return rows

    def compute_device(self, x_rows_dev, f_dev, eatom_dev=None, stream=None):
        """Device tensors in (positions of every row: owned and ghost rows after
        set_topology, owned atoms after reneighbor_device), device forces out;
        returns (energy, virial)."""
        px = device_f64(x_rows_dev, 3 * self._rows(), "positions")
        pf = device_f64(f_dev, 3 * self.n, "forces")
        pe = None if eatom_dev is None else device_f64(eatom_dev, self.n, "per-atom energies")
        if stream is not None:
            self._check(self._lib.so3lr_set_stream(self._h, ctypes.c_void_p(stream)))
        e = ctypes.c_double()
        w = np.zeros(6)
        flags = ENERGY | VIRIAL | (EATOM if eatom_dev is not None else 0)
        self._check(self._lib.so3lr_compute_device(self._h, px, flags, pf, pe, ctypes.byref(e), ptr(w)))
        return e.value, w

    def compute_device_noalloc(self, x_rows_dev, f_dev, eatom_dev=None, stream=None):
        """As compute_device through so3lr_compute_device_noalloc: the work
        buffers are slices of the library's static device array."""
        px = device_f64(x_rows_dev, 3 * self._rows(), "positions")
        pf = device_f64(f_dev, 3 * self.n, "forces")
        pe = None if eatom_dev is None else device_f64(eatom_dev, self.n, "per-atom energies")
        if stream is not None:
            self._check(self._lib.so3lr_set_stream(self._h, ctypes.c_void_p(stream)))
        e = ctypes.c_double()
        w = np.zeros(6)
        flags = ENERGY | VIRIAL | (EATOM if eatom_dev is not None else 0)
        self._check(self._lib.so3lr_compute_device_noalloc(self._h, px, flags, pf, pe, ctypes.byref(e), ptr(w)))
        return e.value, w

    def reneighbor_device(self, x_owned_dev, lo, hi, periodic, skin, stream=None):
        """Device reneighbor; wraps x_owned_dev in place into [lo, hi)."""
        px = device_f64(x_owned_dev, 3 * self.n, "owned positions")
        if stream is not None:
            self._check(self._lib.so3lr_set_stream(self._h, ctypes.c_void_p(stream)))
        lo = np.ascontiguousarray(lo, dtype=np.float64)
        hi = np.ascontiguousarray(hi, dtype=np.float64)
        per = np.ascontiguousarray(periodic, dtype=np.int32)
        self._check(self._lib.so3lr_reneighbor_device(self._h, px, ptr(lo), ptr(hi), ptr(per), float(skin)))
        self.rows = self.n

    def set_box(self, lo, hi):
        lo = np.ascontiguousarray(lo, dtype=np.float64)
        hi = np.ascontiguousarray(hi, dtype=np.float64)
        self._check(self._lib.so3lr_set_box(self._h, ptr(lo), ptr(hi)))

    def raw_compute(self, x_rows, flags, f, eatom, energy, virial):
        return self._lib.so3lr_compute(self._h, x_rows, flags, f, eatom, energy, virial)

    def terms(self):
        n = self.n
        out = {k: np.zeros(n) for k in ("learned", "zbl", "long_range", "charges", "hirshfeld")}
        tot = np.zeros(2)
        img = np.zeros(getattr(self, "n_images", 1))
        self._check(self._lib.so3lr_last_terms(self._h, ptr(out["learned"]), ptr(out["zbl"]),
                                               ptr(out["long_range"]), ptr(out["charges"]),
                                               ptr(out["hirshfeld"]), ptr(tot), ptr(img)))
        out["electrostatic_total"], out["dispersion_total"] = tot
        out["image_energy"] = img
        return out

    def vatom(self, out=None):
        """Per-atom virial of the last evaluation, (n, 6) in LAMMPS order; `out`
        may be a device tensor (written on the context's stream)."""
        if out is not None and hasattr(out, "data_ptr") and getattr(out, "is_cuda", False):
            self._check(self._lib.so3lr_last_vatom(self._h, device_f64(out, 6 * self.n, "per-atom virial"), 1))
            return out
        w = np.zeros((self.n, 6))
        self._check(self._lib.so3lr_last_vatom(self._h, ptr(w), 0))
        return w

    def graph_stats(self):
        a, b, c = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        self._check(self._lib.so3lr_graph_stats(self._h, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
        return a.value, b.value, c.value

    def kernel_timing(self, enable=True):
        self._check(self._lib.so3lr_kernel_timing(self._h, 1 if enable else 0))

    def kernel_timing_read(self, kernel):
        ms, launches, units = ctypes.c_double(), ctypes.c_int64(), ctypes.c_int64()
        self._check(self._lib.so3lr_kernel_timing_read(self._h, kernel.encode(), ctypes.byref(ms),
                                                       ctypes.byref(launches), ctypes.byref(units)))
        return ms.value, launches.value, units.value

    def device_bytes(self):
        return int(self._lib.so3lr_device_bytes(self._h))
