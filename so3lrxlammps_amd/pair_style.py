"""Host-side mirror of `pair_style so3lr/native/mpi` driving libso3lr_hip.

Same commands, argument meaning and error behaviour as PairSO3LRNativeMPI
(source/so3lr-lammps-native/plugins/lammps/pair_so3lr_native_mpi.{h,cpp}):

    pair = PairSO3LRNativeMPI()
    pair.settings(["so3lr.so3lr", "0", "1"])      # pair_style ... MODEL [Q [M]]
    pair.coeff(["*", "*", "O", "H"], ntypes=2)    # pair_coeff * * E1 .. En
    pair.init_style(atoms)                        # newton on, (Q, M) check
    result = pair.compute(atoms, eflag=True, vflag=True)

`atoms` carries what LAMMPS's Atom/Domain would: positions, types (1-based),
box bounds and periodicity.  Ghost rows and the two neighbour lists (full SR,
half LR, cutoff + skin) come from the LAMMPS stand-in in _lib.Lists, rebuilt
when an atom moved more than half the skin (LAMMPS `neigh_modify every 1
delay 0 check yes`).
"""
from dataclasses import dataclass, field

import numpy as np

from . import _lib


class LammpsError(RuntimeError):
    """What error->all(FLERR, ...) would raise inside LAMMPS."""


@dataclass
class Atoms:
    x: np.ndarray                 # (n, 3) owned positions
    types: np.ndarray             # (n,) LAMMPS types, 1-based
    lo: np.ndarray = field(default_factory=lambda: np.zeros(3))
    hi: np.ndarray = field(default_factory=lambda: np.full(3, 40.0))
    periodic: tuple = (0, 0, 0)
    newton_pair: bool = True


class PairSO3LRNativeMPI:
    # constructor flags of the reference (pair_so3lr_native_mpi.cpp:1058-1063)
    manybody_flag = 1
    one_coeff = 1
    restartinfo = 0
    single_enable = 0
    no_virial_fdotr_compute = 1

    def __init__(self, device=0, skin=1.0, comm_cutoff=13.0, nprocs=1):
        self.device = device
        self.skin = skin
        self.comm_cutoff = comm_cutoff
        self.nprocs = nprocs  # MPI ranks of this LAMMPS run
        self.warnings = []    # what error->warning would print
        self.ctx = None
        self.type_to_z = None
        self.total_charge = 0.0
        self.multiplicity = 1.0
        self._lists = None
        self._x_at_build = None
        self.topology_rebuilds = 0
        self.topology_hits = 0

    # -- pair_style so3lr/native/mpi MODEL [charge [multiplicity]] (:1097-1137)
    def settings(self, args):
        if len(args) < 1 or len(args) > 3:
            raise LammpsError("Illegal pair_style so3lr/native/mpi command: expected "
                              "'pair_style so3lr/native/mpi MODEL [charge [multiplicity]]'")
        self.model_path = args[0]
        self.total_charge = float(args[1]) if len(args) > 1 else 0.0
        self.multiplicity = float(args[2]) if len(args) > 2 else 1.0
        try:
            self.ctx = _lib.Context(self.model_path, self.device)
        except _lib.SO3LRError as exc:
            raise LammpsError(str(exc)) from exc
        self.short_range_cutoff = self.ctx.cutoff(0)
        self.long_range_cutoff = self.ctx.cutoff(1)

    # -- pair_coeff * * E1 ... Entypes (:1139-1160)
    def coeff(self, args, ntypes):
        if len(args) != ntypes + 2 or args[0] != "*" or args[1] != "*":
            raise LammpsError("Pair coeff for so3lr/native/mpi must be '* * E1 ... Entypes' "
                              "where each E is an element symbol or atomic number")
        lib = _lib.hip()
        t2z = [0] * (ntypes + 1)
        for t in range(1, ntypes + 1):
            z = lib.so3lr_atomic_number(args[t + 1].encode())
            if z == 0:
                raise LammpsError("Unknown SO3LR element '%s'; use a symbol or atomic number "
                                  "from H/1 through Es/99" % args[t + 1])
            t2z[t] = z
        self.type_to_z = np.array(t2z, dtype=np.int32)

    def init_one(self, i, j):
        if self.type_to_z is None:
            raise LammpsError("All so3lr/native/mpi coefficients are not set")
        return self.short_range_cutoff

    # -- init_style + setup_charge_spin (:1174-1235)
    def init_style(self, atoms):
        if not atoms.newton_pair:
            raise LammpsError("Pair style so3lr/native/mpi requires newton pair on")
        if self.ctx is None:
            raise LammpsError("Pair style so3lr/native/mpi model was not initialized")
        if self.type_to_z is None:
            raise LammpsError("Pair style so3lr/native/mpi coefficients are missing")
        # one rank drives one GPU: ghosts come from LAMMPS's own communication
        if self.nprocs != 1:
            raise LammpsError("Pair style so3lr/native/mpi on libso3lr_hip runs one MPI rank per GPU "
                              "(got %d ranks)" % self.nprocs)
        if self.comm_cutoff < self.long_range_cutoff + self.skin:
            raise LammpsError("Pair style so3lr/native/mpi needs comm_modify cutoff >= %g "
                              "(long-range cutoff + skin)" % (self.long_range_cutoff + self.skin))
        z = self.type_to_z[np.asarray(atoms.types)]
        try:
            self.ctx.set_system(z, self.total_charge, self.multiplicity)
        except _lib.SO3LRError as exc:
            raise LammpsError("Pair style so3lr/native/mpi: %s" % exc) from exc
        if self.total_charge != 0.0 and any(atoms.periodic):
            self.warnings.append("SO3LR: net charge %g in a periodic cell. SO3LR's long range is "
                                 "truncated real-space Coulomb, so the energy is defined, but there is "
                                 "no neutralizing background" % self.total_charge)
        self._lists = None

    def _neighbor(self, atoms):
        x = np.asarray(atoms.x, dtype=np.float64)
        if self._lists is not None:
            disp = np.sqrt(((x - self._x_at_build) ** 2).sum(1)).max()
            if disp <= 0.5 * self.skin:
                self.topology_hits += 1
                return
        lo, hi = np.asarray(atoms.lo, float), np.asarray(atoms.hi, float)
        per = np.asarray(atoms.periodic, dtype=np.int32)
        xw = x.copy()
        box = hi - lo
        for d in range(3):
            if per[d]:
                xw[:, d] = lo[d] + np.mod(xw[:, d] - lo[d], box[d])
                xw[:, d] = np.where(xw[:, d] >= hi[d], lo[d], xw[:, d])
        atoms.x = xw  # LAMMPS remaps owned atoms into the box at reneighbor
        self._lists = _lib.Lists(xw, lo, hi, per, self.short_range_cutoff, self.long_range_cutoff,
                                 self.skin, self.comm_cutoff, sr_full=True)
        try:
            self.ctx.set_topology(self._lists)
        except _lib.SO3LRError as exc:
            raise LammpsError("SO3LR MPI-native LAMMPS evaluation failed: %s" % exc) from exc
        self._x_at_build = xw.copy()
        self.topology_rebuilds += 1

    # -- compute(eflag, vflag) (:1246-1978)
    def compute(self, atoms, eflag=True, vflag=True, eflag_atom=False, vflag_atom=False):
        self._neighbor(atoms)
        x_rows = self._lists.rows_positions(np.asarray(atoms.x, dtype=np.float64))
        try:
            energy, forces, eatom, virial = self.ctx.compute(x_rows, eatom=True)
        except _lib.SO3LRError as exc:
            raise LammpsError("SO3LR MPI-native LAMMPS evaluation failed: %s" % exc) from exc
        # per-atom virial: an addition (the reference refuses vflag_atom,
        # pair_so3lr_native_mpi.cpp:1248-1251)
        vatom = self.ctx.vatom() if vflag_atom else None
        return {"energy": energy if eflag else None, "forces": forces,
                "eatom": eatom if eflag_atom else None, "virial": virial if vflag else None,
                "vatom": vatom}
