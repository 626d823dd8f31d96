"""Rank program of the so3lr/turbo tests: run under mpiexec, one process per
image (test_turbo_cpu.py and test_gpu_turbo.py start it).

  cpu  -- no GPU: the collective (Q, M) check names the failing image on every
          rank; the coordinator's failed model load (no HIP device) reaches
          every rank with one status and message.
  gpu  -- rank 0 owns the GPU.  Each rank runs one reference molecule with its
          own (Q, M) through the pair-style mirror: forces, energy, per-atom
          energy, charges, Hirshfeld ratios and the f.r virial are checked
          against the CPU oracle on the image alone; then a move without
          reneighbor, a move with one, a malformed list on one image and a bad
          (Q, M) on another (every rank must see the same error, and the
          broker must keep working), and a run of steps for the timings.
Each rank prints "[rank r] ..." lines; "PASS" when every check held.
"""
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

import numpy as np  # noqa: E402

import support  # noqa: E402
from so3lrxlammps_amd import _lib, turbo  # noqa: E402
from so3lrxlammps_amd.pair_style import Atoms  # noqa: E402

# reference molecules with their charge and multiplicity
IMAGES = ["acetate", "alanine_cation", "h2o_cation", "o2", "methyl", "methylammonium", "alanine"]


def main():
    mode = sys.argv[1]
    comm, rank, size = turbo.mpi_world()

    def say(*a):
        print("[rank %d] %s" % (rank, " ".join(str(x) for x in a)), flush=True)

    if mode == "cpu":
        z = np.array([8, 1, 1], dtype=np.int32)
        try:
            turbo.check_images(comm, z, 0.0, 2.0 if rank == 1 else 1.0)
            raise AssertionError("an impossible multiplicity passed")
        except _lib.SO3LRError as exc:
            assert exc.code == _lib.ERR_SYSTEM, exc.code
            assert "image 1: charge 0 with multiplicity 2" in str(exc), str(exc)
        turbo.check_images(comm, z, 0.0, 1.0)
        if not os.path.exists("/dev/kfd"):  # no GPU driver on this machine
            try:
                turbo.Broker(comm, support.MODEL, 0, 0)
                raise AssertionError("the coordinator found a GPU")
            except _lib.SO3LRError as exc:
                say("MSG", exc.code, str(exc))
        say("PASS")
        return

    from oracle.oracle import Oracle
    orc = Oracle(support.MODEL)
    name = IMAGES[rank % len(IMAGES)]
    ref, z, pos, _ = support.load_golden(name)
    q, m = float(ref["charge"]), float(ref["multiplicity"])
    symbols = ref["types"]
    types = np.array([symbols.index(support.SYMBOLS[int(zz)]) + 1 for zz in z])
    lo, hi = pos.min(0) - 30.0, pos.max(0) + 30.0

    pair = turbo.PairSO3LRTurbo(comm)
    pair.settings([support.MODEL, repr(q), repr(m)])
    pair.coeff(["*", "*"] + list(symbols), len(symbols))
    assert pair.init_one(1, 1) == pair.long_range_cutoff
    atoms = Atoms(x=pos.copy(), types=types, lo=lo, hi=hi, periodic=(0, 0, 0))
    pair.init_style(atoms)

    def check(res, x, what):
        sr, lr = support.build_graphs(x, None)
        out = orc.evaluate(z, sr, lr, charge=q, multiplicity=m)
        de = abs(res["energy"] - out["energy"])
        df = np.abs(res["forces"] - out["forces"]).max()
        dw = np.abs(res["virial"] - out["virial"]).max()
        dea = np.abs(res["eatom"] - out["eatom"]).max()
        dq = np.abs(res["charges"] - out["charges"]).max()
        dh = np.abs(res["hirshfeld"] - out["hirshfeld"]).max()
        assert de <= 1e-10 * abs(out["energy"]), (what, de)
        assert df <= 1e-9, (what, df)
        assert dw <= 1e-9 * max(1.0, np.abs(out["virial"]).max()), (what, dw)
        assert dea <= 1e-10 * max(1.0, np.abs(out["eatom"]).max()), (what, dea)
        assert dq <= 1e-12 and dh <= 1e-12, (what, dq, dh)
        assert abs(res["charges"].sum() - q) < 1e-12, what
        say(what, name, "n=%d" % len(z), "dE=%.1e dF=%.1e dW=%.1e dq=%.1e" % (de, df, dw, dq))

    res = pair.compute(atoms, eflag_atom=True)
    assert res["lists_changed"]
    check(res, atoms.x, "first call")
    st = pair.broker.stats()
    if rank == 0:
        assert st["images"] == size and st["lists_gathered"] == 1, st
    rng = np.random.default_rng(100 + rank)

    # a move inside half the skin: no reneighbor anywhere, the lists stay put
    atoms.x = atoms.x + rng.uniform(-0.1, 0.1, atoms.x.shape)
    res = pair.compute(atoms, eflag_atom=True)
    assert not res["lists_changed"]
    assert pair.broker.stats()["lists_gathered"] == 0
    check(res, atoms.x, "moved")

    # image 1 moves an atom 0.8 A away from its centre: it reneighbours and
    # sends its lists; the coordinator keeps the other images' lists
    if rank == 1:
        out = atoms.x[0] - atoms.x.mean(0)
        atoms.x[0] += 0.8 * out / np.linalg.norm(out)
    res = pair.compute(atoms, eflag_atom=True)
    assert res["lists_changed"] == (rank == 1)
    # only image 1 sent its lists; the coordinator received them
    assert pair.broker.stats()["lists_gathered"] == (1 if rank in (0, 1) else 0)
    check(res, atoms.x, "reneighbour")

    # a malformed list on image 2: every rank gets the same error
    bad = 2 % size
    lists = pair._lists
    (si, so, sn), (li, lo_, ln) = lists.lists
    assert len(sn) > 0
    sn_bad = sn.copy()
    if rank == bad:
        sn_bad[0] = len(z) + 5  # a ghost row: turbo images have none
    zz = pair.type_to_z[atoms.types].astype(np.int32)
    x = np.ascontiguousarray(atoms.x)
    f = np.zeros((len(z), 3))
    rc = pair.broker.raw_evaluate(len(z), _lib.ptr(zz), _lib.ptr(x), q, m, 1, _lib.LIST_FULL, len(si),
                                  _lib.ptr(si), _lib.ptr(so), _lib.ptr(sn_bad), len(li), _lib.ptr(li),
                                  _lib.ptr(lo_), _lib.ptr(ln), _lib.ptr(f), None, None, None, None)
    assert rc == _lib.ERR_TOPOLOGY, rc
    err = pair.broker.last_error()
    assert ("from image %d" % bad) in err and "ghost rows" in err, err
    say("MSG", rc, err)
    res = pair.compute(atoms, eflag_atom=True)
    check(res, atoms.x, "after a malformed list")

    # a non-integer charge on image 1, given straight to the broker
    bq = 1 % size
    try:
        pair.broker.evaluate(zz, x, 0.5 if rank == bq else q, m, lists, False)
        raise AssertionError("a charge of 0.5 passed")
    except _lib.SO3LRError as exc:
        assert exc.code == _lib.ERR_SYSTEM, exc.code
        assert ("image %d: charge 0.5" % bq) in str(exc), str(exc)
        say("MSG", exc.code, str(exc))
    res = pair.compute(atoms, eflag_atom=True)
    check(res, atoms.x, "after a bad charge")

    # a short run: velocity Verlet with 0.25 fs steps, then the timings
    mass = np.array([{1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999}[int(zz)] for zz in z])
    v = np.zeros_like(atoms.x)
    f = res["forces"]
    dt = 0.25e-3  # ps
    conv = 9648.533212  # eV/(A amu) -> A/ps^2
    steps = int(os.environ.get("SO3LR_TURBO_STEPS", "20"))
    t0 = time.perf_counter()
    tot = {"gather_ms": 0.0, "evaluate_ms": 0.0, "scatter_ms": 0.0, "total_ms": 0.0}
    for _ in range(steps):
        v += 0.5 * dt * f / mass[:, None] * conv
        atoms.x = atoms.x + dt * v
        res = pair.compute(atoms)
        f = res["forces"]
        v += 0.5 * dt * f / mass[:, None] * conv
        st = pair.broker.stats()
        for k in tot:
            tot[k] += st[k]
    wall = time.perf_counter() - t0
    check(pair.compute(atoms, eflag_atom=True), atoms.x, "after %d steps" % steps)
    if rank == 0:
        say("TIMING images=%d packed_atoms=%d steps=%d wall_ms_per_step=%.3f gather_ms=%.3f evaluate_ms=%.3f "
            "scatter_ms=%.3f call_ms=%.3f" % (size, pair.broker.stats()["packed_atoms"], steps,
                                              1e3 * wall / steps, tot["gather_ms"] / steps,
                                              tot["evaluate_ms"] / steps, tot["scatter_ms"] / steps,
                                              tot["total_ms"] / steps))
    pair.broker.close()
    say("PASS")


if __name__ == "__main__":
    try:
        main()
    except Exception:
        import traceback
        traceback.print_exc()
        sys.stdout.flush()
        os._exit(1)  # the launcher then stops the other ranks
    turbo.mpi_finalize()
