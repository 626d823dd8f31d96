"""so3lr/turbo on the CPU: libso3lr_turbo.so loads and exports every symbol
include/so3lr_turbo.h declares, and under mpiexec (3 ranks, no GPU) the
collective checks give every rank the same status and message: the per-image
(Q, M) check names the failing image (pair_so3lr_turbo.cpp:208-222), and the
coordinator's failed model load stops every rank (pair_so3lr_turbo.cpp:122-153).
"""
import os
import re
import subprocess
import sys

import pytest

import support
from so3lrxlammps_amd import turbo

MPIEXEC = os.environ.get("SO3LR_MPIEXEC", "/opt/conda/bin/mpiexec")
RANKS = os.path.join(support.REPO, "tests", "turbo_ranks.py")

needs_mpi = pytest.mark.skipif(not os.path.exists(MPIEXEC) or not os.path.exists(turbo.TURBO_LIB),
                               reason="MPICH launcher or libso3lr_turbo.so missing")


def test_header_symbols_are_listed():
    text = open(os.path.join(support.REPO, "include", "so3lr_turbo.h")).read()
    declared = re.findall(r"^(?:int|void|const char \*)\s*(so3lr_turbo_\w+)\(", text, re.M)
    assert sorted(declared) == sorted(turbo.TURBO_SYMBOLS)


@needs_mpi
def test_library_loads_and_exports_every_symbol():
    code = ("from so3lrxlammps_amd import turbo; lib = turbo.turbo(); "
            "[getattr(lib, s) for s in turbo.TURBO_SYMBOLS]; print('ok')")
    r = subprocess.run([sys.executable, "-c", code], cwd=support.REPO, capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr


@needs_mpi
def test_collective_failures_reach_every_rank():
    r = subprocess.run([MPIEXEC, "-launcher", "fork", "-n", "3", sys.executable, "-u", RANKS, "cpu"], cwd=support.REPO,
                       capture_output=True, text=True, timeout=120)
    out = r.stdout
    assert r.returncode == 0, out + r.stderr
    assert out.count("PASS") == 3, out
    if not os.path.exists("/dev/kfd"):
        # the ranks' lines may share a line of the launcher's stdout
        records = re.findall(r"\[rank (\d+)\] (MSG [^\n\[]*)", out)
        assert sorted(int(r) for r, _ in records) == [0, 1, 2], out
        msgs = {m.strip() for _, m in records}
        assert len(msgs) == 1, msgs  # one status and message on all three ranks
        msg = msgs.pop()
        assert msg.startswith("MSG 5 Cannot initialize the coordinator SO3LR model"), msg
