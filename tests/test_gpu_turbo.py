"""so3lr/turbo on the MI355X: four MPI ranks, each a one-rank partition with
its own reference molecule and (Q, M) (acetate -1, alanine+ doublet, H2O+
doublet, triplet O2); rank 0 is the coordinator and the only process on the
GPU.  tests/turbo_ranks.py checks every image against the CPU oracle on that
image alone (energy 1e-10 relative, forces and the f.r virial 1e-9 eV/A,
per-atom energy 1e-10, charges and Hirshfeld ratios 1e-12), through a move
without reneighbor, one with it, a malformed list on image 2 and a bad charge
on image 1 (both must reach every rank as the same error, and the broker must
keep working), and 20 velocity-Verlet steps.
"""
import os
import re
import subprocess
import sys

import pytest

import support

pytestmark = pytest.mark.gpu

MPIEXEC = os.environ.get("SO3LR_MPIEXEC", "/opt/conda/bin/mpiexec")
RANKS = os.path.join(support.REPO, "tests", "turbo_ranks.py")


def test_turbo_images_match_oracle():
    print("turbo: 4 ranks, molecules acetate, alanine_cation, h2o_cation, o2", flush=True)
    r = subprocess.run([MPIEXEC, "-launcher", "fork", "-n", "4", sys.executable, "-u", RANKS, "gpu"],
                       cwd=support.REPO, capture_output=True, text=True, timeout=240)
    print(r.stdout[-6000:], flush=True)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    out = r.stdout
    assert out.count("PASS") == 4, out
    # the ranks' lines reach the launcher's stdout concurrently and may share
    # a line: take each record up to the next rank marker
    records = [(int(r), m.strip()) for r, m in re.findall(r"\[rank (\d+)\] (MSG [^\n\[]*)", out)]
    for planted in ("from image 2", "image 1: charge 0.5"):
        got = [(r, m) for r, m in records if planted in m]
        assert sorted(r for r, _ in got) == [0, 1, 2, 3], out
        assert len({m for _, m in got}) == 1, got  # the same status and message on every rank
