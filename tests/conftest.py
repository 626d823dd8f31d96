import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")
    config.addinivalue_line("markers", "slow: CPU test that takes more than ~20 s")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The achieved parity margins of this run's GPU tests against the bars
    (energy 1e-10 relative, forces 1e-9 eV/A, virial 1e-9 eV absolute where a
    test holds it to that), one line per comparison."""
    import support
    tr = terminalreporter
    if support.TRAJECTORY:
        tr.section("trajectory margins (HIP-driven vs oracle-driven NVE)")
        tr.write_line("%-58s %10s %10s" % ("case", "max|dx| A", "energy"))
        for case, dx, de, unit in support.TRAJECTORY:
            tr.write_line("%-58s %10.2e %10.2e %s" % (case[:58], dx, de, unit))
    if not support.MARGINS:
        return
    tr.section("parity margins (HIP vs CPU oracle)")
    tr.write_line("%-58s %10s %10s %10s %10s" % ("case", "|dE|/|E|", "max|dF|", "max|dW|", "max|W|"))
    worst = [0.0, 0.0, 0.0]
    for case, de, df, dw, wmax in support.MARGINS:
        tr.write_line("%-58s %10.2e %10.2e %10.2e %10.2e" % (case[:58], de, df, dw, wmax))
        worst = [max(worst[0], de), max(worst[1], df), max(worst[2], dw)]
    tr.write_line("%-58s %10.2e %10.2e %10.2e" % ("worst of %d comparisons" % len(support.MARGINS), *worst))
