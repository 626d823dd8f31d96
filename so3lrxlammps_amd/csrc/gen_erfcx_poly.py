"""Derives the polynomial of the long-range kernels' erf (device_math.hpp).

erf(x) = 1 - exp(-x^2) erfcx(x), with erfcx(x) = exp(x^2) erfc(x) smooth and
slowly varying on [0, 3] (1 down to 0.18).  A degree-26 Chebyshev fit of
erfcx in u = 2 x / 3 - 1 (u in [-1, 1]), written out in powers of u, is
evaluated by Horner's rule in fp64; the resulting erf is checked here
against mpmath at 40 digits: absolute error < 4e-16 on [0, 3], relative
< 1e-15 for x > 0.2.

    python gen_erfcx_poly.py      # prints the C++ table (highest power first)
"""
import math

import mpmath as mp
import numpy as np

X, DEG = 3.0, 26
mp.mp.dps = 50
poly = mp.chebyfit(lambda u: mp.exp(((u + 1) * X / 2) ** 2) * mp.erfc((u + 1) * X / 2), [-1, 1], DEG)
coef = [float(c) for c in poly]  # highest power first

worst_abs = worst_rel = 0.0
for x in np.linspace(0.0, X, 20001):
    u = 2.0 * x / X - 1.0
    p = 0.0
    for c in coef:
        p = p * u + c
    e = 1.0 - math.exp(-x * x) * p
    ref = float(mp.erf(x))
    worst_abs = max(worst_abs, abs(e - ref))
    if x > 0.2:
        worst_rel = max(worst_rel, abs(e - ref) / ref)
assert worst_abs < 4e-16 and worst_rel < 1e-15, (worst_abs, worst_rel)

print("// erfcx(x) on [0, 3] in u = 2 x / 3 - 1, highest power first (gen_erfcx_poly.py)")
print("constexpr double kErfcxPoly[%d] = {" % len(coef))
for i in range(0, len(coef), 3):
    print("    " + ", ".join("%.17g" % c for c in coef[i:i + 3]) + ",")
print("};")
print("// max abs error of erf %.2e, max rel error (x > 0.2) %.2e" % (worst_abs, worst_rel))
