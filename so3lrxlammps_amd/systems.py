"""Seeded synthetic systems of the benchmark configurations.

config 0  one C6H12N2O2 molecule (22 atoms), non-periodic
config 1  1,000 rigid H2O on a jittered cubic lattice, cubic cell 31.04 A
config 2  512 molecules of 12-40 atoms (H, C, N, O, S), packed images
config 3  7,900 H2O + 150 Na+ + 150 Cl-, cubic cell 62.6 A      (headline)
config 4  50,000 H2O, cubic cell 114.0 A
Water follows the reference generator's geometry (O-H 0.9572 A, H-O-H
104.52 deg, random orientations; examples/scaling/generate_water_boxes.py:83-132),
with lattice jitter and a minimum intermolecular distance enforced by
re-drawing orientations.
"""
import numpy as np

SEED = 20261201
MASS = {1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999, 11: 22.990, 16: 32.06, 17: 35.45}

_OH = 0.9572
_ANG = np.radians(104.52)
WATER = np.array([[0.0, 0.0, 0.0],
                  [_OH, 0.0, 0.0],
                  [_OH * np.cos(_ANG), _OH * np.sin(_ANG), 0.0]])
WATER = WATER - WATER.mean(0) * 0.0  # oxygen at the molecule origin


def _rotation(rng):
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                     [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                     [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])


class _Grid:
    """Spatial hash for minimum-distance checks in a periodic cube."""

    def __init__(self, box, cell=3.0):
        self.box = box
        self.nc = max(1, int(box // cell))
        self.cell = box / self.nc
        self.bins = {}

    def _key(self, p):
        return tuple((np.floor(np.mod(p, self.box) / self.cell).astype(int)) % self.nc)

    def near(self, p):
        k = self._key(p)
        out = []
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    out.extend(self.bins.get(((k[0] + dx) % self.nc, (k[1] + dy) % self.nc,
                                              (k[2] + dz) % self.nc), ()))
        return out

    def add(self, p):
        self.bins.setdefault(self._key(p), []).append(p)


def _min_dist(grid, pts, box):
    best = 1e9
    for p in pts:
        for q in grid.near(p):
            d = p - q
            d -= box * np.round(d / box)
            best = min(best, float(np.sqrt((d * d).sum())))
    return best


def solvated_box(n_water, n_na, n_cl, box, seed=SEED, jitter=0.15, min_dist=1.65, ion_o=2.2):
    """Waters and ions on a jittered cubic lattice with random orientations."""
    rng = np.random.default_rng(seed)
    n_sites = n_water + n_na + n_cl
    g = int(np.ceil(n_sites ** (1.0 / 3.0)))
    spacing = box / g
    sites = np.array([[i, j, k] for i in range(g) for j in range(g) for k in range(g)], float)
    sites = (sites + 0.5) * spacing
    sites = sites[rng.permutation(len(sites))[:n_sites]]
    kind = np.array([0] * n_water + [11] * n_na + [17] * n_cl)
    kind = kind[rng.permutation(n_sites)]
    grid = _Grid(box)
    pos, z = [], []
    for s, kd in zip(sites, kind):
        c = s + rng.uniform(-jitter, jitter, 3)
        if kd == 0:
            for _ in range(200):
                mol = WATER @ _rotation(rng).T + c
                if _min_dist(grid, mol, box) >= min_dist:
                    break
            for p, zz in zip(mol, (8, 1, 1)):
                grid.add(p)
                pos.append(p)
                z.append(zz)
        else:
            if _min_dist(grid, [c], box) < ion_o:
                c = s  # lattice site itself keeps >= spacing - 0.96 A from other molecules
            grid.add(c)
            pos.append(c)
            z.append(int(kd))
    pos = np.mod(np.array(pos), box)
    return np.array(z, dtype=np.int32), pos, np.full(3, box)


def config(index, seed=SEED):
    """(z, positions, box or None, charge, multiplicity, description)."""
    if index == 1:
        z, x, b = solvated_box(1000, 0, 0, 31.04, seed)
        return z, x, b, 0.0, 1.0, "1,000 H2O, cubic 31.04 A, periodic"
    if index == 3:
        z, x, b = solvated_box(7900, 150, 150, 62.6, seed)
        return z, x, b, 0.0, 1.0, "7,900 H2O + 150 Na+ + 150 Cl-, cubic 62.6 A, periodic"
    if index == 4:
        z, x, b = solvated_box(50000, 0, 0, 114.0, seed)
        return z, x, b, 0.0, 1.0, "50,000 H2O, cubic 114.0 A, periodic"
    raise ValueError("configuration %d is not a single periodic system" % index)


def maxwell_boltzmann(z, temperature, seed=SEED):
    """Velocities in A/ps (metal units), zero total momentum."""
    rng = np.random.default_rng(seed + 1)
    kB = 8.617333262e-5  # eV/K
    m = np.array([MASS[int(zz)] for zz in z])
    # 1 eV / amu = 9648.533212 A^2/ps^2
    sigma = np.sqrt(kB * temperature / m * 9648.533212)
    v = rng.normal(size=(len(z), 3)) * sigma[:, None]
    v -= (m[:, None] * v).sum(0) / m.sum()
    return v, m
