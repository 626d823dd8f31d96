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
        near = grid.near(p)
        if near:
            d = p - np.asarray(near)
            d -= box * np.round(d / box)
            best = min(best, float(np.sqrt((d * d).sum(1)).min()))
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


# molecule builder ---------------------------------------------------------
_VALENCE = {6: 4, 7: 3, 8: 2, 16: 2}


def _bond_length(rng, a, b):
    """Bond length (A) of heavy atoms a-b: C=O 1.23, bonds to S 1.80, else
    uniform in 1.45-1.54 (C-C, C-N, N-N, ...)."""
    pair = {a, b}
    if pair == {6, 8}:
        return 1.23
    if 16 in pair:
        return 1.80
    return rng.uniform(1.45, 1.54)


def _unit(rng):
    v = rng.normal(size=3)
    return v / np.linalg.norm(v)


def molecule(rng, heavy, n_h, min_nb=1.8, min_angle_pair=1.5, tries=400, bonds_out=None):
    """Seeded molecule geometry: a self-avoiding tree of the heavy atoms
    (`heavy`: atomic numbers, the first one the root), each new atom bonded to
    an earlier one with free valence (oxygen terminal, as a carbonyl on
    carbon), then n_h hydrogens at 1.09 A on atoms with free valence.  Atoms
    further apart than one bond angle (non-bonded pairs) stay at least
    `min_nb` apart; the two ends of a bond angle at least `min_angle_pair`
    (an H-C-H angle of 87 degrees).  Returns (z, positions) centred at the
    origin, or None when the draw fails; bonds_out (a list) receives the
    bonded index pairs."""
    z = [int(heavy[0])]
    pos = [np.zeros(3)]
    free = [_VALENCE[z[0]]]
    bonded = [set()]

    def ok(p, parent):
        d = np.linalg.norm(np.asarray(pos) - p, axis=1)
        bound = np.full(len(pos), min_nb)
        bound[list(bonded[parent])] = min_angle_pair
        bound[parent] = 0.0
        return bool(np.all(d >= bound))

    for zz in heavy[1:]:
        zz = int(zz)
        need = 2 if zz == 8 else 1  # carbonyl oxygen takes two valence units of its carbon
        parents = [k for k in range(len(z)) if free[k] >= need and z[k] != 8 and (zz != 8 or z[k] == 6)]
        if not parents:
            return None
        placed = False
        for _ in range(tries):
            k = parents[rng.integers(len(parents))]
            p = pos[k] + _bond_length(rng, z[k], zz) * _unit(rng)
            if ok(p, k):
                z.append(zz)
                pos.append(p)
                free[k] -= need
                free.append(_VALENCE[zz] - need)
                bonded[k].add(len(z) - 1)
                bonded.append({k})
                placed = True
                break
        if not placed:
            return None
    for _ in range(n_h):
        hosts = [k for k in range(len(z)) if z[k] != 1 and free[k] > 0]
        if not hosts:
            return None
        placed = False
        for _ in range(tries):
            k = hosts[rng.integers(len(hosts))]
            p = pos[k] + 1.09 * _unit(rng)
            if ok(p, k):
                z.append(1)
                pos.append(p)
                free[k] -= 1
                free.append(0)
                bonded[k].add(len(z) - 1)
                bonded.append({k})
                placed = True
                break
        if not placed:
            return None
    pos = np.array(pos)
    if bonds_out is not None:
        bonds_out[:] = [(k, j) for k in range(len(z)) for j in bonded[k] if j > k]
    return np.array(z, dtype=np.int32), pos - pos.mean(0)


def draw_molecule(rng, heavy, n_h, attempts=200, bonds_out=None):
    for _ in range(attempts):
        out = molecule(rng, heavy, n_h, bonds_out=bonds_out)
        if out is not None:
            return out
    raise RuntimeError("no molecule geometry for %s + %d H" % (list(heavy), n_h))


def organic_c6h12n2o2(seed=SEED, bonds_out=None):
    """Config 0: one 22-atom C6H12N2O2 molecule (Q = 0, M = 1)."""
    rng = np.random.default_rng([seed, 0])
    heavy = [6] + list(rng.permutation([6] * 5 + [7] * 2 + [8] * 2))
    # oxygens last so that every one finds a carbon with two free valences
    heavy = [h for h in heavy if h != 8] + [8, 8]
    return draw_molecule(rng, heavy, 12, bonds_out=bonds_out)


def electron_multiplicity(z, charge):
    """Lowest multiplicity of the electron count: 1 if even, 2 if odd."""
    n_e = int(np.sum(z)) - int(charge)
    return 1.0 if n_e % 2 == 0 else 2.0


def packed_molecules(n_mol=512, seed=SEED, spacing=None):
    """Config 2: n_mol molecules of 12-40 atoms (H, C, N, O, S), charge drawn
    from {-1, 0, +1} and multiplicity from the electron-count parity, placed
    on a cubic grid far enough apart that no two molecules interact (every
    inter-molecule distance exceeds the 13 A long-range reach).  Returns
    (z, positions, image_offsets, charges, multiplicities, box_extent)."""
    rng = np.random.default_rng([seed, 2])
    mols, qs, ms = [], [], []
    for _ in range(n_mol):
        n = int(rng.integers(12, 41))
        while True:
            n_heavy = max(4, int(round(n * rng.uniform(0.35, 0.55))))
            n_h = n - n_heavy
            kinds = rng.choice([6, 7, 8, 16], size=n_heavy - 1, p=[0.65, 0.15, 0.15, 0.05])
            heavy = [6] + [k for k in kinds if k != 8] + [k for k in kinds if k == 8]
            chain = [k for k in heavy if k != 8]
            # valence left for hydrogens once the heavy-atom tree and the
            # carbonyl oxygens are in place
            room = sum(_VALENCE[k] for k in chain) - 2 * (len(chain) - 1) - 2 * (len(heavy) - len(chain))
            n_c = sum(1 for k in chain if k == 6)
            if n_h <= room and len(heavy) - len(chain) <= n_c:
                break
        z, x = draw_molecule(rng, heavy, n_h)
        q = float(rng.integers(-1, 2))
        mols.append((z, x))
        qs.append(q)
        ms.append(electron_multiplicity(z, q))
    extent = max(np.abs(x).max() for _, x in mols)
    spacing = spacing or (2.0 * extent + 14.0)
    g = int(np.ceil(n_mol ** (1.0 / 3.0)))
    zs, xs, offs = [], [], [0]
    for k, (z, x) in enumerate(mols):
        c = np.array([k // (g * g), (k // g) % g, k % g], float) * spacing + spacing / 2
        zs.append(z)
        xs.append(x + c)
        offs.append(offs[-1] + len(z))
    return (np.concatenate(zs), np.concatenate(xs), np.array(offs, dtype=np.int64), np.array(qs), np.array(ms),
            g * spacing)


def config(index, seed=SEED):
    """(z, positions, box or None, charge, multiplicity, description) of a
    single system; config 2 (packed images) comes from packed_molecules."""
    if index == 0:
        z, x = organic_c6h12n2o2(seed)
        return z, x + 20.0, None, 0.0, 1.0, "C6H12N2O2 (22 atoms), non-periodic 40 A box"
    if index == 1:
        z, x, b = solvated_box(1000, 0, 0, 31.04, seed)
        return z, x, b, 0.0, 1.0, "1,000 H2O, cubic 31.04 A, periodic"
    if index == 3:
        z, x, b = solvated_box(7900, 150, 150, 62.6, seed)
        return z, x, b, 0.0, 1.0, "7,900 H2O + 150 Na+ + 150 Cl-, cubic 62.6 A, periodic"
    if index == 4:
        z, x, b = solvated_box(50000, 0, 0, 114.0, seed)
        return z, x, b, 0.0, 1.0, "50,000 H2O, cubic 114.0 A, periodic"
    raise ValueError("configuration %d is not a single system (config 2: packed_molecules)" % index)


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
