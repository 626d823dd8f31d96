"""Seeded synthetic systems of the benchmark configurations (CPU only)."""
import numpy as np

import support
from so3lrxlammps_amd import systems


def test_config0_composition_and_geometry():
    z, x, box, q, m, desc = systems.config(0)
    assert box is None and q == 0.0 and m == 1.0
    counts = np.bincount(z, minlength=9)
    assert (counts[1], counts[6], counts[7], counts[8]) == (12, 6, 2, 2)
    assert np.all(x > 0.0) and np.all(x < 40.0)  # inside the 40 A box
    bonds = []
    z2, x2 = systems.organic_c6h12n2o2(bonds_out=bonds)
    assert np.array_equal(z, z2) and np.allclose(x - 20.0, x2)  # deterministic, same draw
    n = len(z)
    assert len(bonds) == n - 1  # a tree: every atom attached
    adj = np.zeros((n, n), dtype=int)
    for a, b in bonds:
        adj[a, b] = adj[b, a] = 1
    d = np.linalg.norm(x[:, None] - x[None], axis=-1)
    for a, b in bonds:
        pair = {int(z[a]), int(z[b])}
        if 1 in pair:
            assert abs(d[a, b] - 1.09) < 1e-9
        elif pair == {6, 8}:
            assert abs(d[a, b] - 1.23) < 1e-9
        else:
            assert 1.45 - 1e-9 <= d[a, b] <= 1.54 + 1e-9
    near = (adj + adj @ adj) > 0  # bonded or sharing a bonded neighbour
    np.fill_diagonal(near, True)
    assert d[~near].min() >= 1.8  # the non-bonded minimum distance
    assert d[near & ~np.eye(n, dtype=bool)].min() >= 1.08


def test_config2_packed_images():
    z, x, offs, qs, ms, extent = systems.packed_molecules(n_mol=27)
    sizes = np.diff(offs)
    assert len(sizes) == 27 and sizes.min() >= 12 and sizes.max() <= 40
    assert set(np.unique(z)) <= {1, 6, 7, 8, 16}
    assert set(qs) <= {-1.0, 0.0, 1.0}
    for k in range(27):
        ne = int(z[offs[k]:offs[k + 1]].sum()) - int(qs[k])
        assert ms[k] == (1.0 if ne % 2 == 0 else 2.0)
    # images never interact: every inter-molecule distance beyond the LR list reach
    img = np.repeat(np.arange(27), sizes)
    d = np.linalg.norm(x[:, None] - x[None], axis=-1)
    assert d[img[:, None] != img[None, :]].min() > 13.0


def test_water_configs_density_and_overlap():
    for index, n, box in ((1, 3000, 31.04), (3, 24000, 62.6)):
        z, x, b, q, m, desc = systems.config(index)
        assert len(z) == n and np.allclose(b, box)
        assert np.all(x >= 0) and np.all(x < box)
        assert abs(z.sum() - (n // 3 * 10 if index == 1 else 7900 * 10 + 150 * 11 + 150 * 17)) == 0
    # the LAMMPS stand-in's lists on config 1 agree with brute force (graph helper)
    z, x, b, *_ = systems.config(1)
    from so3lrxlammps_amd import Lists
    lists = Lists(x, np.zeros(3), b, (1, 1, 1))
    sr, lr = support.graphs_from_lists(lists, x)
    sr2, lr2 = support.build_graphs(x, b)
    key = lambda s, r: np.sort(s * len(z) + r)
    assert np.array_equal(key(sr[0], sr[1]), key(sr2[0], sr2[1]))
    a = np.sort(np.minimum(lr[0], lr[1]) * len(z) + np.maximum(lr[0], lr[1]))
    b2 = np.sort(np.minimum(lr2[0], lr2[1]) * len(z) + np.maximum(lr2[0], lr2[1]))
    assert np.array_equal(a, b2)
