"""Shared helpers for the test-suite: LAMMPS data files, brute-force graphs.

The graphs follow the reference's conventions:
  * SR: full directed list, receiver-major (LAMMPS full list, ilist order),
    v = x_receiver - x_sender  (lammps_neighbor_adapter.cpp:58-101);
  * LR: unique half pairs (LAMMPS newton-on half list), d = x_j - x_i with
    i the sender and j the receiver (kokkos_physical_long_range.cpp:147-170).
Periodic images use the minimum-image convention; every periodic box used in
the tests is wider than twice the largest cutoff, so each pair has at most one
image inside the cutoff.
"""
import os

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden")
MODEL = os.path.join(REPO, "models", "so3lr.so3lr")

# achieved parity margins of the GPU tests, printed at the end of the pytest
# run by tests/conftest.py (pytest keeps the stdout of passing tests to itself)
MARGINS = []
# trajectory comparisons: (case, max|dx| in A, energy difference, its unit)
TRAJECTORY = []


def record_margin(e, f, w, out, what=""):
    """Record one comparison of a HIP result (energy e, forces f, virial w)
    with the oracle's `out`: |dE|/|E|, max|dF| and the absolute max|dW|,
    under the current test's name."""
    case = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0].split("::")[-1]
    row = (case + (" " + what if what else ""),
           abs(e - out["energy"]) / max(abs(out["energy"]), 1e-300),
           float(np.abs(np.asarray(f) - out["forces"]).max()) if len(out["forces"]) else 0.0,
           float(np.abs(np.asarray(w) - out["virial"]).max()),
           float(np.abs(out["virial"]).max()))
    MARGINS.append(row)
    return row



def perturbed_model(path, seed=11, scale=0.2, base=MODEL):
    """A copy of the model `base` (the shipped model by default) in which every float64 parameter tensor is
    scaled elementwise by 1 + scale * u, u uniform in [-1, 1] (seeded); the
    derived and physical constants (basis, Clebsch-Gordan tables, reference
    polarizabilities and C6) are kept. A second set of weights for parity
    tests, written with so3lrxlammps_amd.model_file."""
    from so3lrxlammps_amd.model_file import read_model, write_model
    manifest, arrays = read_model(base)
    rng = np.random.default_rng(seed)
    for rec in manifest["tensors"]:
        if rec["role"] == "parameter" and rec["dtype"] == "float64":
            a = arrays[rec["state_key"]]
            arrays[rec["state_key"]] = a * (1.0 + scale * rng.uniform(-1.0, 1.0, a.shape))
    write_model(str(path), manifest, arrays)
    return str(path)


def relabelled_model(path, swaps=((1, 11), (7, 17)), base=MODEL):
    """A copy of the model `base` in which the element rows of each pair of
    atomic numbers in `swaps` trade places in every per-element table, at the
    reference's indexing of each: the learned one-hot tables 118 wide at
    class Z - 1 (embedding, charge/spin queries, energy scales and shifts;
    kokkos_output_heads.cpp:424-436, kokkos_local_energy_reverse.cpp:190-214),
    the 100-row head tables at row Z (atomic charge embedding, Hirshfeld
    queries and shifts; kokkos_output_heads.cpp:157-174,424-439) and the
    reference polarisabilities and C6 at Z - 1
    (kokkos_physical_long_range.cpp:201-211).  A molecule evaluated with this
    model and its atoms relabelled by the same swaps has the learned energy,
    charges, Hirshfeld ratios and long-range energy of the original
    (everything but the ZBL repulsion, which sees the nuclear charge)."""
    from so3lrxlammps_amd.model_file import read_model, write_model
    manifest, arrays = read_model(base)
    learned = {"model.inv_feature_embedding.embedding.weight", "model.charge_embedding.Wq.weight",
               "model.spin_embedding.Wq.weight", "model.atomic_energy_output_block.energy_scales.weight",
               "model.atomic_energy_output_block.energy_shifts"}
    by_z = {"model.partial_charges_output_block.atomic_embedding.weight",
            "model.hirshfeld_output_block.q_embedding.weight", "model.hirshfeld_output_block.v_shift_embedding.weight"}
    physical = {"physical.reference_alphas", "physical.reference_c6"}
    for key in learned | by_z | physical:
        a = arrays[key].copy()
        for za, zb in swaps:
            if key in learned:
                assert a.shape[-1] == 118, key
                a[..., [za - 1, zb - 1]] = a[..., [zb - 1, za - 1]]
            elif key in by_z:
                assert a.shape[0] == 100, key
                a[[za, zb]] = a[[zb, za]]
            else:
                a[[za - 1, zb - 1]] = a[[zb - 1, za - 1]]
        arrays[key] = a
    # no other tensor may carry a per-element axis
    for rec in manifest["tensors"]:
        k = rec["state_key"]
        if k not in learned | by_z | physical and k != "atomic_numbers_map":
            assert not any(d in (100, 102, 118) for d in arrays[k].shape), k
    write_model(str(path), manifest, arrays)
    return str(path)


def variant_model(path, blocks=None, rms_norm=False, norm2=True, qk_norm=False, resid=None, x0=None,
                  nlh=None, c6=None, message_normalization=None, edit=None, seed=5, base=MODEL):
    """A model file with the reference's optional operators switched on
    (so3lr_architecture.cpp:300-392), written from the shipped model:

    blocks: interaction block count (new blocks copy block b % 3 with weights
      scaled by 1 + 0.2 u, u uniform in [-1, 1]);
    rms_norm: RMSNorm without scale at the enabled positions (the LayerNorm
      tensors are dropped: RMSNorm has none); norm2=False: no second norm;
    qk_norm: RMS-normalised q, k, q_ev, k_ev head rows;
    resid, x0: residual scalars per block (model.resid_lambdas, x0_lambdas);
    nlh: (a, b) NLH tables of shape (cap, cap, 3) (physical.nlh_a, nlh_b);
      the learned-ZBL screening keys are removed;
    c6: "copy" (the C6 head is the Hirshfeld head), "perturb" (a copy with
      weights scaled by 1 + 0.2 u) or a dict of its six tensors by suffix;
    message_normalization: "identity", "sqrt_num_features" or
      "avg_num_neighbors";
    edit: called as edit(manifest, arrays) last, for anything else.
    Records are re-sorted by name, sizes and digests recomputed on writing."""
    from so3lrxlammps_amd.model_file import read_model, write_model
    manifest, arrays = read_model(base)
    arch = manifest["architecture"]
    rng = np.random.default_rng(seed)
    recs = {r["state_key"]: r for r in manifest["tensors"]}

    def add(key, a, role="parameter"):
        a = np.asarray(a, dtype=np.float64)
        arrays[key] = a
        recs[key] = {"dtype": "float64", "name": "wrapper.model." + key, "nbytes": 0, "offset": 0,
                     "role": role, "sha256": "", "shape": list(a.shape), "state_key": key}

    def drop(key):
        recs.pop(key)
        arrays.pop(key)

    def perturbed(a):
        return a * (1.0 + 0.2 * rng.uniform(-1.0, 1.0, a.shape))

    L0 = int(arch["interaction_blocks"])
    if blocks is not None and blocks != L0:
        prefix = "model.euclidean_transformers.%d."
        for b in range(blocks, L0):
            for k in [k for k in recs if k.startswith(prefix % b)]:
                drop(k)
        for b in range(L0, blocks):
            src = prefix % (b % L0)
            for k in [k for k in list(recs) if k.startswith(src)]:
                r = dict(recs[k])
                nk = (prefix % b) + k[len(src):]
                r["state_key"] = nk
                r["name"] = r["name"].replace(src, prefix % b)
                a = arrays[k]
                if r["role"] == "parameter" and r["dtype"] == "float64":
                    a = perturbed(a)
                arrays[nk] = a
                recs[nk] = r
        arch["interaction_blocks"] = blocks
    L = int(arch["interaction_blocks"])
    if rms_norm:
        arch["use_rms_norm"] = True
        for b in range(L):
            for pos in (1, 2):
                for w in ("weight", "bias"):
                    drop("model.euclidean_transformers.%d.layer_norm_inv_%d.%s" % (b, pos, w))
    if not norm2:
        arch["layer_normalization_2"] = False
        for b in range(L):
            for w in ("weight", "bias"):
                k = "model.euclidean_transformers.%d.layer_norm_inv_2.%s" % (b, w)
                if k in recs:
                    drop(k)
    if qk_norm:
        arch["qk_norm"] = True
    if resid is not None:
        arch["use_residual_scalars"] = True
        add("model.resid_lambdas", np.asarray(resid, dtype=np.float64))
        add("model.x0_lambdas", np.asarray(x0 if x0 is not None else np.zeros(L), dtype=np.float64))
    if nlh is not None:
        arch["repulsion_type"] = "nlh"
        for k in ("zbl_p", "zbl_d", "zbl_a1", "zbl_a2", "zbl_a3", "zbl_a4", "zbl_c1", "zbl_c2", "zbl_c3",
                  "zbl_c4", "zbl_enabled"):
            arch.pop(k, None)
        add("physical.nlh_a", nlh[0], role="physical_constant")
        add("physical.nlh_b", nlh[1], role="physical_constant")
    if c6 is not None:
        arch["output_heads"] = list(arch["output_heads"]) + ["c6_ratios_output_block"]
        for suffix in ("q_embedding.weight", "transform_features.0.weight", "transform_features.0.bias",
                       "transform_features.2.weight", "transform_features.2.bias", "v_shift_embedding.weight"):
            h = arrays["model.hirshfeld_output_block." + suffix]
            if isinstance(c6, dict):
                a = c6[suffix]
            else:
                a = h.copy() if c6 == "copy" else perturbed(h)
            add("model.c6_ratios_output_block." + suffix, a)
    if message_normalization is not None:
        arch["message_normalization"] = message_normalization
    if edit is not None:
        edit(manifest, arrays)
    manifest["tensors"] = sorted(recs.values(), key=lambda r: r["name"])
    arch["state_tensor_count"] = len(manifest["tensors"])
    arch["parameter_elements"] = int(sum(np.asarray(arrays[r["state_key"]]).size for r in manifest["tensors"]
                                         if r["role"] == "parameter"))
    write_model(str(path), manifest, arrays)
    return str(path)


def _bernstein_elevation(n, m):
    """M (n+1, n+m+1) with B^n_k = sum_j M[k, j] B^(n+m)_j: degree elevation of
    the Bernstein basis, M[k, j] = C(n, k) C(m, j - k) / C(n + m, j)."""
    from math import comb
    M = np.zeros((n + 1, n + m + 1))
    for k in range(n + 1):
        for j in range(k, k + m + 1):
            M[k, j] = comb(n, k) * comb(m, j - k) / comb(n + m, j)
    return M


def lifted_model(path, base=MODEL, R=64, split=0.3, copies=2):
    """The F = 256 model with R = 64 radial functions and the duplicated degree
    slots 1,1,2,2,3,3,4,4 (the "l" widths the reference runs,
    so3lr_capabilities.cpp:54-85) that computes exactly the same function as
    the F = 128 model `base`: a two-copy lift.

    Invariant head h' (8 heads of 32) is a copy of head h'//2 of `base` and
    degree slot s' a copy of slot s'//2; copy = h' % 2 (s' % 2).  Every weight
    that sums over a lifted input takes the base weight times `split` on copy
    0 and 1 - `split` on copy 1, so both copies of every hidden value equal the
    base value (the forward pass is the base pass twice over) while the
    adjoints of the two copies differ, and a reverse pass that mixes them up
    is caught.  The charge/spin query weights carry sqrt(2) for the
    1/sqrt(F) of their logits, and the radial layer reads the degree-31
    Bernstein basis re-expressed in the degree-R-1 basis (exact degree
    elevation).  The energy and charge heads keep their hidden width 128, so
    it differs from F (the "256 -> 128" heads, kokkos_output_heads.cpp:16-19).
    Energies, forces and the virial equal those of `base` up to rounding.
    copies=1 keeps F = 128 and the degrees and changes only the radial basis
    (to R functions by the same degree elevation)."""
    from so3lrxlammps_amd.model_file import read_model, write_model
    manifest, arrays = read_model(base)
    arch = manifest["architecture"]
    F, R0 = int(arch["invariant_features"]), int(arch["radial_basis_features"])
    assert F == 128 and int(arch["attention_heads"]) == 4 and int(arch["euclidean_degree_channels"]) == 4
    assert copies in (1, 2)
    c = copies
    F2, S2 = c * F, 4 * c

    def part(n):  # weight of copy k of n lifted entries: split, 1 - split (1 unlifted)
        k = np.arange(n) % c if c == 2 else np.zeros(n, dtype=int)
        return np.where(k == 0, split, 1.0 - split) if c == 2 else np.ones(n)
    h2 = np.arange(F2) // 32
    cmap = (h2 // c) * 32 + np.arange(F2) % 32
    csplit = part(F2 // 32)[h2]
    smap = np.arange(S2) // c
    ssplit = part(S2)
    hmap = np.arange(F2 // 4) // c
    hsplit = part(F2 // 4)
    reps0 = [3, 5, 7, 9]
    off0 = np.concatenate([[0], np.cumsum(reps0)])
    reps = [reps0[s // c] for s in range(S2)]
    chmap = np.concatenate([off0[s // c] + np.arange(reps[s]) for s in range(S2)])
    seg = np.concatenate([np.full(reps[s], s) for s in range(S2)])
    elev = _bernstein_elevation(R0 - 1, R - R0)
    rowmap = np.concatenate([cmap, F + smap])
    colsplit = np.concatenate([csplit, ssplit])

    def lift_rows_cols(w):  # (F, F) with the input split
        return w[cmap][:, cmap] * csplit[None, :]

    def lift_cols(w):  # (out, F): a head reading the lifted features
        return w[:, cmap] * csplit[None, :]

    out = {}
    for k, a in arrays.items():
        t = k.split(".")
        if k == "model.inv_feature_embedding.embedding.weight":
            out[k] = a[cmap]
        elif k.startswith(("model.charge_embedding.", "model.spin_embedding.")):
            if t[-2] == "Wq":
                out[k] = a[cmap] * np.sqrt(float(c)) * csplit[:, None]
            elif t[-1] in ("Wk", "Wv"):
                out[k] = a[:, cmap]
            else:
                out[k] = lift_rows_cols(a)
        elif k == "model.radial_embedding.radial_basis_fn.b":
            from math import lgamma
            out[k] = np.array([lgamma(R) - lgamma(j + 1) - lgamma(R - j) for j in range(R)])
        elif k == "model.radial_embedding.radial_basis_fn.k":
            out[k] = np.arange(R, dtype=np.int64)
        elif k == "model.radial_embedding.radial_basis_fn.k_rev":
            out[k] = (R - 1 - np.arange(R)).astype(np.int64)
        elif k.startswith("model.euclidean_transformers."):
            if t[-1] in ("W_q_inv", "W_k_inv", "W_v_inv", "W_q_ev", "W_k_ev"):
                out[k] = a[np.arange(F2 // 32) // c]
            elif t[-1] == "degree_repeats":
                out[k] = np.array(reps, dtype=np.int64)
            elif t[-1] == "cg_rep":
                out[k] = a[chmap]
            elif t[-1] == "segment_ids":
                out[k] = seg.astype(a.dtype)
            elif t[-1] == "segment_sum_matrix":
                out[k] = np.eye(S2)[seg]
            elif "mlp_rbf" in t:
                if ".mlp_rbf.0." in k:
                    out[k] = (a @ elev)[cmap] if t[-1] == "weight" else a[cmap]
                else:
                    out[k] = lift_rows_cols(a) if t[-1] == "weight" else a[cmap]
            elif "mlp_ev" in t:
                if ".mlp_ev.0." in k:
                    out[k] = a[hmap][:, smap] * ssplit[None, :] if t[-1] == "weight" else a[hmap]
                else:
                    out[k] = a[cmap][:, hmap] * hsplit[None, :] if t[-1] == "weight" else a[cmap]
            elif t[-2] in ("layer_norm_inv_1", "layer_norm_inv_2"):
                out[k] = a[cmap]
            elif t[-3] == "mlp_1":
                out[k] = lift_rows_cols(a) if t[-1] == "weight" else a[cmap]
            elif t[-2] == "linear_layer":
                out[k] = a[rowmap][:, rowmap] * colsplit[None, :] if t[-1] == "weight" else a[rowmap]
            else:
                raise KeyError("lifted_model: no rule for " + k)
        elif k in ("model.atomic_energy_output_block.layers.0.weight",
                   "model.partial_charges_output_block.transform_inv_features.0.weight",
                   "model.hirshfeld_output_block.transform_features.0.weight",
                   "model.c6_ratios_output_block.transform_features.0.weight"):
            out[k] = lift_cols(a)
        else:
            out[k] = a  # per-element tables, head outputs, physical constants
    for rec in manifest["tensors"]:
        rec["shape"] = list(np.shape(out[rec["state_key"]]))
    arch["invariant_features"] = F2
    arch["attention_heads"] = F2 // 32
    arch["euclidean_degree_channels"] = S2
    arch["radial_basis_features"] = R
    arch["parameter_elements"] = int(sum(np.asarray(out[r["state_key"]]).size for r in manifest["tensors"]
                                         if r["role"] == "parameter"))
    write_model(str(path), manifest, out)
    return str(path)


def head_width_model(path, width, base=MODEL, live=False):
    """`base` with the energy and charge heads' hidden layer widened to
    `width` units (> F): with the new units' output weights zero (live=False)
    the same function with a head width other than F
    (so3lr_architecture.cpp:444-446); live=True gives them small random output
    weights (another function)."""
    from so3lrxlammps_amd.model_file import read_model, write_model
    manifest, arrays = read_model(base)
    rng = np.random.default_rng(29)
    for pre, w1, b1, w2 in (("model.atomic_energy_output_block.", "layers.0.weight", "layers.0.bias",
                             "final_layer.weight"),
                            ("model.partial_charges_output_block.", "transform_inv_features.0.weight",
                             "transform_inv_features.0.bias", "transform_inv_features.2.weight")):
        W, bb, W2 = arrays[pre + w1], arrays[pre + b1], arrays[pre + w2]
        extra = width - W.shape[0]
        arrays[pre + w1] = np.concatenate([W, 0.1 * rng.standard_normal((extra, W.shape[1]))])
        arrays[pre + b1] = np.concatenate([bb, 0.1 * rng.standard_normal(extra)])
        new = 0.05 * rng.standard_normal((1, extra)) if live else np.zeros((1, extra))
        arrays[pre + w2] = np.concatenate([W2, new], axis=1)
    for rec in manifest["tensors"]:
        rec["shape"] = list(np.shape(arrays[rec["state_key"]]))
    write_model(str(path), manifest, arrays)
    return str(path)


def degrees_model(path, degrees, base=MODEL):
    """`base` (4 degree slots) with the slots' degrees set to `degrees` (four,
    sorted, 1..4, repeats allowed: so3lr_architecture.cpp:246-293), e.g.
    (1, 1, 2, 3) or (1, 2, 3, 3).  Every weight keeps its shape (the slot count
    is unchanged); the equivariant width becomes sum(2l + 1), and the
    Clebsch-Gordan weights, degree repeats and segment tables are those of
    the new degrees (cg = 1/sqrt(2l + 1), as in the shipped model)."""
    from so3lrxlammps_amd.model_file import read_model, write_model
    manifest, arrays = read_model(base)
    assert int(manifest["architecture"]["euclidean_degree_channels"]) == len(degrees) == 4
    reps = [2 * l + 1 for l in degrees]
    seg = np.concatenate([np.full(r, s) for s, r in enumerate(reps)])
    cg = np.concatenate([np.full(r, 1.0 / np.sqrt(r)) for r in reps])
    for k in list(arrays):
        t = k.split(".")
        if not k.startswith("model.euclidean_transformers."):
            continue
        if t[-1] == "degree_repeats":
            arrays[k] = np.array(reps, dtype=np.int64)
        elif t[-1] == "cg_rep":
            arrays[k] = cg.copy()
        elif t[-1] == "segment_ids":
            arrays[k] = seg.astype(arrays[k].dtype)
        elif t[-1] == "segment_sum_matrix":
            arrays[k] = np.eye(len(degrees))[seg]
    for rec in manifest["tensors"]:
        rec["shape"] = list(np.shape(arrays[rec["state_key"]]))
    write_model(str(path), manifest, arrays)
    return str(path)


def zbl_as_nlh(arch, cap=20, terms=(0, 1, 2), garbage_lower=True, seed=3):
    """NLH tables (cap, cap, 3) holding, for every pair (za <= zb), the learned
    ZBL screening terms `terms` (amplitude c_k, rate a_k (za^p + zb^p) d;
    kokkos_physical_zbl.cpp:163-172), zero in unused slots; the unused lower
    triangle (za > zb) holds large random values, so a transposed lookup
    shows."""
    a = np.zeros((cap, cap, 3))
    b = np.zeros((cap, cap, 3))
    rng = np.random.default_rng(seed)
    if garbage_lower:
        lo = np.tril_indices(cap, -1)
        a[lo] = rng.uniform(5, 50, (len(lo[0]), 3))
        b[lo] = rng.uniform(0.1, 1, (len(lo[0]), 3))
    p, d = arch["zbl_p"], arch["zbl_d"]
    for za in range(1, cap + 1):
        for zb in range(za, cap + 1):
            rate = (za ** p + zb ** p) * d
            for slot, k in enumerate(terms):
                a[za - 1, zb - 1, slot] = arch["zbl_c%d" % (k + 1)]
                b[za - 1, zb - 1, slot] = arch["zbl_a%d" % (k + 1)] * rate
    return a, b


SYMBOLS = ["", "H", "He", "Li", "Be", "B", "C", "N", "O", "F", "Ne", "Na", "Mg", "Al",
           "Si", "P", "S", "Cl", "Ar", "K", "Ca"]


def z_of(symbol):
    return SYMBOLS.index(symbol)


def read_lammps_data(path):
    """Return (positions[n,3], types[n], lo[3], hi[3]) sorted by atom id."""
    lines = open(path).read().split("\n")
    lo = np.zeros(3)
    hi = np.zeros(3)
    natoms = 0
    atoms = []
    i = 0
    while i < len(lines):
        s = lines[i].split("#")[0].strip()
        parts = s.split()
        if len(parts) == 2 and parts[1] == "atoms":
            natoms = int(parts[0])
        for a, (l, h) in enumerate((("xlo", "xhi"), ("ylo", "yhi"), ("zlo", "zhi"))):
            if len(parts) == 4 and parts[2] == l and parts[3] == h:
                lo[a], hi[a] = float(parts[0]), float(parts[1])
        if s.startswith("Atoms"):
            i += 1
            while i < len(lines) and not lines[i].split("#")[0].strip():
                i += 1
            while i < len(lines) and len(atoms) < natoms:
                p = lines[i].split("#")[0].split()
                if p:
                    atoms.append((int(p[0]), int(p[1]), float(p[2]), float(p[3]), float(p[4])))
                i += 1
            break
        i += 1
    atoms.sort()
    pos = np.array([[a[2], a[3], a[4]] for a in atoms])
    types = np.array([a[1] for a in atoms])
    return pos, types, lo, hi


def read_molecule(name):
    """(z, positions) of tests/golden/molecules/<name>.data, the element of
    each type read from its mass in the Masses section."""
    from so3lrxlammps_amd.systems import MASS
    path = os.path.join(GOLDEN, "molecules", name + ".data")
    lines = [l.split("#")[0].strip() for l in open(path)]
    k = lines.index("Masses") + 1
    while not lines[k]:
        k += 1
    type_z = {}
    while lines[k]:
        t, mass = lines[k].split()[:2]
        type_z[int(t)] = min(MASS, key=lambda zz: abs(MASS[zz] - float(mass)))
        k += 1
    pos, types, _, _ = read_lammps_data(path)
    return np.array([type_z[int(t)] for t in types], dtype=np.int64), pos


def build_graphs(pos, box=None, rc_sr=4.5, rc_lr=12.0):
    """Brute-force SR full list and LR half list.

    box: None (non-periodic) or a 3-vector of orthogonal periodic lengths.
    Returns sr=(senders, receivers, vectors), lr=(pi, pj, vectors).
    """
    n = len(pos)
    snd, rcv, vec = [], [], []
    pi, pj, pv = [], [], []
    chunk = 512
    for start in range(0, n, chunk):
        idx = np.arange(start, min(n, start + chunk))
        d = pos[None, :, :] - pos[idx, None, :]  # d[a, j] = x_j - x_i
        if box is not None:
            d -= np.round(d / box) * box
        r2 = (d * d).sum(-1)
        for a, i in enumerate(idx):
            # SR full list for receiver i: v = x_i - x_j
            js = np.nonzero((r2[a] > 0.0) & (r2[a] < rc_sr * rc_sr))[0]
            snd.append(js)
            rcv.append(np.full(len(js), i))
            vec.append(-d[a, js])
            # LR half list: j > i
            jl = np.nonzero((r2[a] > 0.0) & (r2[a] < rc_lr * rc_lr))[0]
            jl = jl[jl > i]
            pi.append(np.full(len(jl), i))
            pj.append(jl)
            pv.append(d[a, jl])
    cat = lambda xs, shape=None: (np.concatenate(xs) if xs else np.zeros(0))
    sr = (np.concatenate(snd).astype(np.int64), np.concatenate(rcv).astype(np.int64),
          np.concatenate(vec).reshape(-1, 3))
    lr = (np.concatenate(pi).astype(np.int64), np.concatenate(pj).astype(np.int64),
          np.concatenate(pv).reshape(-1, 3))
    return sr, lr


def load_golden(name):
    """Golden JSON reference plus its geometry: returns (ref, z, pos, box)."""
    import json
    ref = json.load(open(os.path.join(GOLDEN, "refs", "so3lr_%s.json" % name)))
    data = os.path.basename(ref["data"])
    pos, types, lo, hi = read_lammps_data(os.path.join(GOLDEN, "molecules", data))
    z = np.array([z_of(ref["types"][t - 1]) for t in types], dtype=np.int64)
    assert list(z) == list(ref["atomic_numbers"]), name
    box = (hi - lo) if ref["periodic"] else None
    if box is not None:
        pos = lo + np.mod(pos - lo, box)
    return ref, z, pos, box


def graphs_from_lists(lists, x, rc_sr=4.5, rc_lr=12.0):
    """Oracle graphs from the LAMMPS stand-in's candidate lists (ghost rows
    collapsed onto their owners): SR directed edges sender -> receiver with
    v = x_receiver - x_sender, LR unique pairs (i, j) with d = x_j - x_i,
    both cut at the model radii.  For boxes wider than twice the cutoff these
    are the brute-force graphs of build_graphs (test_capi_cpu checks the lists
    against brute force), in LAMMPS list order."""
    xr = lists.rows_positions(x)
    owner = lists.owner.astype(np.int64)
    (il, off, nb), (il2, off2, nb2) = lists.lists
    recv = np.repeat(il.astype(np.int64), np.diff(off))
    v = xr[recv] - xr[nb]
    r2 = (v * v).sum(1)
    m = (r2 > 0.0) & (r2 < rc_sr * rc_sr)
    sr = (owner[nb][m], recv[m], v[m])
    i2 = np.repeat(il2.astype(np.int64), np.diff(off2))
    d = xr[nb2] - xr[i2]
    r2 = (d * d).sum(1)
    m = (r2 > 0.0) & (r2 < rc_lr * rc_lr)
    lr = (i2[m], owner[nb2][m], d[m])
    return sr, lr
