"""The oracle's architecture options (the operators the reference runs beyond
the shipped v1 model: so3lr_capabilities.cpp:54-85) pinned on the CPU.

No reference fixture exists for any of them (the reference ships golden
vectors for the v1 model only), so each option is pinned by what the
mathematics fixes, on models written by support.variant_model:

* RMSNorm and the QK normalisation: orc_rms_rows against the closed form
  x / sqrt(mean x^2 + eps), unit RMS of its rows, and its scaling law;
* residual scalars: (1, 0) in every block reproduces v1 bit for bit; a
  block-0 pair (a, b) equals the v1 model with the embedding scale divided by
  a + b; resid[1] = c equals block 0's second LayerNorm scaled by c; x0[1] = d
  on a one-element system equals block 0's second LayerNorm bias shifted by
  d x_embedding;
* message normalisation: identity and sqrt_num_features equal the v1 model
  with avg_num_neighbors 1 and sqrt(32);
* NLH repulsion: tables holding learned ZBL's terms 1-3 plus tables holding
  its term 4 give per-atom repulsion energies that add up to learned ZBL's
  (the lower triangle holds garbage, so a transposed lookup fails);
* the C6 ratio head: a copy of the Hirshfeld head gives ratios equal to the
  Hirshfeld ratios; with element-constant ratio heads, C6 ratios c = h^2
  give v1's energy and forces (C6 = C6_ref h^2 either way);
* every reverse path: forces and virial equal central finite differences of
  the energy on two models that switch all options on between them.
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle, rms_rows


@pytest.fixture(scope="module")
def tmp(tmp_path_factory):
    return tmp_path_factory.mktemp("variants")


@pytest.fixture(scope="module")
def v1():
    return Oracle(support.MODEL)


def _acetate():
    ref, z, pos, box = support.load_golden("acetate")
    return z, pos, ref.get("charge", 0), ref.get("multiplicity", 1)


def _run(orc, z, pos, q=0, m=1, box=None):
    return orc.evaluate(z, *support.build_graphs(pos, box), charge=q, multiplicity=m)


def _carbon_cluster(n=10, seed=4):
    """n carbon atoms, random, at least 1.3 A apart, within 4 A."""
    rng = np.random.default_rng(seed)
    pts = []
    while len(pts) < n:
        p = rng.uniform(-2.0, 2.0, 3)
        if all(np.linalg.norm(p - o) > 1.3 for o in pts):
            pts.append(p)
    return np.full(n, 6), np.array(pts)


def _close(a, b, rtol=1e-12, atol=1e-12):
    a, b = np.asarray(a), np.asarray(b)
    return np.max(np.abs(a - b)) <= atol + rtol * np.max(np.abs(b))


# ------------------------------------------------------------- RMS rows
def test_rms_rows_closed_form_and_unit_rms():
    rng = np.random.default_rng(1)
    for width, eps in ((128, 1e-6), (32, 1e-6), (7, 0.3)):
        x = rng.normal(size=(9, width)) * rng.uniform(0.01, 10.0, (9, 1))
        y, r = rms_rows(x, eps)
        ms = (x * x).mean(axis=1)
        assert np.allclose(y, x / np.sqrt(ms + eps)[:, None], rtol=1e-14, atol=0)
        assert np.allclose(r, 1.0 / np.sqrt(ms + eps), rtol=1e-14, atol=0)
        # rows of unit RMS up to the eps share: mean(y^2) = ms / (ms + eps)
        assert np.allclose((y * y).mean(axis=1), ms / (ms + eps), rtol=1e-13, atol=0)
        # scaling law: x -> c x with eps -> c^2 eps leaves y unchanged
        y2, r2 = rms_rows(3.0 * x, 9.0 * eps)
        assert np.allclose(y2, y, rtol=1e-14, atol=1e-15) and np.allclose(3.0 * r2, r, rtol=1e-14)


# ------------------------------------------------------- residual scalars
def test_residual_scalars_one_zero_reduce_to_v1(tmp, v1):
    z, pos, q, m = _acetate()
    orc = Oracle(support.variant_model(tmp / "r10.so3lr", resid=[1.0, 1.0, 1.0], x0=[0.0, 0.0, 0.0]))
    a, b = _run(orc, z, pos, q, m), _run(v1, z, pos, q, m)
    for k in ("energy", "forces", "virial", "charges", "hirshfeld", "eatom"):
        assert np.array_equal(a[k], b[k]), k


def test_block0_residual_pair_is_an_embedding_scale(tmp):
    z, pos, q, m = _acetate()
    a_, b_ = 0.7, 0.45
    orc = Oracle(support.variant_model(tmp / "r0.so3lr", resid=[a_, 1.0, 1.0], x0=[b_, 0.0, 0.0]))

    def scale(manifest, arrays):
        manifest["architecture"]["embedding_scale"] /= (a_ + b_)
    ref = Oracle(support.variant_model(tmp / "r0ref.so3lr", edit=scale))
    A, B = _run(orc, z, pos, q, m), _run(ref, z, pos, q, m)
    assert _close(A["energy"], B["energy"]) and _close(A["forces"], B["forces"], 1e-10, 1e-11)
    assert abs(A["energy"] - _run(Oracle(support.MODEL), z, pos, q, m)["energy"]) > 1e-3  # the scalars matter


def test_later_residual_scalar_is_a_layer_norm_scale(tmp):
    z, pos, q, m = _acetate()
    c = 0.8
    orc = Oracle(support.variant_model(tmp / "r1.so3lr", resid=[1.0, c, 1.0], x0=[0.0, 0.0, 0.0]))

    def scale_ln2(manifest, arrays):
        for w in ("weight", "bias"):
            arrays["model.euclidean_transformers.0.layer_norm_inv_2." + w] = \
                c * arrays["model.euclidean_transformers.0.layer_norm_inv_2." + w]
    ref = Oracle(support.variant_model(tmp / "r1ref.so3lr", edit=scale_ln2))
    A, B = _run(orc, z, pos, q, m), _run(ref, z, pos, q, m)
    assert _close(A["energy"], B["energy"]) and _close(A["forces"], B["forces"], 1e-10, 1e-11)
    assert _close(A["virial"], B["virial"], 1e-10, 1e-11)


def test_later_x0_scalar_is_a_layer_norm_bias_on_one_element(tmp):
    z, pos = _carbon_cluster()
    d = 0.3
    orc = Oracle(support.variant_model(tmp / "x1.so3lr", resid=[1.0, 1.0, 1.0], x0=[0.0, d, 0.0]))
    model = Oracle(support.MODEL).model
    # the embedding of carbon (no charge/spin offset at Q = 0, M = 1)
    x_emb = model["model.inv_feature_embedding.embedding.weight"][:, 5] / model.arch["embedding_scale"]

    def shift_bias(manifest, arrays):
        k = "model.euclidean_transformers.0.layer_norm_inv_2.bias"
        arrays[k] = arrays[k] + d * x_emb
    ref = Oracle(support.variant_model(tmp / "x1ref.so3lr", edit=shift_bias))
    A, B = _run(orc, z, pos), _run(ref, z, pos)
    assert _close(A["energy"], B["energy"]) and _close(A["forces"], B["forces"], 1e-10, 1e-11)


# -------------------------------------------------- message normalisation
@pytest.mark.parametrize("kind,value", [("identity", 1.0), ("sqrt_num_features", float(np.sqrt(32.0)))])
def test_message_normalisation_kinds(tmp, kind, value):
    z, pos, q, m = _acetate()
    orc = Oracle(support.variant_model(tmp / ("mn_%s.so3lr" % kind), message_normalization=kind))

    def avg(manifest, arrays):
        manifest["architecture"]["avg_num_neighbors"] = value
    ref = Oracle(support.variant_model(tmp / ("mnref_%s.so3lr" % kind), edit=avg))
    A, B = _run(orc, z, pos, q, m), _run(ref, z, pos, q, m)
    assert A["energy"] == B["energy"] and np.array_equal(A["forces"], B["forces"])


# ---------------------------------------------------------------- NLH
def test_nlh_tables_add_up_to_learned_zbl(tmp, v1):
    z, pos, q, m = _acetate()
    arch = v1.model.arch
    t1 = Oracle(support.variant_model(tmp / "nlh1.so3lr", nlh=support.zbl_as_nlh(arch, terms=(0, 1, 2))))
    t2 = Oracle(support.variant_model(tmp / "nlh2.so3lr", nlh=support.zbl_as_nlh(arch, terms=(3,))))
    e1, e2, e0 = (_run(o, z, pos, q, m)["e_zbl"] for o in (t1, t2, v1))
    assert np.max(np.abs(e0)) > 1e-3
    assert _close(e1 + e2, e0, 1e-12, 1e-14)


# ---------------------------------------------------------------- C6 head
def test_c6_head_copy_gives_the_hirshfeld_ratios(tmp):
    z, pos, q, m = _acetate()
    out = _run(Oracle(support.variant_model(tmp / "c6copy.so3lr", c6="copy")), z, pos, q, m)
    assert np.array_equal(out["c6_ratios"], out["hirshfeld"])


def test_c6_ratios_equal_to_h_squared_reduce_to_v1(tmp):
    z, pos, q, m = _acetate()
    # element-constant ratio heads: zero queries leave |v_shift[z]|
    def hirsh_const(manifest, arrays):
        arrays["model.hirshfeld_output_block.q_embedding.weight"] = \
            np.zeros_like(arrays["model.hirshfeld_output_block.q_embedding.weight"])
    base = support.variant_model(tmp / "hconst.so3lr", edit=hirsh_const)
    Oracle(base)
    from so3lrxlammps_amd.model_file import read_model
    _, arrays = read_model(base)
    h = arrays["model.hirshfeld_output_block.v_shift_embedding.weight"]
    head = {s: arrays["model.hirshfeld_output_block." + s].copy() for s in
            ("q_embedding.weight", "transform_features.0.weight", "transform_features.0.bias",
             "transform_features.2.weight", "transform_features.2.bias")}
    head["v_shift_embedding.weight"] = h * h
    with_c6 = Oracle(support.variant_model(tmp / "c6sq.so3lr", base=base, c6=head))
    A, B = _run(with_c6, z, pos, q, m), _run(Oracle(base), z, pos, q, m)
    assert np.allclose(A["c6_ratios"], B["hirshfeld"] ** 2, rtol=1e-15)
    assert abs(A["e_disp_total"]) > 1e-4
    assert _close(A["energy"], B["energy"]) and _close(A["forces"], B["forces"], 1e-11, 1e-12)


# ------------------------------------------------ finite differences
def _all_options_a(tmp, v1):
    return support.variant_model(tmp / "fd_a.so3lr", blocks=4, rms_norm=True, qk_norm=True,
                                 resid=[0.9, 1.1, 0.8, 1.2], x0=[0.2, -0.3, 0.1, 0.4],
                                 nlh=support.zbl_as_nlh(v1.model.arch, terms=(0, 2, 3), garbage_lower=False),
                                 c6="perturb")


def _all_options_b(tmp):
    # Without the second LayerNorm the trained residual stream grows without
    # bound, so the block's residual branches (MLP output, interaction layer)
    # are scaled by 0.1 to keep the energy finite.  (The message
    # normalisations are equivalences of the avg_num_neighbors value, pinned
    # above.)
    def tame(manifest, arrays):
        for b in range(2):
            for k in ("mlp_1.3.weight", "mlp_1.3.bias", "interaction_block.linear_layer.weight",
                      "interaction_block.linear_layer.bias"):
                key = "model.euclidean_transformers.%d.%s" % (b, k)
                arrays[key] = 0.1 * arrays[key]
    return support.variant_model(tmp / "fd_b.so3lr", blocks=2, norm2=False, resid=[1.05, 0.9], x0=[-0.1, 0.25],
                                 qk_norm=True, edit=tame)


@pytest.mark.parametrize("which", ["a", "b"])
def test_option_models_forces_finite_difference(tmp, v1, which):
    z, pos, q, m = _acetate()
    orc = Oracle(_all_options_a(tmp, v1) if which == "a" else _all_options_b(tmp))
    out = _run(orc, z, pos, q, m)
    assert abs(out["energy"] - _run(v1, z, pos, q, m)["energy"]) > 1e-2
    h = 1e-4
    for i in (0, 2, 5):
        for a in range(3):
            p1 = pos.copy(); p1[i, a] += h
            p2 = pos.copy(); p2[i, a] -= h
            fd = -(_run(orc, z, p1, q, m)["energy"] - _run(orc, z, p2, q, m)["energy"]) / (2 * h)
            assert abs(fd - out["forces"][i, a]) < 2e-6, (i, a, fd, out["forces"][i, a])


def test_option_model_virial_finite_difference(tmp, v1):
    from test_oracle_math import _small_periodic
    z, pos, box = _small_periodic(n_mol=12)
    orc = Oracle(_all_options_a(tmp, v1))
    sr, lr = support.build_graphs(pos, box)
    out = orc.evaluate(z, sr, lr)
    h = 1e-5
    for k, (a, b) in enumerate([(0, 0), (1, 1), (2, 2), (0, 1), (0, 2), (1, 2)]):
        S = np.zeros((3, 3)); S[a, b] += 0.5; S[b, a] += 0.5
        es = []
        for t in (h, -h):
            M = np.eye(3) + t * S
            es.append(orc.evaluate(z, (sr[0], sr[1], sr[2] @ M.T), (lr[0], lr[1], lr[2] @ M.T))["energy"])
        dEdt = (es[0] - es[1]) / (2 * h)
        assert abs(-dEdt - out["virial"][k]) < 2e-6 * max(1.0, abs(out["virial"][k])), (k, -dEdt, out["virial"][k])
