"""HIP path vs the CPU oracle at the widths beyond v1 that the reference runs
(so3lr_capabilities.cpp:54-85): F = 256 (8 heads, 8 degree slots), R = 64,
duplicated degree slots, energy/charge heads narrower than F, and duplicated
or missing degrees at F = 128.  These models run on the generic kernels
(csrc/generic.hip).  The oracle at these widths is pinned by
tests/test_oracle_wide.py.  Same tolerances as test_gpu_parity.py.
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle
from test_gpu_parity import _check, _hip_single_point

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("wide")
    from test_gpu_arch import _variants
    # every option on, filters quietened as in test_gpu_arch (the untrained
    # model's attention logits otherwise give forces of 10^4 eV/A on water)
    options = support.variant_model(d / "options.so3lr", **_variants()["all"])
    lift = support.lifted_model(d / "lift.so3lr")
    return {
        "lift": lift,
        # the lift with every weight perturbed: the two copies no longer agree
        "lift_perturbed": support.perturbed_model(d / "lift_p.so3lr", seed=23, scale=0.2, base=lift),
        "lift_options": support.lifted_model(d / "lift_opt.so3lr", base=options),
        "deg1123": support.degrees_model(d / "d1123.so3lr", (1, 1, 2, 3)),
        "deg1233": support.degrees_model(d / "d1233.so3lr", (1, 2, 3, 3)),
        # the other accepted width combinations (tests/test_oracle_wide.py)
        "f128_r64": support.lifted_model(d / "r64.so3lr", copies=1, R=64),
        "f256_r32": support.lifted_model(d / "f256r32.so3lr", copies=2, R=32),
        "head_width_192": support.head_width_model(d / "hk192_live.so3lr", 192, live=True),
    }


CASES = [(m, n) for m in ("lift", "lift_perturbed", "lift_options", "deg1123", "deg1233")
         for n in ("acetate", "alanine_cation", "water3000")]
CASES += [(m, n) for m in ("f128_r64", "f256_r32", "head_width_192") for n in ("acetate", "water3000")]


@pytest.mark.parametrize("model,name", CASES)
def test_wide_model_matches_oracle(models, model, name):
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden(name)
    q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
    print("case", model, name, flush=True)
    ctx = Context(models[model], 0)
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, q, m)
    ctx.close()
    out = Oracle(models[model]).evaluate(z, *support.build_graphs(pos, box), charge=q, multiplicity=m)
    _check(out, e, f, ea, w, terms, ftol=1e-9 * max(1.0, np.abs(out["forces"]).max() / 10.0))


def test_lift_on_the_gpu_equals_the_v1_model(models):
    """The lift computes the v1 model's function: the generic kernels on it
    agree with the fused v1 kernels on the shipped model."""
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden("water3000")
    res = []
    for path in (models["lift"], support.MODEL):
        ctx = Context(path, 0)
        res.append(_hip_single_point(ctx, z, pos, box, 0, 1))
        ctx.close()
    (e1, f1, _, w1, _), (e0, f0, _, w0, _) = res
    assert abs(e1 - e0) <= 1e-11 * abs(e0)
    assert np.abs(f1 - f0).max() <= 1e-9
    assert np.abs(w1 - w0).max() <= 1e-9 * max(1.0, np.abs(w0).max())


@pytest.mark.parametrize("model,name", [("lift_perturbed", "water3000"), ("lift_options", "alanine_cation"),
                                        ("deg1123", "acetate")])
def test_wide_block0_element_tables_match_full_filters(monkeypatch, models, model, name):
    """Block 0 through the element-pair tables on the generic kernels (one
    image: 2, 4 and 3 elements here) against the full filter GEMMs
    (SO3LR_NO_CLASS_TABLES=1): equal to rounding."""
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden(name)
    q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
    res = []
    for off in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_CLASS_TABLES", off)
        ctx = Context(models[model], 0)
        res.append(_hip_single_point(ctx, z, pos, box, q, m))
        ctx.close()
    (e1, f1, ea1, w1, _), (e2, f2, ea2, w2, _) = res
    print("%s %s: |dE| %.2e max|dF| %.2e" % (model, name, abs(e1 - e2), np.abs(f1 - f2).max()), flush=True)
    assert abs(e1 - e2) <= 1e-12 * abs(e2)
    assert np.abs(f1 - f2).max() <= 1e-10 * max(1.0, np.abs(f2).max() / 10.0)
    assert np.abs(w1 - w2).max() <= 1e-10 * max(1.0, np.abs(w2).max())


@pytest.mark.parametrize("model,name", [("lift", "water3000"), ("lift_perturbed", "alanine_cation"),
                                        ("f128_r64", "acetate"), ("deg1123", "water3000")])
def test_wide_block0_radial_tables_match_element_tables(monkeypatch, models, model, name):
    """Every block on its radial tables (the default) against the
    element-pair MFMA kernels and the full fused filter chains
    (SO3LR_NO_RADIAL_TABLES=1) on the generic kernels, 8 and 4 heads: equal
    to rounding, and the kernel timings show which path ran."""
    from so3lrxlammps_amd import Context, Lists
    from test_gpu_parity import _launches
    ref, z, pos, box = support.load_golden(name)
    q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
    if box is None:
        lo, hi, per = pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0)
    else:
        lo, hi, per = np.zeros(3), box, (1, 1, 1)
    res = []
    for off in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_RADIAL_TABLES", off)
        c = Context(models[model], 0)
        c.kernel_timing(True)
        c.set_system(z, q, m)
        lists = Lists(pos, lo, hi, per)
        c.set_topology(lists)
        e, f, ea, w = c.compute(lists.rows_positions(pos))
        ran = {k: _launches(c, "generic_filter_%s_block0_%s" % (k[0], k[1]))
               for k in (("fwd", "radial"), ("bwd", "radial"), ("fwd", "tables"), ("bwd", "tables"))}
        ran.update({k: _launches(c, "generic_filter_" + k) for k in ("fwd_radial", "bwd_radial", "fwd", "bwd")})
        res.append((e, f.copy(), w.copy(), ran))
        c.close()
    (e1, f1, w1, ran1), (e2, f2, w2, ran2) = res
    print("%s %s: |dE| %.2e max|dF| %.2e max|dW| %.2e" % (model, name, abs(e1 - e2), np.abs(f1 - f2).max(),
                                                          np.abs(w1 - w2).max()), flush=True)
    assert ran1[("fwd", "tables")] == 1 and ran1[("fwd", "radial")] == 0
    assert ran2[("fwd", "radial")] == 1 and ran2[("bwd", "radial")] == 1
    assert ran2[("fwd", "tables")] == 0 and ran2[("bwd", "tables")] == 0
    # the blocks after 0 (two): their radial tables where every fit holds its
    # bound (the perturbed lift's need not: then the full fused chains), or
    # the full chains
    assert ran2["fwd_radial"] + ran2["fwd"] == 2 and ran2["bwd_radial"] + ran2["bwd"] == 2
    assert ran2["fwd_radial"] in (0, 2) and ran2["fwd_radial"] == ran2["bwd_radial"]
    if model != "lift_perturbed":
        assert ran2["fwd_radial"] == 2
    assert ran1["fwd"] == 2 and ran1["bwd"] == 2 and ran1["fwd_radial"] == 0
    assert abs(e1 - e2) <= 1e-12 * abs(e2)
    assert np.abs(f1 - f2).max() <= 1e-10 * max(1.0, np.abs(f2).max() / 10.0)
    assert np.abs(w1 - w2).max() <= 1e-10 * max(1.0, np.abs(w2).max())


@pytest.mark.parametrize("count", [16, 17])
def test_wide_element_table_limit(monkeypatch, models, count):
    """The generic kernels at the table path's limit (perturbed lift, a
    240-atom cluster): 16 elements (136 element pairs) run block 0 through
    the tables, equal to the full filters to rounding; 17 fall back to the
    full filters, bit for bit the SO3LR_NO_CLASS_TABLES=1 result; both
    against the oracle."""
    from so3lrxlammps_amd import Context, Lists
    from test_gpu_parity import _ELEMENTS17, _cluster
    z, pos, mult = _cluster(_ELEMENTS17[:count])
    print("case lift_perturbed cluster of %d elements" % count, flush=True)
    lists = Lists(pos, pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0))
    res = []
    for off in ("1", "0"):
        monkeypatch.setenv("SO3LR_NO_CLASS_TABLES", off)
        c = Context(models["lift_perturbed"], 0)
        c.set_system(z, 0, mult)
        c.set_topology(lists)
        e, f, ea, w = c.compute(lists.rows_positions(pos))
        res.append((e, f.copy(), w.copy()))
        c.close()
    (e1, f1, w1), (e2, f2, w2) = res
    print("%d elements: |dE| %.2e max|dF| %.2e" % (count, abs(e1 - e2), np.abs(f1 - f2).max()), flush=True)
    if count == 17:
        assert e1 == e2 and np.array_equal(f1, f2) and np.array_equal(w1, w2)
    else:
        assert abs(e1 - e2) <= 1e-12 * abs(e2)
        assert np.abs(f1 - f2).max() <= 1e-10 * max(1.0, np.abs(f2).max() / 10.0)
    out = Oracle(models["lift_perturbed"]).evaluate(z, *support.build_graphs(pos, None), charge=0,
                                                    multiplicity=mult)
    ftol = 1e-9 * max(1.0, np.abs(out["forces"]).max() / 10.0)
    assert abs(e2 - out["energy"]) <= 1e-10 * abs(out["energy"])
    assert np.abs(f2 - out["forces"]).max() <= ftol
    assert np.abs(w2 - out["virial"]).max() <= 1e-9 * max(1.0, np.abs(out["virial"]).max())


def test_wide_device_path_and_replay(models):
    """so3lr_reneighbor_device + so3lr_compute_device on the perturbed lift:
    bitwise equal across graph replays and equal to the rows path."""
    import torch
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden("water3000")
    print("case lift_perturbed device path", flush=True)
    ctx = Context(models["lift_perturbed"], 0)
    ctx.set_system(z, 0, 1)
    lists = Lists(pos, np.zeros(3), box, (1, 1, 1))
    ctx.set_topology(lists)
    e0, f0, _, w0 = ctx.compute(lists.rows_positions(pos))
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    runs = []
    with torch.cuda.stream(stream):
        x = torch.tensor(pos, dtype=torch.float64, device=dev)
        f = torch.zeros_like(x)
        ctx.reneighbor_device(x, np.zeros(3), box, (1, 1, 1), 1.0, stream=stream.cuda_stream)
        for _ in range(3):
            e, w = ctx.compute_device(x, f, stream=stream.cuda_stream)
            stream.synchronize()
            runs.append((e, w.copy(), f.cpu().numpy().copy()))
    ctx.close()
    for e, w, ff in runs[1:]:
        assert e == runs[0][0] and np.array_equal(w, runs[0][1]) and np.array_equal(ff, runs[0][2])
    assert abs(runs[0][0] - e0) <= 1e-11 * abs(e0)
    assert np.abs(runs[0][2] - f0).max() <= 1e-10
    assert np.abs(runs[0][1] - w0).max() <= 1e-10 * max(1.0, np.abs(w0).max())


def test_wide_packed_images(models):
    """64 config-2 molecules as packed images (each with its own (Q, M)) on
    the perturbed lift: per-image charge correction and embedding on the
    generic kernels, rows path against the oracle."""
    from so3lrxlammps_amd import Context, Lists, systems
    from test_gpu_configs import _check as check_config
    z, x, offs, qs, ms, extent = systems.packed_molecules(n_mol=64)
    print("case lift_perturbed packed images: %d atoms in %d images" % (len(z), len(qs)), flush=True)
    img = np.repeat(np.arange(len(qs)), np.diff(offs))
    sr, lr = support.build_graphs(x, None)
    out = Oracle(models["lift_perturbed"]).evaluate(z, sr, lr, image=img, image_charge=qs, image_multiplicity=ms)
    c = Context(models["lift_perturbed"], 0)
    c.set_images(z, offs, qs, ms)
    lists = Lists(x, np.zeros(3), np.full(3, extent), (0, 0, 0))
    c.set_topology(lists)
    e, f, ea, w = c.compute(lists.rows_positions(x))
    check_config(e, f, w, out)
    t = c.terms()
    c.close()
    assert np.abs(t["image_energy"] - out["image_energy"]).max() <= 1e-10 * np.abs(out["image_energy"]).max()
    for k in range(len(qs)):
        assert abs(t["charges"][offs[k]:offs[k + 1]].sum() - qs[k]) < 1e-12
