"""HIP path vs the CPU oracle on the architecture options the reference runs
beyond the shipped v1 model (so3lr_capabilities.cpp:54-85): RMSNorm, no
second normalisation, QK normalisation, residual scalars, NLH repulsion, the
C6 ratio head, the message normalisations and other block counts, each on a
model written by support.variant_model and pinned in the oracle by
tests/test_oracle_arch.py.  Same tolerances as test_gpu_parity.py (energies
1e-10 relative, forces 1e-9 eV/A).
"""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle
from test_gpu_parity import _check, _hip_single_point

pytestmark = pytest.mark.gpu


def _tame(blocks):
    """Scale the residual branches (MLP output, interaction layer) by 0.1: a
    trained model without its second LayerNorm grows without bound."""
    def edit(manifest, arrays):
        for b in range(blocks):
            for k in ("mlp_1.3.weight", "mlp_1.3.bias", "interaction_block.linear_layer.weight",
                      "interaction_block.linear_layer.bias"):
                key = "model.euclidean_transformers.%d.%s" % (b, k)
                arrays[key] = 0.1 * arrays[key]
    return edit


def _quiet_filters(blocks):
    """Scale the filters' output layers by 0.1: with unit-RMS q and k rows the
    untrained model's attention logits grow about tenfold per block, and the
    equivariant features with them (forces of thousands of eV/A)."""
    def edit(manifest, arrays):
        for b in range(blocks):
            for fn in ("filter_net_inv.", "filter_net_ev."):
                for k in ("mlp_rbf.mlp_rbf_layer_1.0.weight", "mlp_rbf.mlp_rbf_layer_1.0.bias",
                          "mlp_ev.mlp_ev_layer_1.0.weight", "mlp_ev.mlp_ev_layer_1.0.bias"):
                    key = "model.euclidean_transformers.%d.%s%s" % (b, fn, k)
                    arrays[key] = 0.1 * arrays[key]
    return edit


def _variants():
    arch = Oracle(support.MODEL).model.arch
    return {
        "rms_norm": dict(rms_norm=True),
        "no_norm2": dict(norm2=False, edit=_tame(3)),
        "qk_norm": dict(qk_norm=True, edit=_quiet_filters(3)),
        "qk_norm_wide": dict(qk_norm=True),  # edge invariants up to 1e12: the wide-range SiLU
        "residual_scalars": dict(blocks=4, resid=[0.9, 1.1, 0.8, 1.2], x0=[0.2, -0.3, 0.1, 0.4]),
        "nlh": dict(nlh=support.zbl_as_nlh(arch, terms=(0, 1, 2))),
        "c6_head": dict(c6="perturb"),
        "sqrt_num_features": dict(message_normalization="sqrt_num_features", edit=_quiet_filters(3)),
        "one_block": dict(blocks=1),
        "all": dict(blocks=4, rms_norm=True, qk_norm=True, resid=[0.9, 1.1, 0.8, 1.2],
                    x0=[0.2, -0.3, 0.1, 0.4], nlh=support.zbl_as_nlh(arch, terms=(0, 2, 3), garbage_lower=False),
                    c6="perturb", edit=_quiet_filters(4)),
    }


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("variants")
    return {k: support.variant_model(d / ("%s.so3lr" % k), **v) for k, v in _variants().items()}


CASES = [(v, n) for v in _variants() for n in ("acetate", "water3000") if (v, n) != ("qk_norm_wide", "water3000")]


@pytest.mark.parametrize("variant,name", CASES)
def test_variant_matches_oracle(models, variant, name):
    """Forces within 1e-9 eV/A, relaxed to 1e-10 relative to the largest
    force where an untrained variant's forces exceed 10 eV/A."""
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden(name)
    q, m = ref.get("charge", 0), ref.get("multiplicity", 1)
    print("case", variant, name, flush=True)
    ctx = Context(models[variant], 0)
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, q, m)
    ctx.close()
    sr, lr = support.build_graphs(pos, box)
    out = Oracle(models[variant]).evaluate(z, sr, lr, charge=q, multiplicity=m)
    _check(out, e, f, ea, w, terms, ftol=1e-9 * max(1.0, np.abs(out["forces"]).max() / 10.0))


def test_variant_scalar_filter_path(models, monkeypatch):
    """The scalar filter kernels (SO3LR_NAIVE_FILTERS=1) with every option on."""
    from so3lrxlammps_amd import Context
    ref, z, pos, box = support.load_golden("acetate")
    monkeypatch.setenv("SO3LR_NAIVE_FILTERS", "1")
    ctx = Context(models["all"], 0)
    e, f, ea, w, terms = _hip_single_point(ctx, z, pos, box, -1, 1)
    ctx.close()
    out = Oracle(models["all"]).evaluate(z, *support.build_graphs(pos, box), charge=-1, multiplicity=1)
    _check(out, e, f, ea, w, terms)


def test_variant_device_path_and_replay(models):
    """so3lr_reneighbor_device + so3lr_compute_device (spatial node order,
    graph replay on the repeated call) with every option on: bitwise equal
    across replays and equal to the rows path."""
    import torch
    from so3lrxlammps_amd import Context, Lists
    ref, z, pos, box = support.load_golden("water3000")
    print("case all device path", flush=True)
    ctx = Context(models["all"], 0)
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
