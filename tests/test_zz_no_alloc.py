"""so3lr_compute_device_noalloc (no counterpart in the reference: the entry
point for callers that cannot allocate device memory) against
so3lr_compute_device on the same inputs, through the C ABI.

Both run the same kernels in the same order, so the results must agree bit
for bit.  Two no-allocation calls in a row, the second on a smaller system,
so the second call runs on the first call's leftover contents of the shared
static array; then a system too large for the array is refused.  The
refusal comes from the size check of the work space, after the steps that
size it (the spatial node order of a new topology and the count of the
pairs inside the cutoff) and before any of the evaluation's own kernels."""
import numpy as np
import pytest

import support

pytestmark = pytest.mark.gpu


# the device's free memory may move by the allocator's granularity for
# reasons of its own; a hipMalloc of any work buffer of these systems would
# take at least this much
FREE_SLACK = 2 << 20


def _evaluate(ctx, x, n, noalloc, stream, reneighbor=None, free_check=False):
    """One evaluation on `stream`; with free_check, the device's free memory
    (hipMemGetInfo) is read right before and after the call, with every
    tensor of the call allocated before, and must not drop."""
    import torch
    dev = torch.device("cuda:0")
    with torch.cuda.stream(stream):
        xt = torch.tensor(x, dtype=torch.float64, device=dev)
        if reneighbor is not None:
            lo, hi, per = reneighbor
            ctx.reneighbor_device(xt, lo, hi, per, 1.0, stream=stream.cuda_stream)
        ft = torch.full((n, 3), float("nan"), dtype=torch.float64, device=dev)
        et = torch.full((n,), float("nan"), dtype=torch.float64, device=dev)
        fn = ctx.compute_device_noalloc if noalloc else ctx.compute_device
        if free_check:
            stream.synchronize()
            free0 = torch.cuda.mem_get_info(dev)[0]
        e, w = fn(xt, ft, et, stream=stream.cuda_stream)
        stream.synchronize()
        if free_check:
            free1 = torch.cuda.mem_get_info(dev)[0]
            print("  free device memory %d -> %d bytes" % (free0, free1), flush=True)
            assert free1 >= free0 - FREE_SLACK, (free0, free1)
        return e, np.asarray(w), ft.cpu().numpy(), et.cpu().numpy()


def _same(a, b, what):
    ea, wa, fa, eta = a
    eb, wb, fb, etb = b
    assert ea == eb, (what, ea, eb)
    assert np.array_equal(wa, wb), (what, wa, wb)
    assert np.array_equal(fa, fb), (what, np.abs(fa - fb).max())
    assert np.array_equal(eta, etb), (what, np.abs(eta - etb).max())
    assert np.isfinite(fa).all() and np.isfinite(eta).all(), what


def test_noalloc_matches_compute_device():
    import torch
    from so3lrxlammps_amd import Context, Lists, _lib, systems
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)

    # call 1: 16 packed config-2 molecules (rows path, each with its own (Q, M))
    z, x, offs, qs, ms, _ = systems.packed_molecules(n_mol=16)
    print("noalloc call 1: %d atoms, 16 packed molecules, rows path" % len(z), flush=True)
    c1 = Context(support.MODEL, 0)
    c1.set_images(z, offs, qs, ms)
    lists = Lists(x, x.min(0) - 20.0, x.max(0) + 20.0, (0, 0, 0))
    c1.set_topology(lists)
    xr = lists.rows_positions(x)
    ref1 = _evaluate(c1, xr, len(z), False, stream)
    got1 = _evaluate(c1, xr, len(z), True, stream)
    _same(got1, ref1, "packed molecules")
    # per-atom terms are not kept by the no-allocation call
    with pytest.raises(_lib.SO3LRError) as err:
        c1.terms()
    assert err.value.code == _lib.ERR_STATE

    # call 2, smaller: the acetate anion on the device-reneighbor path (spatial
    # node order inside), in a second context on the same device
    ref, za, pa, _ = support.load_golden("acetate")
    print("noalloc call 2: %d atoms, acetate, device reneighbor path" % len(za), flush=True)
    c2 = Context(support.MODEL, 0)
    c2.set_system(za, -1, 1)
    box = (pa.min(0) - 20.0, pa.max(0) + 20.0, (0, 0, 0))
    got2 = _evaluate(c2, pa, len(za), True, stream, reneighbor=box)
    ref2 = _evaluate(c2, pa, len(za), False, stream, reneighbor=box)
    _same(got2, ref2, "acetate")

    # the first context again: its retained path still agrees after both
    # no-allocation calls wrote the shared array
    again = _evaluate(c1, xr, len(z), False, stream)
    _same(again, ref1, "packed molecules, retained path after the no-allocation calls")

    # a system larger than the static array: refused at the work-space size
    # check, after the node order and the pair count that size it and before
    # the evaluation's own kernels
    _, zw, pw, bw = support.load_golden("water3000")
    print("noalloc oversize: %d atoms, expect a refusal" % len(zw), flush=True)
    c3 = Context(support.MODEL, 0)
    c3.set_system(zw, 0, 1)
    lw = Lists(pw, np.zeros(3), bw, (1, 1, 1))
    c3.set_topology(lw)
    with torch.cuda.stream(stream):
        xt = torch.tensor(lw.rows_positions(pw), dtype=torch.float64, device=dev)
        ft = torch.zeros((len(zw), 3), dtype=torch.float64, device=dev)
        with pytest.raises(_lib.SO3LRError) as err:
            c3.compute_device_noalloc(xt, ft, stream=stream.cuda_stream)
        stream.synchronize()
    assert err.value.code == _lib.ERR_ARGUMENT and "bytes of work space" in str(err.value)
    for c in (c1, c2, c3):
        c.close()


def test_noalloc_generic_widths(tmp_path):
    """The same agreement for a model on the generic kernels (F = 256, R = 64,
    duplicated degrees: support.lifted_model, weights perturbed), two calls
    in a row, the second smaller, each the first evaluation of its topology."""
    import torch
    from so3lrxlammps_amd import Context, Lists
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    path = support.perturbed_model(tmp_path / "wide_p.so3lr", seed=23, scale=0.2,
                                   base=support.lifted_model(tmp_path / "wide.so3lr"))
    ctx = Context(path, 0)
    for k, name in enumerate(("alanine_cation", "acetate")):
        ref, z, pos, _ = support.load_golden(name)
        print("noalloc generic widths: %s, %d atoms" % (name, len(z)), flush=True)
        ctx.set_system(z, ref.get("charge", 0), ref.get("multiplicity", 1))
        lists = Lists(pos, pos.min(0) - 20.0, pos.max(0) + 20.0, (0, 0, 0))
        ctx.set_topology(lists)
        xr = lists.rows_positions(pos)
        # the first evaluation of the topology (it also sets the spatial node
        # order) is the no-allocation one: the library's device memory does
        # not grow, by its own tally and by the device's free memory (read
        # from the second case on, once the first has loaded every kernel's
        # code)
        held = ctx.device_bytes()
        got = _evaluate(ctx, xr, len(z), True, stream, free_check=k > 0)
        assert ctx.device_bytes() == held, name
        want = _evaluate(ctx, xr, len(z), False, stream)
        _same(got, want, name)
    ctx.close()


def test_noalloc_capacity_overflow_reevaluates():
    """The active-pair capacity of a topology is counted at its first
    evaluation (plus 1/8 and 256); a later geometry with more pairs inside
    the cutoff makes the evaluation grow it and run again.  On the
    no-allocation path the second run carves the static array again at the
    new capacity.  16 packed molecules, lists built at their geometry: the
    first no-allocation call at the positions stretched by 10 % (2,489 pairs
    inside 4.5 A, capacity 3,056), the second compressed to 90 % (3,149
    pairs, counted on the CPU from the same candidates).  The second result
    must equal, bit for bit, a retained-path context whose first evaluation
    is that compressed geometry."""
    import torch
    from so3lrxlammps_amd import Context, Lists, systems
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    z, x, offs, qs, ms, _ = systems.packed_molecules(n_mol=16)
    lists = Lists(x, x.min(0) - 20.0, x.max(0) + 20.0, (0, 0, 0))
    xr = lists.rows_positions(x)
    stretched, compressed = np.ascontiguousarray(xr * 1.1), np.ascontiguousarray(xr * 0.9)
    a = Context(support.MODEL, 0)
    a.set_images(z, offs, qs, ms)
    a.set_topology(lists)
    print("noalloc overflow: %d atoms, stretched then compressed" % len(z), flush=True)
    _evaluate(a, stretched, len(z), True, stream)
    n0 = a.graph_stats()[0]
    got = _evaluate(a, compressed, len(z), True, stream)
    n1 = a.graph_stats()[0]
    print("  active pairs %d -> %d (capacity %d)" % (n0, n1, n0 + n0 // 8 + 256), flush=True)
    assert n1 > n0 + n0 // 8 + 256  # the compressed geometry overflowed the capacity
    b = Context(support.MODEL, 0)
    b.set_images(z, offs, qs, ms)
    b.set_topology(lists)
    want = _evaluate(b, compressed, len(z), False, stream)
    _same(got, want, "compressed after stretched, no-allocation path")
    a.close()
    b.close()
