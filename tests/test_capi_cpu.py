"""Host-side checks of the C ABI that need no GPU: the library loads and
exports every declared symbol, the element map, model integrity and
capability refusals (the model is read before any device is touched)."""
import hashlib
import json
import os
import re
import struct

import numpy as np
import pytest

import support
from so3lrxlammps_amd import _lib

INCLUDE = os.path.join(support.REPO, "include")


def _declared(header):
    text = open(os.path.join(INCLUDE, header)).read()
    return sorted(set(re.findall(r"\b(so3lr_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("so3lr_hip.h", _lib.HIP_LIB), ("so3lr_lammps_emu.h", _lib.EMU_LIB)])
def test_library_exports_declared_symbols(header, lib):
    import ctypes
    handle = ctypes.CDLL(lib)
    names = _declared(header)
    assert names
    for name in names:
        assert hasattr(handle, name), name
    if header == "so3lr_hip.h":
        assert sorted(_lib.HIP_SYMBOLS) == names


def test_element_map_known_answers():
    # tests/test_element_map.cpp of the reference
    f = lambda t: _lib.hip().so3lr_atomic_number(t.encode())
    assert f("H") == 1 and f("o") == 8 and f("CL") == 17 and f("C") == 6 and f("99") == 99
    assert f("0") == 0 and f("100") == 0 and f("NULL") == 0 and f("8x") == 0
    assert f("Es") == 99 and f("na") == 11 and f("") == 0


def test_check_system_needs_no_device():
    # the (Q, M) rules of src/so3lr_charge_spin.cpp:52-141 and the empty-rank
    # refusal of src/rank_local_half_pair_graph.cpp:43, before any GPU call
    lib = _lib.hip()

    def check(z, q, m):
        z = np.ascontiguousarray(z, dtype=np.int32)
        rc = lib.so3lr_check_system(len(z), _lib.ptr(z), float(q), float(m))
        return rc, (lib.so3lr_last_error(None) or b"").decode()

    o2 = support.load_golden("o2")[1]
    acetate = support.load_golden("acetate")[1]
    assert check(o2, 0, 3)[0] == _lib.OK and check(acetate, -1, 1)[0] == _lib.OK
    rc, msg = check(o2, 0, 2)  # 16 electrons: an even count needs an odd multiplicity
    assert rc == _lib.ERR_SYSTEM and msg
    assert check(acetate, 0, 2)[0] == _lib.OK  # the neutral radical: 31 electrons, a doublet
    rc, msg = check(acetate, 0, 1)  # 31 electrons: an odd count needs an even multiplicity
    assert rc == _lib.ERR_SYSTEM and msg
    rc, msg = check(acetate, -1, 2)  # the anion's 32 electrons: M = 2 is refused
    assert rc == _lib.ERR_SYSTEM and msg
    rc, msg = check(np.zeros(0), 0, 1)
    assert rc == _lib.ERR_ARGUMENT and "empty" in msg
    rc, msg = check([8, 100], 0, 1)
    assert rc == _lib.ERR_ARGUMENT and "1..99" in msg


def _create(path):
    import ctypes
    lib = _lib.hip()
    h = ctypes.c_void_p()
    rc = lib.so3lr_create(path.encode(), 0, ctypes.byref(h))
    msg = lib.so3lr_last_error(None).decode()
    if rc == 0:
        lib.so3lr_destroy(h)
    return rc, msg


def _rewrite(tmp_path, mutate_manifest=None, mutate_bytes=None):
    data = bytearray(open(support.MODEL, "rb").read())
    msize = struct.unpack("<Q", data[16:24])[0]
    manifest = json.loads(bytes(data[128:128 + msize]))
    payload = bytes(data[128 + msize:])
    if mutate_manifest:
        mutate_manifest(manifest)
    mbytes = json.dumps(manifest, sort_keys=True, separators=(",", ":")).encode()
    header = bytearray(data[:128])
    header[16:24] = struct.pack("<Q", len(mbytes))
    header[32:64] = hashlib.sha256(mbytes).digest()
    header[64:96] = hashlib.sha256(payload).digest()
    out = header + mbytes + payload
    if mutate_bytes:
        mutate_bytes(out)
    p = tmp_path / "m.so3lr"
    p.write_bytes(bytes(out))
    return str(p)


def test_valid_model_reaches_the_device_step():
    rc, msg = _create(support.MODEL)
    assert rc in (_lib.OK, _lib.ERR_DEVICE), msg


def test_corrupt_payload_rejected(tmp_path):
    def flip(b):
        b[-1] ^= 0xFF
    rc, msg = _create(_rewrite(tmp_path, mutate_bytes=flip))
    assert rc == _lib.ERR_MODEL and "payload digest does not match" in msg


def test_wrong_magic_rejected(tmp_path):
    def magic(b):
        b[0:8] = b"NOTSO3LR"
    rc, msg = _create(_rewrite(tmp_path, mutate_bytes=magic))
    assert rc == _lib.ERR_MODEL and "magic" in msg


def test_missing_file_rejected():
    rc, msg = _create("/nonexistent/model.so3lr")
    assert rc == _lib.ERR_MODEL and "cannot read" in msg


@pytest.mark.parametrize("key,value,feature", [
    ("invariant_features", 512, "invariant_features"),
    # the released widths F = 256 and R = 64 load; these manifests keep the
    # v1 tensors, so the contract names what disagrees
    ("invariant_features", 256, "invariant_features / 32 heads"),
    ("interaction_blocks", 9, "interaction_blocks"),
    ("brand_new_operator", 1, "unknown architecture key"),
    ("repulsion_type", "none", "repulsion other than"),
    ("radial_basis_features", 48, "radial_basis_features"),
    ("radial_basis_features", 64, "radial_basis_fn.k"),
    ("euclidean_degree_channels", 3, "euclidean_degree_channels"),
    ("output_heads", ["atomic_energy_output_block", "partial_charges_output_block", "hirshfeld_output_block",
                      "dipole_vec_output_block"], "output heads other than"),
    ("layer_norm_epsilon", 1e-5, "LayerNorm epsilon"),
    # refused by the reference's post-attention block as well
    # (kokkos_post_attention_block0.cpp:386-390)
    ("layer_normalization_1", False, "first position"),
    ("residual_mlp_2", True, "residual MLP layout"),
    ("message_normalization", "sum", "message normalisation"),
    ("qk_nonlinearity", "silu", "QK nonlinearity"),
    # accepted options whose tensors the mutated manifest lacks: the load
    # names the missing tensor
    ("repulsion_type", "nlh", "physical.nlh_a"),
    ("use_residual_scalars", True, "model.resid_lambdas"),
    ("output_heads", ["atomic_energy_output_block", "partial_charges_output_block", "hirshfeld_output_block",
                      "c6_ratios_output_block"], "c6_ratios_output_block"),
])
def test_capability_refusal_names_the_feature(tmp_path, key, value, feature):
    """Structurally valid mutated models (re-serialised manifest, recomputed
    SHA-256), as in the reference's test_capability_rejection.py."""
    def mutate(m):
        m["architecture"][key] = value
    rc, msg = _create(_rewrite(tmp_path, mutate_manifest=mutate))
    assert rc == _lib.ERR_MODEL, msg
    assert feature in msg, msg


def test_weights_beyond_the_activation_range_are_refused(tmp_path):
    """A radial filter weight large enough to take a SiLU argument past the
    table exponential's range is refused at load, not evaluated wrongly."""
    def big(manifest, arrays):
        arrays["model.euclidean_transformers.1.filter_net_ev.mlp_rbf.0.weight"][3, 5] = 5000.0
    path = support.variant_model(tmp_path / "big.so3lr", edit=big)
    rc, msg = _create(path)
    assert rc == _lib.ERR_MODEL and "SiLU arguments" in msg, msg


def test_generic_weights_beyond_the_activation_range_are_refused(tmp_path):
    """The same bound for a model on the generic kernels, whose fused filters
    take the radial hidden layer through the table exponential too."""
    def big(manifest, arrays):
        arrays["model.euclidean_transformers.2.filter_net_inv.mlp_rbf.0.weight"][7, 40] = 5000.0
    base = support.lifted_model(tmp_path / "wide.so3lr")
    path = support.variant_model(tmp_path / "wide_big.so3lr", edit=big, base=base)
    rc, msg = _create(path)
    assert rc == _lib.ERR_MODEL and "SiLU arguments" in msg and "radial" in msg, msg


def test_released_widths_are_accepted(tmp_path):
    """F = 256 with R = 64, duplicated degree slots and an energy/charge head
    narrower than F (support.lifted_model), and duplicated or missing degrees
    at F = 128 (support.degrees_model) load up to the device step."""
    for path in (support.lifted_model(tmp_path / "wide.so3lr"),
                 support.degrees_model(tmp_path / "d1123.so3lr", (1, 1, 2, 3)),
                 support.degrees_model(tmp_path / "d1233.so3lr", (1, 2, 3, 3))):
        rc, msg = _create(path)
        assert rc in (_lib.OK, _lib.ERR_DEVICE), msg


@pytest.mark.parametrize("repeats,feature", [
    ([3, 5, 9, 7], "sorted"), ([3, 5, 7, 11], "2l + 1"), ([3, 4, 7, 9], "2l + 1")])
def test_degree_layout_rules(tmp_path, repeats, feature):
    """Degree slots must be 2l + 1 wide with l in 1..4 and sorted
    (so3lr_architecture.cpp:246-268); a later block with another layout than
    block 0 is refused too."""
    def edit(manifest, arrays):
        for b in range(3):
            for blk in ("euclidean_attention_block", "interaction_block"):
                arrays["model.euclidean_transformers.%d.%s.degree_repeats" % (b, blk)] = np.array(repeats, dtype=np.int64)
    rc, msg = _create(support.variant_model(tmp_path / "deg.so3lr", edit=edit))
    assert rc == _lib.ERR_MODEL and feature in msg, msg


def test_degree_layout_must_agree_across_blocks(tmp_path):
    def edit(manifest, arrays):
        arrays["model.euclidean_transformers.2.interaction_block.degree_repeats"] = np.array([3, 3, 7, 9], dtype=np.int64)
    rc, msg = _create(support.variant_model(tmp_path / "deg2.so3lr", edit=edit))
    assert rc == _lib.ERR_MODEL and "another degree layout" in msg, msg


@pytest.mark.parametrize("key,value", [
    ("use_rms_norm", True), ("qk_norm", True), ("layer_normalization_2", False),
    ("message_normalization", "identity"), ("message_normalization", "sqrt_num_features"),
])
def test_architecture_options_are_accepted(tmp_path, key, value):
    """Options the reference runs and this build implements load (up to the
    device step on a machine without a GPU); RMSNorm needs no tensors, so the
    shipped LayerNorm parameters are simply not read."""
    def mutate(m):
        m["architecture"][key] = value
    rc, msg = _create(_rewrite(tmp_path, mutate_manifest=mutate))
    assert rc in (_lib.OK, _lib.ERR_DEVICE), msg


def test_lammps_lists_match_brute_force():
    ref, z, pos, box = support.load_golden("water3000")
    L = _lib.Lists(pos, np.zeros(3), box, (1, 1, 1))
    sr, lr = support.build_graphs(pos, box, 5.5, 13.0)
    assert len(L.lists[0][2]) == len(sr[0])
    assert len(L.lists[1][2]) == len(lr[0])
    # every ghost row sits at its owner's position plus a lattice vector
    xr = L.rows_positions(pos)
    assert np.allclose(xr[:len(pos)], pos)


def _with_manifest_bytes(tmp_path, edit_text=None, edit_manifest=None, edit_payload=None):
    """The shipped model with its manifest re-encoded canonically (after
    edit_manifest) and then edited as text (edit_text), its payload edited
    (edit_payload), and both digests and sizes recomputed, so only the rule
    under test is broken."""
    data = bytes(open(support.MODEL, "rb").read())
    msize = struct.unpack("<Q", data[16:24])[0]
    manifest = json.loads(data[128:128 + msize])
    payload = bytearray(data[128 + msize:])
    if edit_manifest:
        edit_manifest(manifest, payload)
    if edit_payload:
        edit_payload(manifest, payload)
    text = json.dumps(manifest, sort_keys=True, separators=(",", ":"), ensure_ascii=True)
    if edit_text:
        text = edit_text(text)
    mbytes = text.encode("utf-8")
    header = bytearray(data[:128])
    header[16:24] = struct.pack("<Q", len(mbytes))
    header[24:32] = struct.pack("<Q", len(payload))
    header[32:64] = hashlib.sha256(mbytes).digest()
    header[64:96] = hashlib.sha256(bytes(payload)).digest()
    p = tmp_path / "m.so3lr"
    p.write_bytes(bytes(header) + mbytes + bytes(payload))
    return str(p)


def test_canonical_reencoding_loads(tmp_path):
    rc, msg = _create(_with_manifest_bytes(tmp_path))
    assert rc in (_lib.OK, _lib.ERR_DEVICE), msg


@pytest.mark.parametrize("edit,why", [
    (lambda t: t.replace('{"architecture":', '{ "architecture":', 1), "member name"),
    (lambda t: t.replace(',"endianness"', ', "endianness"', 1), "not a value"),
    (lambda t: t.replace('"lr_pair_scale":0.5', '"lr_pair_scale":0.50', 1), "shortest repr"),
    (lambda t: t.replace('"lr_pair_scale":0.5', '"lr_pair_scale":5e-1', 1), "shortest repr"),
    (lambda t: t.replace('"layer_norm_epsilon":1e-06', '"layer_norm_epsilon":1E-06', 1), "shortest repr"),
    (lambda t: t.replace('"tensor_alignment":64', '"tensor_alignment":064', 1), "leading zero"),
    (lambda t: t.replace('"format":"so3lr-native"', '"format":"so3lr\\u002dnative"', 1), "\\u escape"),
    (lambda t: t.replace('"format":"so3lr-native"', '"format":"so3lr\\/native"', 1), "escape the canonical encoder"),
    (lambda t: t.replace('"format":"so3lr-native"', '"format":"so3lr-nativé"', 1), "printable ASCII"),
    (lambda t: t + " ", "printable ASCII"),
    (lambda t: t + "{}", "after the top-level value"),
    (lambda t: t[:-1], "ends inside a container"),
])
def test_noncanonical_manifest_rejected(tmp_path, edit, why):
    """docs/FORMAT.md:68-82: a reader must reject noncanonical or malformed
    JSON; canonical is the exporter's json.dumps(sort_keys=True,
    separators=(",", ":"), ensure_ascii=True)."""
    rc, msg = _create(_with_manifest_bytes(tmp_path, edit_text=edit))
    assert rc == _lib.ERR_MODEL, msg
    assert "canonical JSON" in msg or why in msg, msg


def test_unsorted_keys_rejected(tmp_path):
    def swap(t):
        # move "schema" in front of "format": keys out of order, still valid JSON
        obj = json.loads(t)
        items = list(obj.items())
        items.insert(0, items.pop([k for k, _ in items].index("schema")))
        return "{" + ",".join(json.dumps(k) + ":" + json.dumps(v, sort_keys=True, separators=(",", ":"))
                              for k, v in items) + "}"
    rc, msg = _create(_with_manifest_bytes(tmp_path, edit_text=swap))
    assert rc == _lib.ERR_MODEL and "strictly increasing" in msg, msg


def _first_tensors(m):
    return m["tensors"][0], m["tensors"][1]


@pytest.mark.parametrize("case,expect", [
    ("version", "version 2"),
    ("reserved", "reserved"),
    ("sizes", "do not add up"),
    ("manifest_digest", "manifest digest"),
    ("dup_name", "out of order or repeated"),
    ("dup_key", "appears twice"),
    ("dtype", "not a version-1 dtype"),
    ("unaligned", "not 64-byte aligned"),
    ("overlap", "overlaps"),
    ("padding", "not zero-filled"),
    ("tensor_digest", "digest does not match its bytes"),
    ("trailing", "belong to none"),
    ("nbytes", "bytes recorded"),
    ("totals", "tensor_count / tensor_bytes"),
    ("count_float", "non-negative integer"),
    ("range", "reaches past the payload"),
])
def test_container_rules(tmp_path, case, expect):
    """Each rejection rule of docs/FORMAT.md:68-82, one at a time."""
    em = ep = et = None
    post = None
    if case == "version":
        post = lambda b: b.__setitem__(slice(8, 12), struct.pack("<I", 2))
    elif case == "reserved":
        post = lambda b: b.__setitem__(100, 1)
    elif case == "sizes":
        post = lambda b: b.__setitem__(slice(24, 32), struct.pack("<Q", struct.unpack("<Q", bytes(b[24:32]))[0] + 1))
    elif case == "manifest_digest":
        post = lambda b: b.__setitem__(40, b[40] ^ 1)
    elif case == "dup_name":
        def em(m, p):
            a, b = _first_tensors(m)
            b["name"] = a["name"]
    elif case == "dup_key":
        def em(m, p):
            a, b = _first_tensors(m)
            b["state_key"] = a["state_key"]
    elif case == "dtype":
        def em(m, p):
            m["tensors"][0]["dtype"] = "float16"
    elif case == "unaligned":
        def em(m, p):
            m["tensors"][1]["offset"] += 8
    elif case == "overlap":
        def em(m, p):
            a, b = _first_tensors(m)
            b["offset"] = a["offset"]
            b["sha256"] = hashlib.sha256(bytes(p[b["offset"]:b["offset"] + b["nbytes"]])).hexdigest()
    elif case == "padding":
        def ep(m, p):
            a, b = _first_tensors(m)
            gap = a["offset"] + a["nbytes"]
            assert gap < b["offset"], "needs a padded gap"
            p[gap] = 7
    elif case == "tensor_digest":
        def ep(m, p):
            t = m["tensors"][0]
            p[t["offset"]] ^= 0x40
    elif case == "trailing":
        def ep(m, p):
            p.extend(b"\0" * 64)
    elif case == "nbytes":
        def em(m, p):
            m["tensors"][0]["nbytes"] += 8
    elif case == "totals":
        def em(m, p):
            m["tensor_bytes"] += 1
    elif case == "count_float":
        et = lambda t: t.replace('"tensor_alignment":64', '"tensor_alignment":64.0', 1)
    elif case == "range":
        def em(m, p):
            t = m["tensors"][-1]
            t["offset"] = (len(p) + 127) // 64 * 64
    path = _with_manifest_bytes(tmp_path, edit_text=et, edit_manifest=em, edit_payload=ep)
    if post:
        b = bytearray(open(path, "rb").read())
        post(b)
        open(path, "wb").write(bytes(b))
    rc, msg = _create(path)
    assert rc == _lib.ERR_MODEL, msg
    assert expect in msg, msg


def test_binding_refuses_bad_device_buffers():
    """The ctypes binding checks what the C ABI cannot see (device, dtype,
    contiguity, size) before any pointer reaches a kernel."""
    import torch
    with pytest.raises(ValueError, match="GPU tensor"):
        _lib.device_f64(torch.zeros(6, dtype=torch.float64), 6, "positions")
    with pytest.raises(ValueError, match="GPU tensor"):
        _lib.device_f64(np.zeros(6), 6, "positions")
    with pytest.raises(ValueError, match="required"):
        _lib.device_f64(None, 6, "forces")

    class FakeCuda:  # the attributes a torch CUDA tensor exposes
        def __init__(self, dtype, contiguous, n):
            self.is_cuda, self.dtype, self._c, self._n = True, dtype, contiguous, n

        def is_contiguous(self):
            return self._c

        def numel(self):
            return self._n

        def data_ptr(self):
            return 0

    with pytest.raises(ValueError, match="float64"):
        _lib.device_f64(FakeCuda(torch.float32, True, 6), 6, "positions")
    with pytest.raises(ValueError, match="contiguous"):
        _lib.device_f64(FakeCuda(torch.float64, False, 6), 6, "positions")
    with pytest.raises(ValueError, match="hold 6 values"):
        _lib.device_f64(FakeCuda(torch.float64, True, 3), 6, "positions")
    _lib.device_f64(FakeCuda(torch.float64, True, 6), 6, "positions")

    ctx = object.__new__(_lib.Context)  # no device: the checks run before any library call
    ctx.n, ctx.rows, ctx._h = 2, 2, None
    with pytest.raises(ValueError, match="forces"):
        ctx.compute_device(FakeCuda(torch.float64, True, 6), FakeCuda(torch.float64, True, 5))
    with pytest.raises(ValueError, match="one entry more"):
        ctx.set_images([8, 1, 1], [0, 2], [0.0, 0.0], [1.0, 1.0])
