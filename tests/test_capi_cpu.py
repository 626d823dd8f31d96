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
    assert rc == _lib.ERR_MODEL and "payload SHA-256 mismatch" in msg


def test_wrong_magic_rejected(tmp_path):
    def magic(b):
        b[0:8] = b"NOTSO3LR"
    rc, msg = _create(_rewrite(tmp_path, mutate_bytes=magic))
    assert rc == _lib.ERR_MODEL and "wrong magic" in msg


def test_missing_file_rejected():
    rc, msg = _create("/nonexistent/model.so3lr")
    assert rc == _lib.ERR_MODEL and "cannot open" in msg


@pytest.mark.parametrize("key,value,feature", [
    ("use_rms_norm", True, "RMSNorm"),
    ("qk_norm", True, "QK normalisation"),
    ("invariant_features", 256, "invariant_features"),
    ("interaction_blocks", 9, "interaction_blocks"),
    ("brand_new_operator", 1, "unknown architecture key"),
    ("repulsion_type", "nlh", "repulsion other than learned ZBL"),
    ("use_residual_scalars", True, "residual scalars"),
    ("radial_basis_features", 64, "radial_basis_features"),
    ("output_heads", ["atomic_energy_output_block", "partial_charges_output_block", "hirshfeld_output_block",
                      "c6_ratios_output_block"], "output heads other than"),
    ("layer_norm_epsilon", 1e-5, "LayerNorm epsilon"),
])
def test_capability_refusal_names_the_feature(tmp_path, key, value, feature):
    """Structurally valid mutated models (re-serialised manifest, recomputed
    SHA-256), as in the reference's test_capability_rejection.py."""
    def mutate(m):
        m["architecture"][key] = value
    rc, msg = _create(_rewrite(tmp_path, mutate_manifest=mutate))
    assert rc == _lib.ERR_MODEL, msg
    assert feature in msg, msg


def test_lammps_lists_match_brute_force():
    ref, z, pos, box = support.load_golden("water3000")
    L = _lib.Lists(pos, np.zeros(3), box, (1, 1, 1))
    sr, lr = support.build_graphs(pos, box, 5.5, 13.0)
    assert len(L.lists[0][2]) == len(sr[0])
    assert len(L.lists[1][2]) == len(lr[0])
    # every ghost row sits at its owner's position plus a lattice vector
    xr = L.rows_positions(pos)
    assert np.allclose(xr[:len(pos)], pos)
