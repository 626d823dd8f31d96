"""The model-file reader and writer (so3lrxlammps_amd/model_file.py) on the
CPU: a read -> write round trip reproduces the shipped model byte for byte
(the layout of exporter/so3lr_native_format.py:15-127: header, canonical JSON,
64-byte alignment, digests); a model with perturbed weights passes the
library's loader up to the device step, changes the energy, and keeps the
oracle's forces equal to central finite differences of its energy."""
import numpy as np
import pytest

import support
from oracle.oracle import Oracle
from so3lrxlammps_amd import _lib
from so3lrxlammps_amd.model_file import read_model, write_model


def test_round_trip_reproduces_the_shipped_model(tmp_path):
    manifest, arrays = read_model(support.MODEL)
    out = tmp_path / "copy.so3lr"
    write_model(str(out), manifest, arrays)
    assert out.read_bytes() == open(support.MODEL, "rb").read()


def test_reader_rejects_a_changed_tensor(tmp_path):
    data = bytearray(open(support.MODEL, "rb").read())
    data[-1] ^= 1  # last payload byte: the payload digest no longer matches
    bad = tmp_path / "bad.so3lr"
    bad.write_bytes(bytes(data))
    with pytest.raises(ValueError, match="SHA-256"):
        read_model(str(bad))


def test_writer_rejects_a_wrong_shape(tmp_path):
    manifest, arrays = read_model(support.MODEL)
    key = next(r["state_key"] for r in manifest["tensors"] if r["role"] == "parameter")
    arrays[key] = arrays[key].ravel()[:-1]
    with pytest.raises(ValueError, match="shape"):
        write_model(str(tmp_path / "x.so3lr"), manifest, arrays)


@pytest.fixture(scope="module")
def perturbed(tmp_path_factory):
    return support.perturbed_model(tmp_path_factory.mktemp("model") / "perturbed.so3lr")


def test_perturbed_model_passes_the_loader(perturbed):
    import ctypes
    lib = _lib.hip()
    h = ctypes.c_void_p()
    rc = lib.so3lr_create(perturbed.encode(), 0, ctypes.byref(h))
    if rc == _lib.OK:
        lib.so3lr_destroy(h)
    assert rc in (_lib.OK, _lib.ERR_DEVICE), lib.so3lr_last_error(None).decode()


def test_perturbed_model_forces_are_the_energy_gradient(perturbed):
    ref, z, pos, box = support.load_golden("acetate")
    q, m = -1, 1
    orc, base = Oracle(perturbed), Oracle(support.MODEL)

    def run(o, p):
        return o.evaluate(z, *support.build_graphs(p), charge=q, multiplicity=m)

    out = run(orc, pos)
    e0 = run(base, pos)["energy"]
    assert abs(out["energy"] - e0) > 1e-3 * abs(e0)  # the weights matter
    h = 1e-4
    for i in (0, 3):
        for a in range(3):
            p1 = pos.copy(); p1[i, a] += h
            p2 = pos.copy(); p2[i, a] -= h
            fd = -(run(orc, p1)["energy"] - run(orc, p2)["energy"]) / (2 * h)
            assert abs(fd - out["forces"][i, a]) < 2e-6, (i, a, fd, out["forces"][i, a])


def test_verify_command_prints_the_reference_keys(tmp_path):
    import subprocess
    import sys
    out = subprocess.run([sys.executable, "-m", "so3lrxlammps_amd.model_file", support.MODEL, "--manifest",
                          str(tmp_path / "manifest.json")], cwd=support.REPO, capture_output=True, text=True,
                         check=True).stdout
    kv = dict(line.split("=", 1) for line in out.split())
    assert kv["format_version"] == "1" and kv["model_family"] == "SO3LR"
    assert kv["tensor_count"] == "213" and kv["payload_bytes"] == str(len(open(support.MODEL, "rb").read())
                                                                     - 128 - _manifest_size())
    assert float(kv["short_range_cutoff"]) == 4.5 and float(kv["long_range_cutoff"]) == 12.0
    assert kv["native_model_format_validation"] == "PASS"
    assert (tmp_path / "manifest.json").read_text().startswith("{\n")


def _manifest_size():
    import struct
    return struct.unpack("<Q", open(support.MODEL, "rb").read(24)[16:24])[0]
