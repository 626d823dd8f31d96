"""Reader and writer of the SO3LR native model file (`.so3lr`).

The layout is the one the reference's exporter writes
(source/so3lr-lammps-native/exporter/so3lr_native_format.py:15-127) and the
library's loader checks (csrc/model.cpp, Model::load_bytes):

* a 128-byte little-endian header: the magic b"SO3LRN1\\0", version 1 and
  flags 0 (two u32), the manifest and payload sizes (two u64), the SHA-256 of
  the manifest and of the payload, then 32 reserved zero bytes;
* the manifest: JSON with sorted keys and no whitespace;
* the payload: every tensor at a 64-byte aligned offset, in manifest order,
  zero padding between them; each manifest record carries its tensor's
  offset, byte count and SHA-256.

`python -m so3lrxlammps_amd.model_file MODEL [--manifest OUT]` verifies a
file and prints its summary as key=value lines, with the keys of the
reference's check (exporter/so3lr_native_format.py:218-236), so scripts that
read them keep working.

`write_model` takes a manifest and the tensors by state key, lays the payload
out again and recomputes every size and digest, so a manifest read from one
file can carry new tensor values (tests use it for models with perturbed
weights).
"""
import argparse
import hashlib
import json
import struct

import numpy as np

MAGIC = b"SO3LRN1\0"
HEADER = struct.Struct("<8sIIQQ32s32s32s")  # 128 bytes
ALIGN = 64
_DTYPES = {"float64": "<f8", "float32": "<f4", "int64": "<i8", "int32": "<i4"}


def _canonical(manifest):
    return json.dumps(manifest, sort_keys=True, separators=(",", ":")).encode()


def read_model(path):
    """(manifest, {state_key: ndarray}) of a model file, digests checked."""
    raw = open(path, "rb").read()
    if len(raw) < HEADER.size:
        raise ValueError("%s: shorter than the header" % path)
    magic, version, flags, msize, psize, mhash, phash, reserved = HEADER.unpack(raw[:HEADER.size])
    if magic != MAGIC or version != 1 or flags != 0 or any(reserved):
        raise ValueError("%s: not a version-1 SO3LR native model" % path)
    if HEADER.size + msize + psize != len(raw):
        raise ValueError("%s: header sizes do not match the file" % path)
    mbytes = raw[HEADER.size:HEADER.size + msize]
    payload = raw[HEADER.size + msize:]
    if hashlib.sha256(mbytes).digest() != mhash or hashlib.sha256(payload).digest() != phash:
        raise ValueError("%s: SHA-256 mismatch" % path)
    manifest = json.loads(mbytes)
    arrays = {}
    for rec in manifest["tensors"]:
        blob = payload[rec["offset"]:rec["offset"] + rec["nbytes"]]
        if hashlib.sha256(blob).hexdigest() != rec["sha256"]:
            raise ValueError("%s: tensor %s SHA-256 mismatch" % (path, rec["name"]))
        arrays[rec["state_key"]] = np.frombuffer(blob, dtype=_DTYPES[rec["dtype"]]).reshape(rec["shape"]).copy()
    return manifest, arrays


def write_model(path, manifest, arrays):
    """Write `manifest` with the tensors of `arrays` (by state key; shapes and
    dtypes as the manifest records them) as a model file."""
    manifest = json.loads(json.dumps(manifest))  # a private copy
    chunks, offset, total = [], 0, 0
    for rec in manifest["tensors"]:
        a = np.asarray(arrays[rec["state_key"]], dtype=_DTYPES[rec["dtype"]])  # 0-d stays 0-d; tobytes is C order
        if list(a.shape) != list(rec["shape"]):
            raise ValueError("tensor %s: shape %s, manifest %s" % (rec["name"], a.shape, rec["shape"]))
        blob = a.tobytes()
        pad = (-offset) % ALIGN
        chunks.append(b"\0" * pad)
        offset += pad
        rec["offset"], rec["nbytes"], rec["sha256"] = offset, len(blob), hashlib.sha256(blob).hexdigest()
        chunks.append(blob)
        offset += len(blob)
        total += len(blob)
    manifest["tensor_count"] = len(manifest["tensors"])
    manifest["tensor_bytes"] = total
    manifest["tensor_alignment"] = ALIGN
    mbytes = _canonical(manifest)
    payload = b"".join(chunks)
    header = HEADER.pack(MAGIC, 1, 0, len(mbytes), len(payload), hashlib.sha256(mbytes).digest(),
                         hashlib.sha256(payload).digest(), b"\0" * 32)
    with open(path, "wb") as f:
        f.write(header + mbytes + payload)


def main(argv=None):
    ap = argparse.ArgumentParser(description="Verify an SO3LR native model file and print its summary.")
    ap.add_argument("model")
    ap.add_argument("--manifest", help="also write the manifest here, indented")
    args = ap.parse_args(argv)
    manifest, arrays = read_model(args.model)
    if args.manifest:
        with open(args.manifest, "w") as f:
            f.write(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    arch = manifest.get("architecture", {})
    with open(args.model, "rb") as f:
        payload = HEADER.unpack(f.read(HEADER.size))[4]  # payload size, checked by read_model
    for key, value in (("format_version", manifest["format_version"]), ("model_family", manifest.get("model_family")),
                       ("tensor_count", manifest["tensor_count"]), ("tensor_bytes", manifest["tensor_bytes"]),
                       ("payload_bytes", payload),
                       ("short_range_cutoff", arch.get("short_range_cutoff_angstrom")),
                       ("long_range_cutoff", arch.get("long_range_cutoff_angstrom"))):
        print("%s=%s" % (key, value))
    print("native_model_format_validation=PASS")


if __name__ == "__main__":
    main()
