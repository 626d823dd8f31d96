"""Minimal `.so3lr` reader for the oracle -- TEST INFRASTRUCTURE ONLY.

Reads the fixed 128-byte header, the JSON manifest and the tensor payload of a
`.so3lr` v1 file (layout per source/so3lr-lammps-native/docs/FORMAT.md:12-46)
into numpy arrays keyed by `state_key`.  Integrity checks (SHA-256 of manifest,
payload and tensors) are repeated here so a corrupted fixture cannot silently
feed the oracle; the full rejection rules live in the product's C++ reader.
"""
import hashlib
import json
import struct

import numpy as np

_DTYPES = {"float64": np.float64, "float32": np.float32, "int64": np.int64,
           "int32": np.int32, "uint8": np.uint8, "bool": np.uint8}


class Model:
    def __init__(self, manifest, tensors):
        self.manifest = manifest
        self.tensors = tensors
        self.arch = manifest["architecture"]

    def __getitem__(self, key):
        return self.tensors[key]


def load(path):
    data = open(path, "rb").read()
    if data[:8] != b"SO3LRN1\x00":
        raise ValueError("wrong magic")
    version, flags, msize, psize = struct.unpack("<IIQQ", data[8:32])
    if version != 1 or flags != 0 or 128 + msize + psize != len(data):
        raise ValueError("bad header")
    manifest_bytes = data[128:128 + msize]
    payload = data[128 + msize:]
    if hashlib.sha256(manifest_bytes).digest() != data[32:64]:
        raise ValueError("manifest sha256 mismatch")
    if hashlib.sha256(payload).digest() != data[64:96]:
        raise ValueError("payload sha256 mismatch")
    manifest = json.loads(manifest_bytes)
    tensors = {}
    for rec in manifest["tensors"]:
        raw = payload[rec["offset"]:rec["offset"] + rec["nbytes"]]
        if hashlib.sha256(raw).hexdigest() != rec["sha256"]:
            raise ValueError("tensor sha256 mismatch: " + rec["state_key"])
        arr = np.frombuffer(raw, dtype=_DTYPES[rec["dtype"]]).copy()
        tensors[rec["state_key"]] = arr.reshape(rec["shape"]) if rec["shape"] else arr.reshape(())
    return Model(manifest, tensors)
