"""Reader of the reference's golden datasets (tests/golden/<set>/manifest.json
+ tensors.bin, the format of tests/test.infer.ref.pas:1-30 in the reference):
little-endian raw blobs described by name, dtype, shape, offset and sha256."""
import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_DT = {"f32": np.float32, "i32": np.int32, "u8": np.uint8}


class GoldenSet:
    def __init__(self, name):
        d = os.path.join(GOLDEN, name)
        with open(os.path.join(d, "manifest.json")) as f:
            self.manifest = json.load(f)
        with open(os.path.join(d, self.manifest["blob"]["file"]), "rb") as f:
            self.blob = f.read()
        if hashlib.sha256(self.blob).hexdigest() != self.manifest["blob"]["sha256"]:
            raise ValueError(f"{name}: tensors.bin does not match its sha256")
        self.tensors = {t["name"]: t for t in self.manifest["tensors"]}

    def __getitem__(self, name):
        t = self.tensors[name]
        raw = self.blob[t["offset"]:t["offset"] + t["bytes"]]
        if hashlib.sha256(raw).hexdigest() != t["sha256"]:
            raise ValueError(f"{name}: sha256 mismatch")
        return np.frombuffer(raw, dtype=_DT[t["dtype"]]).reshape(t["shape"]).copy()


def compare(a, r, atol, rtol):
    """InferCompare of tests/test.infer.ref.pas:344-394: every element
    |a - r| <= atol + rtol * |r| (NaN never passes)."""
    a = np.asarray(a, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    ok = np.abs(a - r) <= atol + rtol * np.abs(r)
    return bool(np.all(ok)), float(np.max(np.abs(a - r))) if a.size else 0.0


def rel_error(a, b):
    """RelError of tests/test.infer.fast.pas:348-360: max|a - b| / max|b|."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / m) if m > 0 else float(np.max(np.abs(a - b)))


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    n = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / n) if n > 0 else float(np.linalg.norm(a - b))
