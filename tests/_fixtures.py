"""Reader for the reference's CPPAIENG v1 tensor files (the PyTorch-replay fixtures).

Layout (little endian), as written by the reference's save_parameters
(src/serialize.cpp:70-101) and by its fixture generator:
  8 bytes  magic "CPPAIENG"
  u32      version (1)
  u32      tensor count
  per tensor: u32 name length, name bytes, u32 ndim, ndim x u64 dims, fp32 data.
The reader is plain struct/numpy: nothing in the file is executed.
"""
import os
import struct

import numpy as np

FIXTURE_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures")


def load_tensors(path):
    with open(path, "rb") as f:
        blob = f.read()
    if blob[:8] != b"CPPAIENG":
        raise ValueError(f"{path}: not a CPPAIENG file")
    version, count = struct.unpack_from("<II", blob, 8)
    if version != 1:
        raise ValueError(f"{path}: unsupported version {version}")
    off = 16
    out = {}
    for _ in range(count):
        (nlen,) = struct.unpack_from("<I", blob, off)
        off += 4
        name = blob[off:off + nlen].decode("utf-8")
        off += nlen
        (ndim,) = struct.unpack_from("<I", blob, off)
        off += 4
        dims = struct.unpack_from("<" + "Q" * ndim, blob, off)
        off += 8 * ndim
        n = int(np.prod(dims)) if ndim else 1
        data = np.frombuffer(blob, dtype="<f4", count=n, offset=off).astype(np.float32)
        off += 4 * n
        out[name] = data.reshape(dims)
    if off != len(blob):
        raise ValueError(f"{path}: {len(blob) - off} trailing bytes")
    return out


def load(name):
    return load_tensors(os.path.join(FIXTURE_DIR, name + ".bin"))


ALL = sorted(f[:-4] for f in os.listdir(FIXTURE_DIR) if f.endswith(".bin"))
