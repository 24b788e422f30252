"""The engine's IDX reader (engine/src/data.cpp, the reference's src/data.cpp) on the host:
header dimensions are untrusted, so a header whose payload overflows or exceeds the file
reads as a truncated file instead of wrapping the size or allocating it. No GPU needed."""
import ctypes as C
import struct

import pytest

import engine_capi

LABELS, IMAGES = 0x00000801, 0x00000803


@pytest.fixture(scope="module")
def lib():
    lib = engine_capi.load_library()
    lib.eng_idx_probe.argtypes = [C.c_char_p, C.c_uint32, C.c_int64,
                                  C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
    return lib


def probe(lib, path, magic, max_items=0):
    count, nbytes = C.c_int64(-1), C.c_int64(-1)
    rc = lib.eng_idx_probe(str(path).encode(), magic, max_items, C.byref(count), C.byref(nbytes))
    if rc != 0:
        raise RuntimeError(lib.eng_last_error().decode())
    return count.value, nbytes.value


def write(path, magic, dims, payload):
    path.write_bytes(struct.pack(">I", magic) + b"".join(struct.pack(">I", d) for d in dims)
                     + payload)
    return path


def test_well_formed_files(lib, tmp_path):
    f = write(tmp_path / "lab", LABELS, [5], bytes(range(5)))
    assert probe(lib, f, LABELS) == (5, 5)
    assert probe(lib, f, LABELS, 3) == (3, 3)
    f = write(tmp_path / "img", IMAGES, [3, 4, 5], bytes(60))
    assert probe(lib, f, IMAGES) == (3, 60)
    assert probe(lib, f, IMAGES, 2) == (2, 40)


def test_short_payload_is_truncated(lib, tmp_path):
    f = write(tmp_path / "img", IMAGES, [3, 4, 5], bytes(59))
    with pytest.raises(RuntimeError, match="fewer than 3 items"):
        probe(lib, f, IMAGES)


def test_huge_header_is_truncated_not_allocated(lib, tmp_path):
    # 4e9 labels claimed by a 10-byte payload: refused before any allocation.
    f = write(tmp_path / "lab", LABELS, [0xFFFFFFFF], bytes(10))
    with pytest.raises(RuntimeError, match="fewer than"):
        probe(lib, f, LABELS)
    # Dimensions whose product overflows 64 bits (2^32-1 cubed).
    f = write(tmp_path / "img", IMAGES, [0xFFFFFFFF] * 3, bytes(16))
    with pytest.raises(RuntimeError, match="fewer than"):
        probe(lib, f, IMAGES)


def test_header_errors(lib, tmp_path):
    f = write(tmp_path / "bad", 0x00000802, [1], b"x")
    with pytest.raises(RuntimeError, match="magic"):
        probe(lib, f, LABELS)
    f = tmp_path / "short"
    f.write_bytes(struct.pack(">I", IMAGES) + struct.pack(">I", 1))
    with pytest.raises(RuntimeError, match="header"):
        probe(lib, f, IMAGES)
    with pytest.raises(RuntimeError, match="Cannot open"):
        probe(lib, tmp_path / "missing", LABELS)
