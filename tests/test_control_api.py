"""The runtime control API (the reference's include/engine/cuda.hpp:23-125 under
engine::hip): the enabled switch, the version queries and the per-kernel occupancy report,
through the C ABI and through the C++ wrappers (engine/src/hip_runtime.cpp via capi.cpp)."""
import ctypes as C

import numpy as np
import pytest

from _hip import backend, print_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return backend()


@pytest.fixture(scope="module")
def eng():
    # torch's HIP runtime first, as the other GPU fixtures do: initialised after the engine
    # library in a fresh process, torch reports no device.
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a visible GPU")
    from engine_capi import Engine
    e = Engine()
    e.lib.eng_set_enabled.argtypes = [C.c_int]
    e.lib.eng_set_enabled.restype = None
    e.lib.eng_versions.argtypes = [C.POINTER(C.c_int)] * 3
    e.lib.eng_versions.restype = None
    e.lib.eng_kernel_occupancy.argtypes = [C.c_char_p, C.c_int64]
    return e


def test_enabled_switch(eng, hip):
    """Switched off, the engine refuses to launch (it has no CPU path, so it raises where the
    reference would run its CPU loops); switched back on, the same call computes."""
    print_case("control: enabled switch")
    a = np.ones((4, 4), np.float32)
    assert eng.lib.eng_enabled() == 1 and hip.lib.ehip_enabled() == 1
    eng.lib.eng_set_enabled(0)
    try:
        assert eng.lib.eng_enabled() == 0 and hip.lib.ehip_enabled() == 0
        with pytest.raises(RuntimeError, match="switched off"):
            eng.matmul(a, a)
    finally:
        eng.lib.eng_set_enabled(1)
    assert eng.lib.eng_enabled() == 1
    assert np.array_equal(eng.matmul(a, a), np.full((4, 4), 4.0, np.float32))


def test_versions(eng, hip):
    print_case("control: versions")
    compiled, runtime, driver = hip.versions()
    assert compiled >= 60000000 and runtime > 0 and driver > 0, (compiled, runtime, driver)
    v = [C.c_int(-1) for _ in range(3)]
    eng.lib.eng_versions(*[C.byref(x) for x in v])
    assert tuple(x.value for x in v) == (compiled, runtime, driver)


def test_kernel_occupancy(eng, hip):
    """Every registered kernel reports a block size, registers, at least one resident block
    per CU, an occupancy in (0, 1] and a limiter; the C++ report lists the same kernels."""
    print_case("control: kernel occupancy")
    occ = hip.kernel_occupancy()
    assert len(occ) >= 20, len(occ)
    names = set()
    for k in occ:
        name = k.name.decode()
        names.add(name)
        assert k.block_threads in (256, 512, 1024), (name, k.block_threads)
        assert 0 < k.registers <= 512, (name, k.registers)
        assert k.blocks_per_cu >= 1, (name, k.blocks_per_cu)
        assert 0.0 < k.occupancy <= 1.0, (name, k.occupancy)
        assert k.limiter.decode() in ("registers", "lds", "waves"), (name, k.limiter)
        print(f"{name:55s} {k.block_threads:5d} thr {k.registers:4d} vgpr {k.lds_bytes:7d} B "
              f"{k.blocks_per_cu:2d} blk {k.occupancy:.3f} ({k.limiter.decode()})")
    gemm = [k for k in occ if k.name.decode().startswith("gemm_kernel 128x128x32, 8 waves")]
    assert gemm and gemm[0].lds_bytes > 0
    buf = C.create_string_buffer(1 << 16)
    n = eng.lib.eng_kernel_occupancy(buf, len(buf))
    assert n == len(occ)
    lines = buf.value.decode().strip().splitlines()
    assert {ln.split("|")[0] for ln in lines} == names
