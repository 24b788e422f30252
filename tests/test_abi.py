"""The C ABI without a GPU: the library loads, exports exactly what include/ehip.h
declares, and reports a missing device as an error status instead of crashing."""
import ctypes
import os

import pytest

import ehip as E

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def lib():
    return E.load_library()


def test_header_declares_the_boundary():
    names = E.header_symbols()
    assert len(names) >= 45, names
    for must in ("ehip_gemm_f32", "ehip_adam_f32", "ehip_softmax_xent_backward_f32",
                 "ehip_im2col_f32", "ehip_col2im_f32", "ehip_maxpool_f32",
                 "ehip_layernorm_backward_f32", "ehip_arena_alloc"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in E.header_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert set(E.header_symbols()) == set(E._SIGS), \
        set(E.header_symbols()) ^ set(E._SIGS)


def test_header_has_no_torch_or_hip_types():
    import re
    text = re.sub(r"/\*.*?\*/", "", open(E.HEADER).read(), flags=re.S)
    for banned in ("torch", "at::", "hipStream_t", "c10", "std::", "hip/"):
        assert banned not in text, banned


def test_no_device_is_an_error_not_a_crash(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert lib.ehip_init() == 3  # EHIP_ENODEV
    assert b"device" in lib.ehip_last_error()
    assert lib.ehip_available() == 0
    assert lib.ehip_relu_f32(None, None, 16, None) == 3
    p = ctypes.c_void_p()
    assert lib.ehip_arena_alloc(1024, ctypes.byref(p)) == 3 and not p.value


def test_igemm_supported_is_a_pure_query(lib):
    """ehip_conv2d_igemm_supported needs no device and says 0 beyond the implicit GEMM's
    limits (65535 images; 2^31 output pixels over the batch), where the engine composes
    im2col + GEMM instead."""
    def win(n, c, h, w, k=3, s=1, p=1):
        oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
        return E.Window(n, c, h, w, k, k, s, p, oh, ow)
    f = lib.ehip_conv2d_igemm_supported
    assert f(ctypes.byref(win(32, 64, 28, 28)), 128) == 1
    assert f(ctypes.byref(win(65535, 64, 4, 4)), 128) == 1
    assert f(ctypes.byref(win(65536, 64, 4, 4)), 128) == 0
    assert f(ctypes.byref(win(4096, 3, 1024, 1024)), 16) == 0
    assert f(None, 16) == 0 and f(ctypes.byref(win(1, 1, 4, 4)), 0) == 0


def test_control_queries_without_a_device(lib):
    """The version and occupancy queries report a missing device as a status, and the
    compiled-in HIP version is known without one."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    v = [ctypes.c_int(-1) for _ in range(3)]
    lib.ehip_version_info(*[ctypes.byref(x) for x in v])
    assert v[0].value >= 60000000, v[0].value  # HIP 6.0 or later in HIP's encoding
    count = ctypes.c_int(-1)
    assert lib.ehip_kernel_occupancy(None, 0, ctypes.byref(count)) == 3  # EHIP_ENODEV
