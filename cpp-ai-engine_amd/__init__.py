"""cpp-ai-engine on MI355X: the HIP backend of the fp32 training path.

The product is native: lib/libehip.so (kernels and the C ABI of include/ehip.h)
and lib/libengine_hip.so (the C++ Tensor/autograd/nn/optim engine on top of it).
This package file only locates and loads them for Python callers (tests, bench).
"""
import os

ROOT = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(ROOT, "lib")
EHIP_SO = os.path.join(LIB_DIR, "libehip.so")
