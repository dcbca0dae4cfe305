"""The C ABI driven from plain C on the GPU (tests/c/abi_gpu.c, no Python or torch in its code): device buffers
from hipMalloc, the table update and the owner sum with the fused norm through include/yoco_z1.h, checked against
the oracle's C functions.  Its abi_gpu_run() is called in-process from tests/c/libabi_gpu.so, built by
__graft_entry__.build()."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'c', 'libabi_gpu.so')


def test_plain_c_consumer_on_gpu(pkg, dev):
    if not os.path.exists(LIB):
        pytest.fail(f'{LIB} is missing: run __graft_entry__.build() first')
    lib = ctypes.CDLL(LIB)           # after torch (the conftest imports it): one HIP runtime in the process
    lib.abi_gpu_run.restype = ctypes.c_int
    assert lib.abi_gpu_run() == 0
