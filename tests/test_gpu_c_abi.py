"""The C ABI driven from plain C (tests/c_abi/harness.c, built by the build
step into tests/c_abi/libjlust_c_harness.so): known answers for SpMV (both
origins), a prepared SpMV plan's life cycle, SpMM, SDDMM and the error path,
with device memory from the HIP runtime and no Python or torch between the
caller and the library.  Loaded and called in this process."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "libjlust_c_harness.so")


def test_c_harness():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert os.path.exists(HARNESS), f"{HARNESS} is missing: run __graft_entry__.build() first"
    from jlust_amd import _lib
    _lib.lib()                                  # the library this process already uses
    h = ctypes.CDLL(HARNESS)
    h.jlust_c_harness_run.restype = ctypes.c_int
    h.jlust_c_harness_run.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    buf = ctypes.create_string_buffer(512)
    rc = h.jlust_c_harness_run(buf, len(buf))
    assert rc == 0, f"C harness check {rc}: {buf.value.decode()}"
