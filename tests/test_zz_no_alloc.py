"""The self check without a device allocation against the allocating one.

nanorts_amd_self_check_no_alloc keeps its probe words in the library's own
per-device array instead of a hipMalloc'd buffer.  Two calls in a row, the
second with fewer probe waves, must each agree with nanorts_amd_self_check
and write back exactly their own probe words."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_no_alloc_self_check_matches_the_allocating_one():
    import torch

    from nanorts_amd import native

    print("no-alloc self check", flush=True)
    torch.cuda.set_device(0)
    lib = native.load()
    device = (ctypes.c_int32 * 1)(0)
    want = lib.nanorts_amd_self_check(device, 1).decode()
    assert want == ""
    for waves in (1024, 5):
        words = np.full(1024, -3, np.int32)
        got = lib.nanorts_amd_self_check_no_alloc(device, 1, waves, words.ctypes.data_as(ctypes.c_void_p)).decode()
        assert got == want
        assert (words[:waves] == 1).all(), words[:waves]
        assert (words[waves:] == -3).all()
    assert lib.nanorts_amd_self_check(device, 1).decode() == want
