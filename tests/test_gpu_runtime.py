"""GPU: the runtime's device buffers.  A buffer made from a byte count has no host
shape, so reading it back needs an output array of at least its size; anything
else is refused before any copy (a copy into a smaller host array would overrun
it)."""

from __future__ import annotations

import numpy as np
import pytest

from tilegen_amd import runtime as rt

pytestmark = pytest.mark.gpu


def test_to_host_needs_a_large_enough_output(hip_ready):
    src = rt.DeviceBuffer(np.arange(4, dtype=np.float64))
    raw = rt.DeviceBuffer(nbytes=32)
    try:
        assert rt.lib().tg_memcpy_dtod(raw.ptr, src.ptr, 32) == 0
        with pytest.raises(ValueError, match="out="):
            raw.to_host()
        with pytest.raises(ValueError, match="32 bytes"):
            raw.to_host(np.empty(3))
        with pytest.raises(ValueError, match="C-contiguous"):
            raw.to_host(np.empty((4, 2))[:, 0])
        assert raw.to_host(np.empty(4)).tolist() == [0.0, 1.0, 2.0, 3.0]
        assert src.to_host().tolist() == [0.0, 1.0, 2.0, 3.0]
    finally:
        src.free()
        raw.free()
