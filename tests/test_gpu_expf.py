"""The device's binary:logistic sigmoid against the host libm on all 2^32
binary32 inputs: the prediction transform (mgb_transform, which shares the
gradient kernel's sigmoid) runs over every bit pattern on the GPU, and a
position-weighted checksum of the output bits is compared with the same
checksum of upstream XGBoost's sigmoid over the host's expf
(tests/expf_sweep.cpp).  A position weight 2i + 1 is odd, so any single
differing output changes the sum."""
import ctypes

import numpy as np
import pytest

import device_lib as D
import expf_build

pytestmark = pytest.mark.gpu


def test_device_sigmoid_equals_host_libm_on_all_inputs():
    host = int(expf_build.run("checksum").split()[1])
    chunk = 1 << 27
    buf = D.Device(chunk * 4)
    total = np.uint64(0)
    with np.errstate(over="ignore"):
        for start in range(0, 1 << 32, chunk):
            index = np.arange(start, start + chunk, dtype=np.uint64)
            bits = index.astype(np.uint32)
            D.check(D.lib().mgb_memcpy_h2d(buf.ptr, bits.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(chunk * 4)))
            D.check(D.lib().mgb_transform(buf.ptr, ctypes.c_uint64(chunk), ctypes.c_uint32(1)))
            out = buf.read(np.uint32, chunk)
            values = out.view(np.float32)
            canon = np.where(np.isnan(values), np.uint32(0x7FC00000), out).astype(np.uint64)
            total += np.sum(canon * (2 * index + 1), dtype=np.uint64)
    assert int(total) == host
