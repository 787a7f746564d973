"""The gather probe (f3s_probe_gather, a measurement helper of bench.py):
each wave's output word is the XOR of every 32-bit word of the K and V rows
(first 128 bytes at the row stride) of its columns -- checked against numpy,
so the probe's loads are the ones it claims to make."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,cpw,cols", [(1, 8, 32 * 8 * 5), (3, 1, 32 * 7), (2, 4, 32 * 37)])
def test_probe_gather_folds_the_named_rows(gpu, H, cpw, cols):
    rows = 5000
    r = rng(70 + H)
    k = r.integers(0, 2**16, (rows, H, 64), dtype=np.uint16)
    v = r.integers(0, 2**16, (rows, H, 64), dtype=np.uint16)
    idx = r.integers(0, rows, cols, dtype=np.int64).astype(np.int32)
    dk, dv = gpu.DeviceArray.from_numpy(k), gpu.DeviceArray.from_numpy(v)
    didx = gpu.DeviceArray.from_numpy(idx)
    nw = (cols // 32 + cpw - 1) // cpw
    out = gpu.DeviceArray((nw,), np.uint32)
    gpu.probe_gather(dk, dv, rows, H * 128, didx, out, cpw)
    gpu.synchronize()
    got = out.numpy()
    # head 0 of each row, as 32-bit words
    kw = k[:, 0, :].copy().view(np.uint32)
    vw = v[:, 0, :].copy().view(np.uint32)
    per_col = np.bitwise_xor.reduce(kw[idx] ^ vw[idx], axis=1)
    want = np.array([np.bitwise_xor.reduce(per_col[w * cpw * 32:(w + 1) * cpw * 32])
                     for w in range(nw)], np.uint32)
    assert np.array_equal(got, want)


def test_probe_gather_rejects_bad_shapes(gpu):
    k = gpu.DeviceArray((64, 64), np.uint16, zero=True)
    idx = gpu.DeviceArray.from_numpy(np.zeros(31, np.int32))
    out = gpu.DeviceArray((4,), np.uint32)
    with pytest.raises(gpu.F3SError):
        gpu.probe_gather(k, k, 64, 128, idx, out)          # not a multiple of 32
    idx32 = gpu.DeviceArray.from_numpy(np.zeros(32, np.int32))
    with pytest.raises(gpu.F3SError):
        gpu.probe_gather(k, k, 64, 100, idx32, out)        # stride below a row
