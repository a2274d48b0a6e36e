"""The measurement entry points bench.py's floor and stamp legs use (no counterpart
in the reference): they run, they refuse what they do not take, and the stamped
matvec computes the same y as asmhip_matmul_q4_0, bit for bit."""

import numpy as np
import pytest

from asmllm_amd import native
from asmllm_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def _cus(hip) -> int:
    from asmllm_amd.device import device_info

    return int(device_info()["compute_units"])


def test_stamped_matvec_equals_plain_and_stamps_are_ordered(hip):
    M, K = 11008, 4096
    dw = DeviceBuffer(M * (K // 32) * 18)
    assert hip.asmhip_random_blocks(native.Q4_0, dw.ptr, M, K, 3, 0.02, None) == 0
    x = np.random.default_rng(1).standard_normal(K).astype(np.float32)
    dx, dy, dy2 = DeviceBuffer.from_numpy(x), DeviceBuffer(4 * M), DeviceBuffer(4 * M)
    grid = min((M + 15) // 16, _cus(hip))
    n = grid * 16 * 8
    ds = DeviceBuffer(8 * n)
    assert hip.asmhip_matmul_q4_0_stamped(dw.ptr, dx.ptr, dy.ptr, M, K, ds.ptr, n, None) == 0, hip.asmhip_last_error()
    assert hip.asmhip_matmul_q4_0(dw.ptr, dx.ptr, dy2.ptr, M, K, None) == 0
    synchronize()
    np.testing.assert_array_equal(dy.download(np.uint32, M), dy2.download(np.uint32, M))
    st = ds.download(np.uint64, (grid * 16, 8)).astype(np.int64)
    assert np.all(st > 0)
    # per wave, in program order: entry, loads issued, digits, first unit, last unit,
    # stream done, all waves done, y written
    for a in range(7):
        assert np.all(st[:, a] <= st[:, a + 1]), a
    span_us = (st[:, 7].max() - st[:, 0].min()) * 0.01
    assert 0.5 < span_us < 1000.0


def test_stamped_matvec_refuses_other_shapes(hip):
    d = DeviceBuffer(1 << 20)
    assert hip.asmhip_matmul_q4_0_stamped(d.ptr, d.ptr, d.ptr, 1024, 4096, d.ptr, 1 << 16, None) == \
        native.ERR_UNSUPPORTED  # M <= 2048: the nontemporal instantiation, not the headline's
    assert hip.asmhip_matmul_q4_0_stamped(d.ptr, d.ptr, d.ptr, 4096, 2048, d.ptr, 1 << 16, None) == \
        native.ERR_UNSUPPORTED
    M, K = 4096, 4096
    dw = DeviceBuffer(M * (K // 32) * 18)
    assert hip.asmhip_matmul_q4_0_stamped(dw.ptr, d.ptr, d.ptr, M, K, d.ptr, 10, None) == native.ERR_INVALID_ARGUMENT


def test_shaped_read_and_empty_launch_run(hip):
    nbytes = 25_422_848
    buf, sink = DeviceBuffer(nbytes), DeviceBuffer(4096)
    x = DeviceBuffer.from_numpy(np.full(4096, 0.5, np.float32))
    y_floats = 1 << 16
    y = DeviceBuffer(4 * y_floats)
    assert hip.asmhip_fill_f32(buf.ptr, nbytes // 4, 1.0, None) == 0
    for flags in (0, 1, 3, 7):
        assert hip.asmhip_stream_read_shaped(buf.ptr, nbytes, x.ptr, 4096, y.ptr, y_floats, flags, 155 * 1024,
                                             sink.ptr, None) == 0, hip.asmhip_last_error()
    for grid, threads, lds in ((256, 1024, 155 * 1024), (64, 64, 0)):
        assert hip.asmhip_empty_launch(grid, threads, lds, None) == 0, hip.asmhip_last_error()
    synchronize()
    # the store path wrote x's sum (2048) plus a bit of the loaded data into every workgroup's 16 floats
    out = y.download(np.float32, 16 * _cus(hip))
    assert np.all(np.isfinite(out))
    bad = native.ERR_INVALID_ARGUMENT
    assert hip.asmhip_stream_read_shaped(buf.ptr, nbytes, x.ptr, 4096, y.ptr, 16, 7, 0, sink.ptr, None) == bad
    assert hip.asmhip_stream_read_shaped(buf.ptr, nbytes, x.ptr + 4, 4096, y.ptr, y_floats, 2, 0, sink.ptr,
                                         None) == bad
    assert hip.asmhip_empty_launch(1, 2048, 0, None) == bad


def test_grid_barrier_completes(hip):
    counter, err = DeviceBuffer.from_numpy(np.zeros(64, np.uint32)), DeviceBuffer.from_numpy(np.zeros(64, np.uint32))
    rc = hip.asmhip_grid_barrier(counter.ptr, 50, err.ptr, None)
    if rc == native.ERR_UNSUPPORTED:
        pytest.skip("no cooperative launch on this device")
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    assert int(err.download(np.uint32, 1)[0]) == 0
    # every barrier added 2^31 in all: 50 barriers leave the counter where it started
    assert int(counter.download(np.uint32, 1)[0]) == 0
