"""GPU checks of the benchmark's runtime helpers: the seeded draft source that a replayed round
graph uses (one table row per call, the counter advanced on the device, also under graph replay)
and the bandwidth controls (the stream copy moves every byte; both read forms complete on payloads
that end inside a 4 KiB chunk and leave the sink untouched)."""
import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import device
from ninfer_amd.device import DeviceArray, DeviceBuffer, Graph, Stream, synchronize

pytestmark = pytest.mark.gpu


def test_next_row_cycles_the_table_eagerly_and_in_a_graph():
    rows, cols = 5, 3
    table = np.arange(rows * cols, dtype=np.int32).reshape(rows, cols) * 7 + 1
    dt = DeviceArray.from_numpy(na.I32, table, (cols, rows))
    ctr = DeviceArray.from_numpy(na.I32, np.array([0], np.int32), (1,))
    dst = DeviceArray(na.I32, (cols,))
    s = Stream()
    for i in range(7):
        device.next_row_i32(dt, ctr, dst, s)
        s.synchronize()
        np.testing.assert_array_equal(dst.numpy(), table[i % rows])
    assert int(ctr.numpy()[0]) == 7
    g = Graph(s)
    with g:
        device.next_row_i32(dt, ctr, dst, s)
    for i in range(7, 13):
        g.launch()
        s.synchronize()
        np.testing.assert_array_equal(dst.numpy(), table[i % rows])
    assert int(ctr.numpy()[0]) == 13


@pytest.mark.parametrize("nbytes", [16, 4096 * 37 + 48, (3 << 20) + 4096 * 5 + 2032])
def test_bandwidth_controls(nbytes):
    s = Stream()
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 256, nbytes, dtype=np.uint8)
    src, dst = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    src.upload(host)
    dst.fill(0, s)
    sink = DeviceBuffer(256)
    sink.fill(0xAB, s)
    device.stream_copy(dst.ptr, src.ptr, nbytes, s)
    device.read_ceiling(src.ptr, nbytes, device.READ_VECTOR, sink, s)
    device.read_ceiling(src.ptr, nbytes, device.READ_LDS_DMA, sink, s)
    s.synchronize()
    np.testing.assert_array_equal(dst.download(np.uint8, nbytes), host)
    assert (sink.download(np.uint8, 256) == 0xAB).all()
    synchronize()
