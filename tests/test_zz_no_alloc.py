"""ec_topk_dev_noalloc -- the device top-k selection with its scratch in the
library's file-scope device array instead of allocations -- against
ec_topk_dev, which allocates its scratch: identical values, indices and
status, bit for bit, on two calls in a row, the second with a smaller input
(fewer rows, a smaller vocabulary, a smaller k) than the first; and a call
needing more scratch than the array holds is refused with a message."""
import ctypes as C

import numpy as np
import pytest

import edgecore_amd as ec

pytestmark = pytest.mark.gpu


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _topk(name, logits, top_k):
    rows, V = logits.shape
    buf = ec.DeviceBuffer.from_array(np.ascontiguousarray(logits, np.float32))
    try:
        vals = np.full((rows, top_k + 1), np.nan, np.float32)
        idx = np.full((rows, top_k + 1), -1, np.int32)
        status = np.full(rows, -1, np.int32)
        rc = getattr(ec.lib(), name)(buf.ptr, rows, V, V, top_k, _ptr(vals), _ptr(idx), _ptr(status))
        assert rc == 0, ec.last_error()
        return vals, idx, status
    finally:
        buf.close()


def test_noalloc_topk_equals_allocating_twice():
    rng = np.random.default_rng(11)
    first = rng.normal(0, 3, (8, 151936)).astype(np.float32)
    first[2, 1000:1010] = first[2].max() + 1.0  # a tie at the top
    first[5, 7] = np.nan                         # status 1: the whole row is needed
    second = rng.normal(0, 1, (3, 50257)).astype(np.float32)
    for logits, k in ((first, 40), (second, 7)):
        got = _topk("ec_topk_dev_noalloc", logits, k)
        want = _topk("ec_topk_dev", logits, k)
        assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
        assert np.array_equal(got[1], want[1]) and np.array_equal(got[2], want[2])
    assert list(want[2]) == [0, 0, 0]


def test_noalloc_topk_refuses_oversize():
    rows, V, k = 200, 151936, 128  # ~8 MB of scratch, above the array's 4 MiB
    buf = ec.DeviceBuffer(rows * V * 4)
    try:
        vals = np.empty((rows, k + 1), np.float32)
        idx = np.empty((rows, k + 1), np.int32)
        status = np.empty(rows, np.int32)
        rc = ec.lib().ec_topk_dev_noalloc(buf.ptr, rows, V, V, k, _ptr(vals), _ptr(idx), _ptr(status))
        assert rc < 0 and "scratch" in ec.last_error()
    finally:
        buf.close()
