"""ec_topk_dev_noalloc -- the device top-k selection with its scratch in the
library's file-scope device array instead of allocations -- against
ec_topk_dev, which allocates its scratch: identical values, indices and
status, bit for bit, on two calls in a row, the second with a smaller input
(fewer rows, a smaller vocabulary, a smaller k) than the first; a call
needing more scratch than the array holds is refused with a message; and, as
the first call into the library of a fresh process, on logits that the
process allocated through the HIP runtime itself, it makes no allocation."""
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


_FIRST_CALL = r"""
import ctypes as C, json, sys
import numpy as np
hip = C.CDLL("libamdhip64.so")
import edgecore_amd as ec
rows, V, k = 4, 151936, 40
rng = np.random.default_rng(5)
logits = rng.normal(0, 2, (rows, V)).astype(np.float32)
p = C.c_void_p()
assert hip.hipMalloc(C.byref(p), C.c_size_t(logits.nbytes)) == 0
assert hip.hipMemcpy(p, logits.ctypes.data_as(C.c_void_p), C.c_size_t(logits.nbytes), 1) == 0  # host to device
vals = np.empty((rows, k + 1), np.float32)
idx = np.empty((rows, k + 1), np.int32)
status = np.empty(rows, np.int32)
L = ec.lib()
rc = L.ec_topk_dev_noalloc(p, rows, V, V, k, vals.ctypes.data_as(C.c_void_p), idx.ctypes.data_as(C.c_void_p),
                           status.ctypes.data_as(C.c_void_p))
print(json.dumps({"rc": rc, "err": ec.last_error(), "allocs": L.ec_alloc_count(), "idx": idx.tolist(),
                  "vals": vals.view(np.uint32).tolist(), "status": status.tolist()}))
"""


def test_noalloc_topk_first_call_allocates_nothing():
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL], cwd=root, env=dict(os.environ), capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["rc"] == 0, out["err"]
    assert out["allocs"] == 0
    rng = np.random.default_rng(5)
    logits = rng.normal(0, 2, (4, 151936)).astype(np.float32)
    idx = np.array(out["idx"], np.int32)
    for r_ in range(4):
        want = np.lexsort((np.arange(151936), -logits[r_]))[:41]
        assert list(idx[r_]) == list(want)
        assert np.array_equal(np.array(out["vals"][r_], np.uint32), logits[r_][want].view(np.uint32))
    assert out["status"] == [0, 0, 0, 0]
