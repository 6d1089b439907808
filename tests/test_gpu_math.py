"""Device arithmetic of the kernels against the host reference arithmetic.

expf (ec_expf.h) and SiLU must be bit-exact with the reference's glibc-based
formulas (the int8 path amplifies a last-bit difference); fp16 conversions
bit-exact with the F16C conversion of the reference; the activation
quantizer bit-exact with lrintf; GELU within one ulp of the reference (its
tanhf is glibc's; the device rounds a double tanh once).
"""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle

pytestmark = pytest.mark.gpu

OPS = {"expf": 0, "silu": 1, "gelu": 2, "f32_to_f16": 3, "f16_to_f32": 4, "quant1": 5}


def device(op, x):
    x = np.ascontiguousarray(x)
    out_dt = {3: np.uint16, 5: np.int8}.get(op, np.float32)
    din = ec.DeviceBuffer.from_array(x)
    dout = ec.DeviceBuffer(x.size * np.dtype(out_dt).itemsize)
    try:
        rc = ec.lib().ec_device_math(op, din.ptr, dout.ptr, x.size)
        assert rc == 0, ec.last_error()
        return dout.to_array(out_dt, x.shape)
    finally:
        din.close()
        dout.close()


def sample_floats(n, lo, hi, seed):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x) & (x > lo) & (x < hi)]
    dense = rng.uniform(lo, hi, n).astype(np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 88.72, -103.9, -87.0, 32.5351, -63.0994,
                        float.fromhex("0x1.04845ep+5"), float.fromhex("-0x1.f8cbb2p+5")], np.float32)
    return np.concatenate([x, dense, special]).astype(np.float32)


def same_bits(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.float32:
        nan = np.isnan(a) & np.isnan(b)
        return np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])
    return np.array_equal(a, b)


def test_expf_bit_exact():
    x = sample_floats(1 << 22, -110.0, 95.0, 1)
    x = np.concatenate([x, np.array([np.inf, -np.inf, np.nan], np.float32)])
    assert same_bits(device(0, x), oracle.map_op(0, x))


def test_silu_bit_exact():
    x = sample_floats(1 << 22, -100.0, 100.0, 2)
    assert same_bits(device(1, x), oracle.map_op(1, x))


def test_gelu_within_tanh_ulp():
    """0.5x(1 + tanh(u)): the device tanh is within one ulp of glibc's tanhf,
    so the results differ by at most ~|x/2| * ulp(tanh) plus final roundings
    (relative error is unbounded where 1 + tanh(u) cancels, x << 0)."""
    x = sample_floats(1 << 20, -20.0, 20.0, 3)
    got, want = device(2, x), oracle.map_op(2, x)
    bound = 2.0 * np.abs(0.5 * x.astype(np.float64)) * 2.0 ** -23 + 4 * np.spacing(np.abs(want))
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)
    assert np.mean(got == want) > 0.9


def test_fp16_conversions_bit_exact():
    rng = np.random.default_rng(4)
    bits = rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32),
                        np.array([65504, 65519.99, 65520, 1e-8, 2.98e-8, 6.1e-5, -0.0], np.float32)])
    x = x[~np.isnan(x)]
    assert np.array_equal(device(3, x), oracle.map_op(3, x))
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert same_bits(device(4, h), oracle.map_op(4, h))


def test_quant1_ties_and_clamp():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 127.5, 128.0, -128.5, -200.0, 1e9, np.nan,
                  np.inf, -np.inf, 0.49999997, 3.5000002], np.float32)
    x = np.concatenate([x, sample_floats(1 << 16, -300.0, 300.0, 5)])
    assert np.array_equal(device(5, x), oracle.map_op(5, x))
