"""GPU parity of the kernel ABI (src/kernels.c:129-168, src/gpt2.c:446-461)
against the CPU oracle, through the C ABI of libedgecore_hip.so.

int8: bit-exact (exact int32 dot, same epilogue rounding sequence).
fp16/bf16: fp32 accumulation in a different order than the reference's
8-lane AVX2 order; bounded by |gpu - ref| <= 2 * K * 2^-24 * sum_k |a_k b_k|
(+1e-30), and checked against a float64 brute force with the same bound.
"""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle

pytestmark = pytest.mark.gpu

I8_SHAPES = [
    (1, 896, 1152), (1, 896, 896), (1, 4864, 896), (1, 896, 4864),  # Qwen2-0.5B decode
    (1, 1536, 256), (1, 8960, 1536),                                  # Qwen2.5-1.5B
    (3, 896, 896), (8, 4864, 896), (16, 1536, 1536), (37, 896, 1152),  # batched / prefill
    (256, 896, 1152), (300, 4864, 896), (64, 896, 4864),              # matrix-core tiles
    (130, 64, 192), (17, 1040, 200), (33, 16, 129),                   # K, M and N tails
    (1, 64, 192), (2, 256, 64),                                       # tiny GPT-2
    (5, 40, 7), (2, 1, 3), (3, 17, 33),                               # odd K: generic path
]


def _rand_i8(rng, shape):
    return rng.integers(-128, 128, size=shape, dtype=np.int16).astype(np.int8)


@pytest.mark.parametrize("M,K,N", I8_SHAPES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_int8_bit_exact(M, K, N, with_bias):
    rng = np.random.default_rng(M * 7 + K * 13 + N)
    A = _rand_i8(rng, (M, K))
    B = _rand_i8(rng, (N, K))
    a_s = rng.uniform(1e-4, 1e-1, M).astype(np.float32)
    b_s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    bias = rng.normal(0, 0.02, N).astype(np.float32) if with_bias else None
    got = ec.gemm_int8(A, a_s, B, b_s, bias)
    want = oracle.gemm_int8(A, a_s, B, b_s, bias)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemm_int8_null_scale_and_adversarial():
    K = 4864
    A = np.full((2, K), -128, np.int8)
    A[1] = 127
    B = np.full((3, K), -128, np.int8)
    B[1] = 127
    B[2, ::2] = 127
    a_s = np.array([1.0, 0.5], np.float32)
    got = ec.gemm_int8(A, a_s, B, None, None)
    want = oracle.gemm_int8(A, a_s, B, None, None)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the exact dots: (-128)(-128)K, (-128)(127)K, 127*127*K ...
    assert got[0, 0] == np.float32(float(128 * 128 * K))
    assert got[1, 1] == np.float32(float(127 * 127 * K) * 0.5)


def _f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def _bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


W16_SHAPES = [(1, 896, 151936), (1, 768, 2304), (1, 3072, 768), (4, 896, 4864), (9, 64, 50257),
              (2, 37, 5), (1, 8, 3)]


@pytest.mark.parametrize("M,K,N", W16_SHAPES)
@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_w16_within_bound(M, K, N, bf16):
    rng = np.random.default_rng(M + K + N + bf16)
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    Wf = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    B = _bf16_bits(Wf) if bf16 else _f16_bits(Wf)
    got = (ec.gemm_bf16_fp32 if bf16 else ec.gemm_fp16_fp32)(A, B)
    want = oracle.gemm_w16(A, B, bf16=bf16)
    Bf = (B.astype(np.uint32) << 16).view(np.float32) if bf16 else B.view(np.float16).astype(np.float32)
    exact = A.astype(np.float64) @ Bf.astype(np.float64).T
    bound = 2.0 * K * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(Bf).astype(np.float64).T) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    assert np.all(np.abs(want - exact) <= bound)


def test_quantize_rows_bit_exact_with_ties():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (6, 896)).astype(np.float32)
    # row 1: exact .5 ties after division by s = 127/127 = 1 -> maxabs 127
    x[1, :] = np.linspace(-127, 127, 896).astype(np.float32)
    x[1, :8] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 127.0, -126.5]
    x[2, :] = 0.0  # all-zero row: scale 1, codes 0
    x[3, 5] = np.inf
    x[4, 7] = np.nan
    src = ec.DeviceBuffer.from_array(x)
    q = ec.DeviceBuffer(x.size)
    s = ec.DeviceBuffer(4 * x.shape[0])
    try:
        rc = ec.lib().ec_quantize_rows_dev(src.ptr, x.shape[0], x.shape[1], q.ptr, s.ptr)
        assert rc == 0, ec.last_error()
        gq = q.to_array(np.int8, x.shape)
        gs = s.to_array(np.float32, x.shape[0])
    finally:
        for b in (src, q, s):
            b.close()
    oq, os_ = oracle.quantize_rows(x)
    assert np.array_equal(gq, oq)
    assert np.array_equal(gs.view(np.uint32), os_.view(np.uint32))
    assert list(gq[1, :6]) == [0, 2, 2, 0, -2, -2]
    assert gs[2] == 1.0 and not gq[2].any()


@pytest.mark.parametrize("M,K", [(16, 8960), (3, 37), (2, 4100), (40, 1536)])
def test_quantize_rows_vector_and_scalar_paths(M, K):
    """K % 4 == 0 takes the float4 kernel, other K the scalar one; both give
    the oracle's codes and scales bit for bit."""
    rng = np.random.default_rng(M * K)
    x = rng.normal(0, 2, (M, K)).astype(np.float32)
    x[0, K // 2] = 0.5 * np.abs(x).max() * 2  # a row max inside the row
    src = ec.DeviceBuffer.from_array(x)
    q = ec.DeviceBuffer(x.size)
    s = ec.DeviceBuffer(4 * M)
    try:
        assert ec.lib().ec_quantize_rows_dev(src.ptr, M, K, q.ptr, s.ptr) == 0, ec.last_error()
        gq = q.to_array(np.int8, x.shape)
        gs = s.to_array(np.float32, M)
    finally:
        for b in (src, q, s):
            b.close()
    oq, os_ = oracle.quantize_rows(x)
    assert np.array_equal(gq, oq)
    assert np.array_equal(gs.view(np.uint32), os_.view(np.uint32))


def test_dev_entry_points_reject_bad_shapes():
    L = ec.lib()
    assert L.ec_gemm_int8_dev(None, None, None, None, None, None, -1, 4, 4) < 0
    assert "negative" in ec.last_error()
    assert L.ec_gemm_fp16_fp32_dev(None, None, None, 2, 16, 4) < 0
    assert L.ec_gemm_int8_dev(None, None, None, None, None, None, 0, 4, 4) == 0


# ------------------------------------------------------------------ matrix-core tiles x epilogues
# ec_gemm_int8_epi_dev runs the prefill linears' int8 matrix-core GEMM with
# every fused epilogue and each row tile (32, 64, 128 rows), on shapes with
# row and column tails; 0 lets the library pick, as the forward does (the
# C4 shapes: gate/up of 2048 rows takes 128-row tiles, qkv 64-row tiles).
TILE_SHAPES = [(200, 896, 300), (130, 1536, 129), (257, 64, 200), (64, 4864, 128)]


def _epi_inputs(M, K, N, seed):
    rng = np.random.default_rng(seed)
    A = _rand_i8(rng, (M, K))
    B = _rand_i8(rng, (N, K))
    B2 = _rand_i8(rng, (N, K))
    a_s = rng.uniform(1e-4, 1e-2, M).astype(np.float32)
    b_s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    b2_s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    bias = rng.normal(0, 0.02, N).astype(np.float32)
    C0 = rng.normal(0, 1.0, (M, N)).astype(np.float32)
    return A, B, B2, a_s, b_s, b2_s, bias, C0


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _device_gelu(v):
    din = ec.DeviceBuffer.from_array(np.ascontiguousarray(v, np.float32))
    dout = ec.DeviceBuffer(v.size * 4)
    try:
        assert ec.lib().ec_device_math(2, din.ptr, dout.ptr, v.size) == 0, ec.last_error()
        return dout.to_array(np.float32, v.shape)
    finally:
        din.close()
        dout.close()


@pytest.mark.parametrize("bm", [32, 64, 128])
@pytest.mark.parametrize("M,K,N", TILE_SHAPES)
def test_gemm_int8_tiles_and_epilogues(bm, M, K, N):
    A, B, B2, a_s, b_s, b2_s, bias, C0 = _epi_inputs(M, K, N, seed=M + K + N + bm)
    v = oracle.gemm_int8(A, a_s, B, b_s, bias)
    store = ec.gemm_int8_epi(0, bm, A, a_s, B, b_s, bias=bias)
    assert np.array_equal(_bits(store), _bits(v))
    resid = ec.gemm_int8_epi(1, bm, A, a_s, B, b_s, bias=bias, C0=C0)
    assert np.array_equal(_bits(resid), _bits(C0 + v))
    # GELU: the device's gelu_new (checked against the reference's in
    # test_gpu_math) applied to the exact linear value
    gelu = ec.gemm_int8_epi(2, bm, A, a_s, B, b_s, bias=bias)
    assert np.array_equal(_bits(gelu), _bits(_device_gelu(v)))
    g = oracle.gemm_int8(A, a_s, B, b_s)
    u = oracle.gemm_int8(A, a_s, B2, b2_s)
    swi = ec.gemm_int8_epi(3, bm, A, a_s, B, b_s, B2=B2, b2_scale=b2_s)
    assert np.array_equal(_bits(swi), _bits(oracle.map_op(1, g) * u))


@pytest.mark.parametrize("M,K,N", [(2048, 896, 2048), (1024, 1536, 4096), (1000, 896, 2120), (2040, 896, 2100)])
def test_gemm_int8_auto_tile_prefill_shapes(M, K, N):
    """Shapes whose automatic tile is 128 rows (2048x2048, 1024x4096,
    2040x2100) or 64 rows (1000x2120), with row and column tails."""
    A, B, B2, a_s, b_s, b2_s, bias, C0 = _epi_inputs(M, K, N, seed=M ^ N)
    store = ec.gemm_int8_epi(0, 0, A, a_s, B, b_s, bias=bias)
    assert np.array_equal(_bits(store), _bits(oracle.gemm_int8(A, a_s, B, b_s, bias)))
    swi = ec.gemm_int8_epi(3, 0, A, a_s, B, b_s, B2=B2, b2_scale=b2_s)
    want = oracle.map_op(1, oracle.gemm_int8(A, a_s, B, b_s)) * oracle.gemm_int8(A, a_s, B2, b2_s)
    assert np.array_equal(_bits(swi), _bits(want))


# ------------------------------------------------------------------ 16-bit weights on the matrix cores
# ec_gemm_w16_epi_dev / ec_gemm_{fp16,bf16}_fp32_dev at M >= 16: the fp32
# rows are split into 16-bit parts (fp16: 2 under a per-row 2^e; bf16: 3),
# multiplied exactly and summed in fp32.  Every value is checked against the
# float64 product with the fp32 bound of the vector path (2 K 2^-24 sum|a b|),
# propagated through the epilogue.
W16_MFMA_SHAPES = [(16, 768, 2304), (128, 768, 3072), (40, 3072, 768), (100, 896, 1000), (257, 64, 200),
                   (33, 1536, 129)]


def _w16_inputs(M, K, N, bf16, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    A = (rng.normal(0, 1, (M, K)) * scale).astype(np.float32)
    mk = _bf16_bits if bf16 else _f16_bits
    B, B2 = (mk(rng.normal(0, 0.02, (N, K)).astype(np.float32)) for _ in range(2))
    bias = rng.normal(0, 0.02, N).astype(np.float32)
    C0 = rng.normal(0, 1.0, (M, N)).astype(np.float32)
    return A, B, B2, bias, C0


def _w16_f64(B, bf16):
    return ((B.astype(np.uint32) << 16).view(np.float32) if bf16 else B.view(np.float16)).astype(np.float64)


def _exact_and_bound(A, B, bf16):
    Bf = _w16_f64(B, bf16)
    A64 = A.astype(np.float64)
    K = A.shape[1]
    return A64 @ Bf.T, 2.0 * K * 2.0 ** -24 * (np.abs(A64) @ np.abs(Bf).T) + 1e-30


def _gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def _silu64(x):
    return x / (1.0 + np.exp(-x))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", W16_MFMA_SHAPES)
def test_gemm_w16_matrix_core_within_bound(M, K, N, bf16):
    A, B, _, _, _ = _w16_inputs(M, K, N, bf16, seed=M * 3 + K + N + bf16)
    got = (ec.gemm_bf16_fp32 if bf16 else ec.gemm_fp16_fp32)(A, B)
    exact, bound = _exact_and_bound(A, B, bf16)
    assert np.all(np.abs(got - exact) <= bound)
    # the split keeps far more than the bound needs: typically within a few fp32 ulps
    assert np.median(np.abs(got - exact) / (np.abs(exact) + 1e-30)) < 1e-6


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("bm,M,K,N", [(bm, M, K, N) for bm in (0, 32, 64, 128)
                                      for M, K, N in ((200, 768, 300), (130, 3072, 129), (64, 896, 128),
                                                      (128, 3072, 768))]
                         + [(bm, M, K, N) for bm in (0, 16)
                            for M, K, N in ((16, 1536, 600), (32, 768, 129), (20, 3072, 200), (1, 8, 17),
                                            (16, 768, 16500))])
def test_gemm_w16_tiles_and_epilogues(bm, M, K, N, bf16):
    wt = 2 if bf16 else 1
    A, B, B2, bias, C0 = _w16_inputs(M, K, N, bf16, seed=M + K + N + bm + 7 * bf16)
    v, bv = _exact_and_bound(A, B, bf16)
    b64, c64 = bias.astype(np.float64), C0.astype(np.float64)
    ulp = 2.0 ** -23

    def check(got, want, tol):
        assert np.all(np.abs(got.astype(np.float64) - want) <= tol + 2 * ulp * np.abs(want) + 1e-30)

    check(ec.gemm_w16_epi(wt, 0, bm, A, B, bias=bias), v, bv)             # store: bias ignored
    check(ec.gemm_w16_epi(wt, 4, bm, A, B, bias=bias), v + b64, bv)       # store + bias
    check(ec.gemm_w16_epi(wt, 1, bm, A, B, C0=C0), c64 + v, bv)           # residual
    check(ec.gemm_w16_epi(wt, 5, bm, A, B, bias=bias, C0=C0), c64 + (v + b64), bv)
    check(ec.gemm_w16_epi(wt, 2, bm, A, B), _gelu64(v), 1.2 * bv + 1e-6)  # GELU (tanh form)
    check(ec.gemm_w16_epi(wt, 6, bm, A, B, bias=bias), _gelu64(v + b64), 1.2 * bv + 1e-6)
    u, bu = _exact_and_bound(A, B2, bf16)
    want = _silu64(v) * u
    tol = 1.1 * (np.abs(u) * bv + np.abs(_silu64(v)) * bu) + 1e-6 * np.abs(want)
    check(ec.gemm_w16_epi(wt, 3, bm, A, B, B2=B2), want, tol)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", [(128, 3072, 768), (130, 3072, 129), (40, 3072, 768)])
def test_gemm_w16_split_k_repeatable(M, K, N, bf16):
    """Few tiles over long rows run split K (the tile's K stages over
    several blocks, the partial tiles added in a fixed order by the last
    block): the same call gives the same bits every time, with the
    residual epilogue reading C0 while other blocks of the tile still run."""
    wt = 2 if bf16 else 1
    A, B, _, bias, C0 = _w16_inputs(M, K, N, bf16, seed=K + N + bf16)
    first = ec.gemm_w16_epi(wt, 5, 32, A, B, bias=bias, C0=C0)
    for _ in range(3):
        assert np.array_equal(_bits(ec.gemm_w16_epi(wt, 5, 32, A, B, bias=bias, C0=C0)), _bits(first))
    v, bv = _exact_and_bound(A, B, bf16)
    want = C0.astype(np.float64) + (v + bias.astype(np.float64))
    assert np.all(np.abs(first - want) <= bv + 2 * 2.0 ** -23 * np.abs(want) + 1e-30)


@pytest.mark.parametrize("scale", [1e-30, 1e-8, 1e4, 3e5, 1e30])
def test_gemm_fp16_matrix_core_row_scale_range(scale):
    """fp16 parts hold 2^-e x with e from each row's largest |x|: rows far
    outside fp16 range (1e30, 3e5 > 65504) or deep in its subnormals
    (1e-30) keep fp32-level accuracy.  One row is all zeros."""
    M, K, N = 32, 768, 256
    A, B, _, _, _ = _w16_inputs(M, K, N, False, seed=11, scale=scale)
    A[3] = 0.0
    got = ec.gemm_fp16_fp32(A, B)
    exact, bound = _exact_and_bound(A, B, False)
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - exact) <= bound)
    assert not got[3].any()


# ------------------------------------------------------------------ skinny int8 GEMM (M <= 32)
# bm=16 forces the batched-decode kernel: one block per 16 output columns,
# MFMA fragments straight from global memory, K split over up to 16 waves
# whose exact int32 partial tiles are summed through LDS.  Up to 16 rows with
# K >= 4096 and fewer than 192 column tiles also split K over several blocks
# per 64 columns (the last block to finish adds their int32 tiles):
# (16, 8960, 1536), (16, 4864, 896), (1, 4864, 70), (9, 4112, 200) and
# (16, 5008, 2900).  Shapes give few and many K steps per wave, row / column /
# K tails and both row fragments.
SKINNY_SHAPES = [(16, 8960, 1536), (16, 1536, 2048), (16, 4864, 896), (32, 8960, 300), (20, 1040, 200),
                 (17, 16, 129), (1, 4864, 70), (25, 2048, 8960), (16, 896, 17000),  # 4 tiles per block
                 (9, 4112, 200), (16, 5008, 2900)]


@pytest.mark.parametrize("M,K,N", SKINNY_SHAPES)
def test_gemm_int8_skinny_epilogues_bit_exact(M, K, N):
    A, B, B2, a_s, b_s, b2_s, bias, C0 = _epi_inputs(M, K, N, seed=3 * M + K + N)
    v = oracle.gemm_int8(A, a_s, B, b_s, bias)
    for _ in range(2):  # two launches in a row give the same floats
        store = ec.gemm_int8_epi(0, 16, A, a_s, B, b_s, bias=bias)
        assert np.array_equal(_bits(store), _bits(v))
    resid = ec.gemm_int8_epi(1, 16, A, a_s, B, b_s, bias=bias, C0=C0)
    assert np.array_equal(_bits(resid), _bits(C0 + v))
    gelu = ec.gemm_int8_epi(2, 16, A, a_s, B, b_s, bias=bias)
    assert np.array_equal(_bits(gelu), _bits(_device_gelu(v)))
    g = oracle.gemm_int8(A, a_s, B, b_s)
    u = oracle.gemm_int8(A, a_s, B2, b2_s)
    swi = ec.gemm_int8_epi(3, 16, A, a_s, B, b_s, B2=B2, b2_scale=b2_s)
    assert np.array_equal(_bits(swi), _bits(oracle.map_op(1, g) * u))


def test_gemm_int8_skinny_rejects_tall_inputs():
    A = np.zeros((33, 64), np.int8)
    B = np.zeros((8, 64), np.int8)
    with pytest.raises(ec.EdgeCoreError, match="M <= 32"):
        ec.gemm_int8_epi(0, 16, A, np.ones(33, np.float32), B)
