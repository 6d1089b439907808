"""The device attention kernels alone against the oracle's per-row attention
(src/gpt2.c:527-557 GPT-2, 744-777 Qwen2 GQA) on the same seeded q and fp16
caches, through ec_attention_dev.

Bar: the kernels keep the reference's order for every float operation; the
one difference is the double sum of the exponentials, added in a tree order,
whose last bits can move a probability's float rounding in rare ties.  So
almost every element is bit-identical (at least 99.9% asserted) and none is
further than 1e-5 from the oracle (values are O(1))."""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle

pytestmark = pytest.mark.gpu


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _case(seed, M, H, KVH, hd, C, nslots):
    rng = np.random.default_rng(seed)
    kc = _f16(rng.normal(0, 1, (nslots, C, KVH * hd)))
    vc = _f16(rng.normal(0, 1, (nslots, C, KVH * hd)))
    q = rng.normal(0, 1, (M, H * hd)).astype(np.float32)
    return rng, q, kc, vc


def _check(got, want, rows):
    g, w = got[rows], want[rows]
    assert np.isfinite(g).all()
    err = np.abs(g - w).max()
    exact = (g == w).mean()
    print(f"rows {len(rows)}: max-abs {err:.3e}, bit-identical {exact:.6f}")
    assert err <= 1e-5, err
    assert exact >= 0.999, exact


def _rows(rng, M, k):
    edge = [0, 1, 15, 16, 17, 63, 64, 65, 127, 128, M // 2, M - 17, M - 16, M - 2, M - 1]
    return np.unique(np.concatenate([[r for r in edge if 0 <= r < M], rng.choice(M, min(k, M), replace=False)]))


def test_prefill_qwen2_05b_2048():
    """The 2048-token prompt of the prefill benchmark (Qwen2-0.5B heads: 14
    query heads, 2 KV heads, head_dim 64): 16 tokens per block, the whole-tile
    and partial-tile paths and the diagonal tiles."""
    M, H, KVH, hd = 2048, 14, 2, 64
    rng, q, kc, vc = _case(1, M, H, KVH, hd, M, 1)
    pos, slot = np.arange(M), np.zeros(M)
    got = ec.attention_dev(q, kc, vc, pos, slot, H, KVH, path=0)
    rows = _rows(rng, M, 160)
    want = oracle.attention_rows(q, kc, vc, pos, slot, H, KVH, rows=rows)
    _check(got, want, rows)


@pytest.mark.parametrize("H,KVH,hd,M,p0,window,nslots,slot", [
    (14, 2, 64, 200, 100, 48, 2, 1),   # mid-cache start, sliding window, second slot
    (14, 2, 64, 333, 0, 0, 1, 0),      # ragged last block
    (12, 2, 128, 300, 17, 0, 1, 0),    # head_dim 128: one token per wave
    (4, 4, 32, 150, 0, 0, 1, 0),       # head_dim 32, GPT-2-style heads (KVH = H)
    (4, 4, 64, 700, 0, 100, 1, 0),     # window spanning tiles
])
def test_prefill_shapes(H, KVH, hd, M, p0, window, nslots, slot):
    C = p0 + M + 8
    rng, q, kc, vc = _case(M + hd, M, H, KVH, hd, C, nslots)
    pos = p0 + np.arange(M)
    sl = np.full(M, slot)
    got = ec.attention_dev(q, kc, vc, pos, sl, H, KVH, window=window, path=0)
    want = oracle.attention_rows(q, kc, vc, pos, sl, H, KVH, window=window)
    _check(got, want, np.arange(M))


@pytest.mark.parametrize("hd,window", [(64, 0), (128, 0), (64, 300)])
def test_decode_kernel_long_positions(hd, window):
    """The per-token kernel: 8 tokens in 4 slots at positions up to 2047."""
    H, KVH, C, ns = 14, 2, 2048, 4
    rng, q, kc, vc = _case(5 + hd, 8, H, KVH, hd, C, ns)
    pos = np.array([2047, 2000, 1536, 1023, 511, 64, 3, 0])
    sl = np.array([0, 1, 2, 3, 0, 1, 2, 3])
    got = ec.attention_dev(q, kc, vc, pos, sl, H, KVH, window=window, path=1)
    want = oracle.attention_rows(q, kc, vc, pos, sl, H, KVH, window=window)
    _check(got, want, np.arange(8))


@pytest.mark.parametrize("H,KVH,hd,window", [(12, 2, 128, 0), (12, 2, 128, 700), (16, 1, 128, 0), (6, 6, 128, 0)])
def test_decode_scores_pass_equals_per_token_kernel(H, KVH, hd, window):
    """The long-context decode form of head_dim 128 (path 2: a scores pass
    per token, KV group and 256 positions, then the per-token kernel's
    softmax and sums on those scores) against the per-token kernel (path 1)
    bit for bit, and against the oracle: GQA groups of 6 and 16 heads and
    GPT-2-style heads, with and without a window; 8 tokens in 4 slots at
    positions up to 2047."""
    C, ns = 2048, 4
    rng, q, kc, vc = _case(77 + hd + H + window, 8, H, KVH, hd, C, ns)
    pos = np.array([2047, 2000, 1536, 1023, 511, 256, 3, 0])
    sl = np.array([0, 1, 2, 3, 0, 1, 2, 3])
    one = ec.attention_dev(q, kc, vc, pos, sl, H, KVH, window=window, path=1)
    two = ec.attention_dev(q, kc, vc, pos, sl, H, KVH, window=window, path=2)
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))
    want = oracle.attention_rows(q, kc, vc, pos, sl, H, KVH, window=window)
    _check(two, want, np.arange(8))


def test_attention_dev_rejects_bad_arguments():
    H, KVH, hd, C = 4, 2, 64, 32
    _, q, kc, vc = _case(9, 4, H, KVH, hd, C, 1)
    with pytest.raises(ec.EdgeCoreError):
        ec.attention_dev(q, kc, vc, [0, 1, 2, 40], [0, 0, 0, 0], H, KVH)        # position past the cache
    with pytest.raises(ec.EdgeCoreError):
        ec.attention_dev(q, kc, vc, [0, 1, 3, 4], [0, 0, 0, 0], H, KVH, path=0)  # not consecutive
    with pytest.raises(ec.EdgeCoreError):
        ec.attention_dev(q, kc, vc, [0, 1, 2, 3], [0, 0, 1, 0], H, KVH)          # slot outside the cache
