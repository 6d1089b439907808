"""Host sampling of the driver (src/runtime_main.c:205-248) -- CPU only.

ec_sample_full restates sample_token; it is compared with the reference's
own sample_token (compiled from src/runtime_main.c into oracle/_ref, where the
reference tree exists) on random rows and on rows built to stress its
tie-breaking (few distinct values, -0/+0, infinities, NaN), token and LCG
state after every draw.  ec_sample_candidates, which sees only the row's
top_k + 1 largest logits, must give the same token and state as the full row
whenever the device would report status 0 (no NaN, top_k-th and
(top_k+1)-th values different); that is checked on rows with many ties
inside the top_k, where the reference's swap order decides.
"""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle


def _rows(rng, V, n):
    """random rows, rows of few distinct values, rows with signed zeros and infinities"""
    out = []
    for _ in range(n):
        out.append(rng.normal(0, 2, V).astype(np.float32))
        out.append(rng.integers(-3, 4, V).astype(np.float32))          # heavy ties
        r = rng.normal(0, 1, V).astype(np.float32)
        r[rng.integers(0, V, 5)] = 0.0
        r[rng.integers(0, V, 5)] = -0.0
        r[rng.integers(0, V, 2)] = np.inf
        r[rng.integers(0, V, 2)] = -np.inf
        out.append(r)
    return out


def _candidates(row, top_k):
    """top_k + 1 largest (value descending, index ascending) and the status rule"""
    order = np.lexsort((np.arange(len(row)), -row.astype(np.float64)))
    c = order[:top_k + 1]
    ok = not np.isnan(row).any() and row[c[top_k - 1]] != row[c[top_k]]
    return row[c], c.astype(np.int32), ok


@pytest.mark.skipif(not oracle.ref_sample_available(), reason="reference build oracle/_ref absent")
@pytest.mark.parametrize("V", [7, 300, 4099])
def test_sample_full_equals_reference(V):
    rng = np.random.default_rng(V)
    rows = _rows(rng, V, 4)
    nanrow = rng.normal(0, 1, V).astype(np.float32)
    nanrow[rng.integers(0, V, 3)] = np.nan
    nanrow[0] = np.nan  # a NaN at the front wins the first selection round
    rows.append(nanrow)
    state = 42
    for row in rows:
        for temp in (0.0, 0.7, 1.5):
            for top_k in (0, 1, 5, 40, V - 1, V):
                want, ws = oracle.ref_sample(row, temp, top_k, state)
                got, gs = ec.sample_full(row, temp, top_k, state)
                assert (got, gs) == (want, ws), (temp, top_k)
                state = gs


@pytest.mark.parametrize("V", [50, 1000, 151936])
def test_sample_candidates_equals_full_row(V):
    rng = np.random.default_rng(V + 1)
    state = 1
    checked = 0
    for row in _rows(rng, V, 2 if V > 10000 else 6):
        for top_k in (1, 2, 7, 40, 128):
            if top_k >= V:
                continue
            vals, idx, ok = _candidates(row, top_k)
            if not ok:
                continue
            for temp in (0.7, 1.5):
                want, ws = ec.sample_full(row, temp, top_k, state)
                got, gs = ec.sample_candidates(vals, idx, V, temp, top_k, state)
                assert (got, gs) == (want, ws), (top_k, temp)
                state = gs
                checked += 1
    assert checked > 10


def test_sample_candidates_rejects_what_it_cannot_do():
    v = np.array([3.0, 2.0, 1.0], np.float32)
    i = np.array([0, 1, 2], np.int32)
    assert ec.sample_candidates(v, i, 10, 0.0, 2, 1)[0] == -1    # greedy is not a top-k draw
    assert ec.sample_candidates(v, i, 10, 0.7, 0, 1)[0] == -1    # top_k 0 samples the whole row
    assert ec.sample_candidates(v, i, 3, 0.7, 3, 1)[0] == -1     # top_k >= vocab
    assert ec.sample_candidates(v, i, 10, 0.7, 5, 1)[0] == -1    # fewer than top_k + 1 candidates


def test_lcg_matches_the_reference_constants():
    # state' = state * 6364136223846793005 + 1442695040888963407 (mod 2^64), output state' >> 33
    s = 1
    for _ in range(5):
        nxt = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        import ctypes as C
        st = C.c_ulonglong(s)
        out = ec.lib().ec_rng_next(C.byref(st))
        assert st.value == nxt and out == nxt >> 33
        s = nxt
