"""Device top-k selection for sampled decoding (topk.hip) and the driver's
sampled generation, on the GPU.

ec_topk_dev must return, per row, the top_k + 1 largest logits (value
descending, index ascending) exactly as numpy orders them, and status 0
exactly when the row has no NaN and its top_k-th and (top_k+1)-th values
differ.  gpt2_forward_topk must select from the same logits that
gpt2_forward_ex returns for the same step.  The driver's sampled generation
(device top-k + ec_sample_candidates) must produce the ids of a replay that
copies every logit row and draws with ec_sample_full.
"""
import json
import subprocess

import numpy as np
import pytest

import edgecore_amd as ec
from tests.conftest import prompt_ids

pytestmark = pytest.mark.gpu


def _np_topk(row, k1):
    order = np.lexsort((np.arange(len(row)), -row.astype(np.float64)))
    return row[order[:k1]], order[:k1].astype(np.int32)


def _status(row, top_k):
    v, _ = _np_topk(row, top_k + 1)
    return 0 if (not np.isnan(row).any() and v[top_k - 1] != v[top_k]) else 1


@pytest.mark.parametrize("V", [151936, 50257, 4097, 1000, 130])
@pytest.mark.parametrize("top_k", [1, 40, 128])
def test_topk_dev_matches_numpy(V, top_k):
    if top_k >= V:
        pytest.skip("top_k must be below the vocabulary")
    rng = np.random.default_rng(V + top_k)
    rows = [rng.normal(0, 3, V).astype(np.float32),
            rng.integers(-50, 50, V).astype(np.float32),          # ties everywhere
            np.full(V, -1.0, np.float32)]                          # one value
    r = rng.normal(0, 1, V).astype(np.float32)
    r[rng.integers(0, V, 4)] = np.inf
    r[rng.integers(0, V, 4)] = -np.inf
    rows.append(r)
    r = rng.normal(0, 1, V).astype(np.float32)
    r[V // 2] = np.nan
    rows.append(r)
    L = np.stack(rows)
    vals, idx, status = ec.topk_dev(L, top_k)
    for i, row in enumerate(rows):
        want_status = _status(row, top_k)
        assert status[i] == want_status, i
        if np.isnan(row).any():
            continue
        wv, wi = _np_topk(row, top_k + 1)
        assert np.array_equal(vals[i], wv) and np.array_equal(idx[i], wi), i


def test_topk_dev_signed_zero_at_the_boundary_is_a_tie():
    row = np.linspace(-5, -1, 200).astype(np.float32)
    row[10], row[20] = 1.0, 2.0
    row[30], row[40] = 0.0, -0.0   # 3rd and 4th largest compare equal
    _, _, status = ec.topk_dev(row, 3)
    assert status[0] == 1
    _, _, status = ec.topk_dev(row, 2)   # boundary 2.0 / 1.0 / 0.0: no tie at the 2nd
    assert status[0] == 0


def test_forward_topk_selects_from_the_step_logits(make_model):
    path = make_model("qwen2-window-yarn-int8")
    with ec.Model(path, 2, 0) as m:
        prompt = prompt_ids(30, m.vocab, seed=12)
        n = len(prompt)
        for b in range(2):
            m.forward(prompt, np.arange(n), np.full(n, b, np.int32), lm_from=n, want_logits=False)
        toks, pos = [5, 17], [n, n]
        logits, _ = m.forward(toks, pos, None)            # the step, full logits
        vals, idx, status = m.forward_topk(toks, pos, None, top_k=40)   # the same step again
        for b in range(2):
            wv, wi = _np_topk(logits[b], 41)
            assert status[b] == _status(logits[b], 40)
            assert np.array_equal(vals[b], wv) and np.array_equal(idx[b], wi)
            assert np.array_equal(m.last_logits(b), logits[b])


def test_driver_sampling_equals_full_row_replay(make_model, tmp_path):
    path = make_model("tiny-qwen2-int8")
    prompt = prompt_ids(8, 512, seed=1)
    pf = tmp_path / "p.txt"
    pf.write_text(" ".join(map(str, prompt)))
    p = subprocess.run([str(ec.RUNTIME), "--model", str(path), "--mode", "generate", "--tokens-file", str(pf),
                        "--n-tokens", "24", "--temp", "0.8", "--top-k", "40", "--seed", "7", "--no-print"],
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stderr
    got = json.loads(p.stdout)["token_ids"]
    # replay: full logits each step, ec_sample_full with the driver's seed
    with ec.Model(path, 1, 0) as m:
        n = len(prompt)
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        cur, pos, state, ids = int(prompt[-1]), n, 7, []
        for _ in range(24):
            lg, _ = m.forward([cur], [pos], None)
            cur, state = ec.sample_full(lg[0], 0.8, 40, state)
            ids.append(cur)
            pos += 1
    assert got == ids
