"""Headline shape: Qwen2-0.5B architecture, int8 per-channel weights N(0, 0.02)
from seed 0, 256-token prompt (ids uniform in [0, 151936), seed 1), greedy
decode.  The first 32 generated tokens must equal the oracle's, and every
step's logits must be within max-abs 2e-2 of the oracle's."""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


@pytest.fixture(scope="module")
def c3_model(model_dir):
    path = model_dir / "qwen2-0.5b-int8.ecm"
    if not path.exists():
        ec.synth(path, preset="qwen2-0.5b")
    return path


def test_qwen2_05b_int8_generate_matches_oracle(c3_model):
    prompt = prompt_ids(256, 151936, seed=1)
    with ec.Model(c3_model, 1, 256 + 32 + 8) as m:
        ids, lg = m.generate(prompt, 32, want_logits=True)
    om = oracle.OracleModel(c3_model, 1, 256 + 32 + 8)
    oids, olg = om.generate(prompt, 32, want_logits=True)
    om.close()
    err = float(np.abs(lg - olg).max())
    print(f"C3 max-abs logits diff over 32 steps: {err:.3e}")
    assert np.array_equal(ids, oids), (ids[256:], oids[256:])
    assert err <= 2e-2


def test_qwen2_05b_int8_prefill_rows(c3_model):
    """Prefill of 64 tokens: every row's logits vs the oracle."""
    prompt = prompt_ids(64, 151936, seed=7)
    n = len(prompt)
    with ec.Model(c3_model, 1, 128) as m:
        m.kv_reset()
        got, _ = m.forward(prompt, np.arange(n), np.zeros(n, np.int32))
    om = oracle.OracleModel(c3_model, 1, 128)
    om.kv_reset()
    want = om.forward(prompt, np.arange(n), np.zeros(n, np.int32))
    om.close()
    err = float(np.abs(got - want).max())
    assert err <= 2e-2, err
    assert (got.argmax(1) == want.argmax(1)).all()
