"""GPT-2 small shape (12 layers, d_model 768, 12 heads of head_dim 64, GELU
FFN 3072, LayerNorm, learned positions, vocabulary 50257), fp16 weights
N(0, 0.02) from seed 0, at the configuration's full workload: a 128-token
prompt (ids uniform, seed 2) prefilled on the GPU's 16-bit path, then 128
greedy steps (positions 128-255).  Tokens identical to the oracle's and every
step's logits within max-abs 1e-2 (the fp16 bar)."""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


@pytest.fixture(scope="module")
def c2_model(model_dir):
    path = model_dir / "gpt2-small-fp16.ecm"
    if not path.exists():
        ec.synth(path, preset="gpt2-small")
    return path


def test_gpt2_small_fp16_generate_matches_oracle(c2_model):
    n, steps = 128, 128
    prompt = prompt_ids(n, 50257, seed=2)
    with ec.Model(c2_model, 1, n + steps + 8) as m:
        assert m.precision == 1
        ids, lg = m.generate(prompt, steps, want_logits=True)
    om = oracle.OracleModel(c2_model, 1, n + steps + 8)
    oids, olg = om.generate(prompt, steps, want_logits=True)
    om.close()
    err = float(np.abs(lg - olg).max())
    print(f"C2 max-abs logits diff over {steps} steps: {err:.3e}")
    assert np.array_equal(ids, oids), (ids[n:], oids[n:])
    assert err <= 1e-2
