"""The prefill-heavy Qwen2-0.5B workload: 4 slots, each prefilled with its
own 2048-token prompt one slot at a time (src/runtime_main.c:325-330), then 32
greedy decode steps at M=4, one token per slot (src/gpt2.c:667-805).

The model has the Qwen2-0.5B per-layer shapes (E896, 14 query / 2 KV heads of
head_dim 64, SwiGLU 4864, RMSNorm, RoPE theta 1e6, tied vocabulary 151936,
int8 per-channel weights N(0, 0.02)) at 2 of its 24 layers, so that the CPU
oracle finishes in seconds.  A 2048-row prefill runs the matrix-core GEMMs
with the tiles the full model uses (gate/up: 128-row tiles with the SwiGLU
epilogue; qkv: 64-row tiles; o and down: 32-row tiles with the residual
epilogue) and the prefill attention over 2048 positions; the M=4 decode runs
the batched GEMVs and decode attention at positions 2048-2079.

Bar: each prefill's last-row logits and every decode step's logits within
max-abs 2e-2 of the oracle, and identical greedy tokens."""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

SLOTS, PROMPT, STEPS, V = 4, 2048, 32, 151936


@pytest.fixture(scope="module")
def c4_model(model_dir):
    path = model_dir / "qwen2-0.5b-2l-int8.ecm"
    if not path.exists():
        ec.synth(path, name="qwen2-0.5b-2l", arch="qwen2", layers=2, embd=896, heads=14, kv_heads=2,
                 ffn=4864, ctx=32768, vocab=V, precision="int8", tie=1)
    return path


def test_c4_prefill_4x2048_then_batched_decode(c4_model):
    ctx = PROMPT + STEPS + 8
    with ec.Model(c4_model, SLOTS, ctx) as m:
        om = oracle.OracleModel(c4_model, SLOTS, ctx)
        m.kv_reset()
        om.kv_reset()
        prompts = [prompt_ids(PROMPT, V, seed=b + 1) for b in range(SLOTS)]
        first = []
        worst = 0.0
        for b, p in enumerate(prompts):
            pos, slot = np.arange(PROMPT), np.full(PROMPT, b, np.int32)
            got, am = m.forward(p, pos, slot, lm_from=PROMPT - 1, want_logits=True, want_argmax=True)
            want = om.forward(p, pos, slot, lm_from=PROMPT - 1)
            err = float(np.abs(got - want).max())
            worst = max(worst, err)
            assert err <= 2e-2, (b, err)
            assert int(am[0]) == int(want[0].argmax()), b
            first.append(int(am[0]))
            print(f"slot {b}: 2048-token prefill, last-row logits max-abs diff {err:.3e}", flush=True)
        cur, pos = list(first), [PROMPT] * SLOTS
        for s in range(STEPS):
            got, am = m.forward(cur, pos, None, want_logits=True, want_argmax=True)
            want = om.forward(cur, pos, None)
            err = float(np.abs(got - want).max())
            worst = max(worst, err)
            assert err <= 2e-2, (s, err)
            assert list(am) == [int(r.argmax()) for r in want], s
            cur, pos = [int(x) for x in am], [p + 1 for p in pos]
        om.close()
    print(f"C4-shape worst max-abs logits diff: {worst:.3e}")
