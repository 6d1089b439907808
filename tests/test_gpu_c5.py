"""Qwen2.5-1.5B shape (E1536, 12 query / 2 KV heads of head_dim 128, SwiGLU
FFN 8960, RMSNorm, RoPE theta 1e6, tied vocabulary 151936, int8 per-channel
weights N(0, 0.02)) at 2 of its 28 layers, in the batched-decode regime of
that configuration: 16 slots, each prompt prefilled on its own slot (as
src/runtime_main.c:325-330 does), then greedy decode steps at M=16 with one
token per slot (the M=16 matrix-core GEMM, the head_dim-128 attention
kernels).  Every step's logits must be within max-abs 2e-2 of the oracle's and
the greedy tokens identical.  The layer count is cut so that the CPU oracle
finishes in seconds; every per-layer shape is the real one."""
import os

import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

B, PROMPT, STEPS, V = 16, 40, 12, 151936


@pytest.fixture(scope="module")
def c5_model(model_dir):
    path = model_dir / "qwen2.5-1.5b-2l-int8.ecm"
    if not path.exists():
        ec.synth(path, name="qwen2.5-1.5b-2l", arch="qwen2", layers=2, embd=1536, heads=12, kv_heads=2,
                 ffn=8960, ctx=4096, vocab=V, precision="int8", tie=1)
    return path


def test_qwen25_15b_shape_batched_decode(c5_model):
    ctx = PROMPT + STEPS + 8
    with ec.Model(c5_model, B, ctx) as m:
        om = oracle.OracleModel(c5_model, B, ctx)
        m.kv_reset()
        om.kv_reset()
        prompts = [prompt_ids(PROMPT, V, seed=20 + b) for b in range(B)]
        for b, p in enumerate(prompts):
            n = len(p)
            m.forward(p, np.arange(n), np.full(n, b, np.int32), lm_from=n, want_logits=False)
            om.forward(p, np.arange(n), np.full(n, b, np.int32), lm_from=n)
        cur = [int(p[-1]) for p in prompts]
        pos = [PROMPT] * B
        worst = 0.0
        for _ in range(STEPS):
            got, am = m.forward(cur, pos, None, want_logits=True, want_argmax=True)
            want = om.forward(cur, pos, None)
            err = float(np.abs(got - want).max())
            worst = max(worst, err)
            assert err <= 2e-2, err
            assert list(am) == [int(r.argmax()) for r in want]
            cur = [int(x) for x in am]
            pos = [p + 1 for p in pos]
        om.close()
    print(f"C5-shape max-abs logits diff over {STEPS} steps of 16 tokens: {worst:.3e}")


def test_qwen25_15b_shape_long_prefill(c5_model):
    """Two 1024-token prompts prefilled on their own slots (gate/up N=8960 at
    M=1024 takes the 128-row matrix-core tiles, attention over 1024 positions
    at head_dim 128), then 8 greedy steps at M=2."""
    n, slots, steps = 1024, 2, 8
    ctx = n + steps + 8
    with ec.Model(c5_model, slots, ctx) as m:
        om = oracle.OracleModel(c5_model, slots, ctx)
        m.kv_reset()
        om.kv_reset()
        cur = []
        for b in range(slots):
            p = prompt_ids(n, V, seed=40 + b)
            pos, slot = np.arange(n), np.full(n, b, np.int32)
            got, am = m.forward(p, pos, slot, lm_from=n - 4, want_logits=True, want_argmax=True)
            want = om.forward(p, pos, slot, lm_from=n - 4)
            assert float(np.abs(got - want).max()) <= 2e-2
            assert list(am) == [int(r.argmax()) for r in want]
            cur.append(int(am[-1]))
        pos = [n] * slots
        for _ in range(steps):
            got, am = m.forward(cur, pos, None, want_logits=True, want_argmax=True)
            want = om.forward(cur, pos, None)
            assert float(np.abs(got - want).max()) <= 2e-2
            assert list(am) == [int(r.argmax()) for r in want]
            cur, pos = [int(x) for x in am], [p + 1 for p in pos]
        om.close()


def test_qwen25_15b_shape_c5_workload(c5_model):
    """The C5 decode workload at 2 layers: 16 slots, each prefilled with a
    1024-token prompt (ids from seeds 1-16, as the benchmark's batched leg
    draws them), then 32 greedy steps at M=16 from position 1024 -- the
    two-pass head_dim-128 attention (scores pass over the 16 slots' scores
    workspace, then softmax and sums) and the M=16 decode graph of the
    1024-1535 position bucket.  First the steps as the benchmark runs them
    (argmax only: the captured graph), ids against the oracle; then the same
    steps again from a fresh prefill with logits (direct launches), every
    step within max-abs 2e-2 of the oracle."""
    n, steps = 1024, 32
    ctx = n + steps + 8
    prompts = [prompt_ids(n, V, seed=b + 1) for b in range(B)]
    with ec.Model(c5_model, B, ctx) as m:
        om = oracle.OracleModel(c5_model, B, ctx)
        om.kv_reset()
        first = []
        for b, p in enumerate(prompts):
            want = om.forward(p, np.arange(n), np.full(n, b, np.int32), lm_from=n - 1)
            first.append(int(want[0].argmax()))
        ocur, opos, oids, ologits = list(first), [n] * B, [], []
        for _ in range(steps):
            want = om.forward(ocur, opos, None)
            ocur = [int(r.argmax()) for r in want]
            oids.append(ocur)
            ologits.append(want)
            opos = [p + 1 for p in opos]
        om.close()

        def prefill():
            m.kv_reset()
            out = []
            for b, p in enumerate(prompts):
                _, am = m.forward(p, np.arange(n), np.full(n, b, np.int32), lm_from=n - 1, want_logits=False,
                                  want_argmax=True)
                out.append(int(am[0]))
            return out

        assert prefill() == first
        cur, pos = list(first), [n] * B
        for s in range(steps):
            _, am = m.forward(cur, pos, None, want_logits=False, want_argmax=True)
            cur, pos = [int(x) for x in am], [p + 1 for p in pos]
            assert cur == oids[s], s

        assert prefill() == first
        cur, pos, worst = list(first), [n] * B, 0.0
        for s in range(steps):
            got, am = m.forward(cur, pos, None, want_logits=True, want_argmax=True)
            err = float(np.abs(got - ologits[s]).max())
            worst = max(worst, err)
            assert err <= 2e-2, (s, err)
            cur, pos = [int(x) for x in am], [p + 1 for p in pos]
            assert cur == oids[s], s
    print(f"C5 workload (16 x 1024 + 32 steps at M=16, 2 layers): max-abs logits diff {worst:.3e}")


def _decode_m16(path, fuse: bool, prompt: int, steps: int, vocab: int):
    """16 slots prefilled with `prompt`-token prompts, then `steps` greedy
    steps at M=16 with logits; the model loaded with the o / down
    quantization inside the skinny GEMMs (fuse) or as its own pass."""
    old = os.environ.get("EDGECORE_FUSEQ")
    os.environ["EDGECORE_FUSEQ"] = "1" if fuse else "0"
    try:
        with ec.Model(path, B, prompt + steps + 8) as m:
            m.kv_reset()
            prompts = [prompt_ids(prompt, vocab, seed=60 + b) for b in range(B)]
            for b, p in enumerate(prompts):
                m.forward(p, np.arange(prompt), np.full(prompt, b, np.int32), lm_from=prompt, want_logits=False)
            cur, pos, out = [int(p[-1]) for p in prompts], [prompt] * B, []
            for _ in range(steps):
                got, am = m.forward(cur, pos, None, want_logits=True, want_argmax=True)
                out.append(got)
                cur, pos = [int(x) for x in am], [p + 1 for p in pos]
            return np.stack(out)
    finally:
        if old is None:
            del os.environ["EDGECORE_FUSEQ"]
        else:
            os.environ["EDGECORE_FUSEQ"] = old


@pytest.mark.parametrize("prompt", [40, 600])
def test_fused_quantization_equals_separate_pass(c5_model, prompt):
    """Batched decode at M=16 with the o and down projections quantizing
    their fp32 inputs inside the skinny GEMM (row maxima from the attention's
    and the gate/up epilogue's partial maxima) against the separate
    quantization pass: the same logits bit for bit, after short prompts (the
    one-pass attention) and past 512 positions (the scores pass)."""
    a = _decode_m16(c5_model, True, prompt, 6, V)
    b = _decode_m16(c5_model, False, prompt, 6, V)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fused_quantization_gpt2_int8(make_model):
    """The same on the tiny int8 GPT-2 (fc with the GELU epilogue writes the
    partial maxima the down projection quantizes with; head_dim 32 attention)."""
    path = make_model("tiny-gpt2-int8")
    a = _decode_m16(path, True, 20, 6, 50257)
    b = _decode_m16(path, False, 20, 6, 50257)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
