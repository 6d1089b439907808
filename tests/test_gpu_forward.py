"""End-to-end GPU forward parity against the CPU oracle (src/gpt2.c:470-805
semantics) on seeded synthetic models.

Bar: greedy tokens identical for the first 32 generated tokens;
logits within max-abs 2e-2 (int8 models) / 1e-2 (fp16 and bf16 models) of
the oracle, which itself is bit-exact with the reference build.
"""
import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = pytest.mark.gpu

TOL = {0: 2e-2, 1: 1e-2, 2: 1e-2}

SMALL = ["tiny-gpt2-int8", "tiny-gpt2-fp16", "tiny-qwen2-int8", "tiny-qwen2-fp16",
         "tiny-qwen2-bf16", "tiny-qwen2-tied", "qwen2-hd128-int8"]


@pytest.mark.parametrize("name", SMALL)
def test_prefill_logits(make_model, name):
    path = make_model(name)
    with ec.Model(path, 1, 0) as m:
        om = oracle.OracleModel(path, 1, 0)
        toks = prompt_ids(24, m.vocab, seed=3)
        n = len(toks)
        m.kv_reset()
        om.kv_reset()
        got, _ = m.forward(toks, np.arange(n), np.zeros(n, np.int32))
        want = om.forward(toks, np.arange(n), np.zeros(n, np.int32))
        err = np.abs(got - want).max()
        assert err <= TOL[m.precision], err
        assert (got.argmax(1) == want.argmax(1)).mean() >= 0.95


@pytest.mark.parametrize("name", ["tiny-gpt2-int8", "tiny-qwen2-int8", "qwen2-hd128-int8"])
@pytest.mark.parametrize("n", [16, 64, 120])
def test_prefill_int8_rows_match_oracle(make_model, name, n):
    """Prompts of 16+ tokens run the int8 linears on the matrix-core GEMM
    (row tiles 32/64/128 by size): its int32 dots are exact and its epilogues
    (bias, residual, GELU, SwiGLU) are the GEMV's, so every row's logits stay
    at the fp16 LM head's rounding distance from the oracle."""
    path = make_model(name)
    with ec.Model(path, 1, 0) as m:
        om = oracle.OracleModel(path, 1, 0)
        toks = prompt_ids(n, m.vocab, seed=7 + n)
        m.kv_reset()
        om.kv_reset()
        got, _ = m.forward(toks, np.arange(n), np.zeros(n, np.int32))
        want = om.forward(toks, np.arange(n), np.zeros(n, np.int32))
        assert np.abs(got - want).max() <= 1e-4
        assert np.array_equal(got.argmax(1), want.argmax(1))


@pytest.mark.parametrize("name", SMALL)
def test_generate_32_tokens_identical(make_model, name):
    path = make_model(name)
    with ec.Model(path, 1, 0) as m:
        om = oracle.OracleModel(path, 1, 0)
        prompt = prompt_ids(8, m.vocab, seed=1)
        ids, lg = m.generate(prompt, 32, want_logits=True)
        oids, olg = om.generate(prompt, 32, want_logits=True)
        assert np.array_equal(ids, oids), (ids[8:], oids[8:])
        err = np.abs(lg - olg).max()
        assert err <= TOL[m.precision], err


def test_sliding_window_and_yarn(make_model):
    """Qwen2 with a 48-position sliding window and YaRN RoPE (src/gpt2.c:616-643,
    753-754): a 60-token prompt (prefill attention with lo > 0 from position 48)
    and 40 greedy steps (decode attention, graph-replayed, every step windowed)."""
    path = make_model("qwen2-window-yarn-int8")
    with ec.Model(path, 1, 0) as m:
        om = oracle.OracleModel(path, 1, 0)
        prompt = prompt_ids(60, m.vocab, seed=9)
        ids_graph, _ = m.generate(prompt, 40, want_logits=False)
        ids, lg = m.generate(prompt, 40, want_logits=True)
        oids, olg = om.generate(prompt, 40, want_logits=True)
        assert np.array_equal(ids, oids), (ids[60:], oids[60:])
        assert np.array_equal(ids_graph, oids)
        assert np.abs(lg - olg).max() <= 1e-4
        m.kv_reset()
        om.kv_reset()
        n = len(prompt)
        got, _ = m.forward(prompt, np.arange(n), np.zeros(n, np.int32))
        want = om.forward(prompt, np.arange(n), np.zeros(n, np.int32))
        assert np.abs(got - want).max() <= 1e-4


@pytest.mark.parametrize("name,B", [("tiny-qwen2-int8", 4), ("tiny-gpt2-int8", 3), ("qwen2-hd128-int8", 2),
                                    ("qwen2-ffn5120-int8", 3), ("qwen2-ffn5120-int8", 4),
                                    ("qwen2-ffn1040-int8", 2)])
def test_batched_decode_slots(make_model, name, B):
    """Per-slot prefill (seqs=b), then M=B decode with seqs=NULL
    (src/runtime_main.c:325-352): the decode GEMVs' M tiles of 2 and 4 rows
    (3 rows: a clamped fourth), RMSNorm and LayerNorm prologues, and the down
    projection's quantizing prologue over rows of 1040 and 5120."""
    path = make_model(name)
    with ec.Model(path, B, 64) as m:
        om = oracle.OracleModel(path, B, 64)
        m.kv_reset()
        om.kv_reset()
        prompts = [prompt_ids(10 + b, m.vocab, seed=10 + b) for b in range(B)]
        for b, p in enumerate(prompts):
            n = len(p)
            m.forward(p, np.arange(n), np.full(n, b, np.int32), lm_from=n, want_logits=False)
            om.forward(p, np.arange(n), np.full(n, b, np.int32))
        cur = [int(p[-1]) for p in prompts]
        pos = [len(p) for p in prompts]
        for _ in range(6):
            got, am = m.forward(cur, pos, None, want_logits=True, want_argmax=True)
            want = om.forward(cur, pos, None)
            assert np.abs(got - want).max() <= 2e-2
            assert list(am) == [int(r.argmax()) for r in want]
            cur = [int(x) for x in am]
            pos = [p + 1 for p in pos]


def test_slot_clamp_matches_reference(make_model):
    """seqs beyond batch_cap clamp to batch_cap-1 (src/gpt2.c:512-513)."""
    path = make_model("tiny-gpt2-fp16")
    with ec.Model(path, 2, 32) as m:
        om = oracle.OracleModel(path, 2, 32)
        m.kv_reset()
        om.kv_reset()
        toks = [5, 6, 7]
        got, _ = m.forward(toks, [0, 1, 2], [7, 7, 7])
        want = om.forward(toks, [0, 1, 2], [7, 7, 7])
        assert np.abs(got - want).max() <= 1e-2


def test_argmax_matches_first_maximum(make_model):
    path = make_model("tiny-gpt2-int8")
    with ec.Model(path, 1, 0) as m:
        m.kv_reset()
        lg, am = m.forward([1, 2, 3], [0, 1, 2], [0, 0, 0], want_logits=True, want_argmax=True)
        assert list(am) == [int(np.argmax(r)) for r in lg]


def test_invalid_inputs_rejected_before_launch(make_model):
    path = make_model("tiny-gpt2-int8")
    with ec.Model(path, 1, 16) as m:
        with pytest.raises(ec.EdgeCoreError, match="position"):
            m.forward([1], [16])
        with pytest.raises(ec.EdgeCoreError, match="token"):
            m.forward([m.vocab], [0])
        with pytest.raises(ec.EdgeCoreError, match="M="):
            m.forward(list(range(17)), list(range(17)))
        with pytest.raises(ec.EdgeCoreError, match="slot"):
            m.forward([1], [0], [-1])
        # the model still works afterwards
        m.kv_reset()
        lg, _ = m.forward([1, 2], [0, 1], [0, 0])
        assert np.isfinite(lg).all()


@pytest.mark.parametrize("name", ["tiny-qwen2-int8", "tiny-gpt2-fp16", "tiny-qwen2-bf16", "qwen2-hd128-int8"])
def test_graph_decode_equals_direct_and_oracle(make_model, name):
    """The single-token greedy step replays a captured HIP graph (argmax only);
    asking for logits takes the direct launches.  Both must give the oracle's ids."""
    path = make_model(name)
    with ec.Model(path, 1, 0) as m:
        prompt = prompt_ids(8, m.vocab, seed=3)
        ids_graph, _ = m.generate(prompt, 32, want_logits=False)
        ids_direct, _ = m.generate(prompt, 32, want_logits=True)
        ids_again, _ = m.generate(prompt, 32, want_logits=False)  # the cached graph, after kv_reset
    oids, _ = oracle.OracleModel(path, 1, 0).generate(prompt, 32)
    assert np.array_equal(ids_graph, ids_direct)
    assert np.array_equal(ids_graph, ids_again)
    assert np.array_equal(ids_graph, oids)


@pytest.mark.parametrize("name,B", [("tiny-qwen2-int8", 3), ("tiny-gpt2-fp16", 16), ("qwen2-hd128-int8", 16)])
def test_batched_graph_decode_equals_direct_and_oracle(make_model, name, B):
    """A greedy step of B tokens in B slots (argmax only) replays a HIP graph
    captured per (B, position bucket); asking for logits takes the direct
    launches.  Graph ids, direct ids and the oracle's ids must agree, also on
    a second pass that replays the cached graph after a cache reset."""
    path = make_model(name)
    steps = 8
    with ec.Model(path, B, 64) as m:
        prompts = [prompt_ids(6 + b % 5, m.vocab, seed=40 + b) for b in range(B)]

        def run(want_logits):
            m.kv_reset()
            for b, p in enumerate(prompts):
                m.forward(p, np.arange(len(p)), np.full(len(p), b, np.int32), lm_from=len(p), want_logits=False)
            cur, pos, out = [int(p[-1]) for p in prompts], [len(p) for p in prompts], []
            for _ in range(steps):
                _, am = m.forward(cur, pos, None, want_logits=want_logits, want_argmax=True)
                cur, pos = [int(x) for x in am], [q + 1 for q in pos]
                out.append(cur)
            return np.array(out)

        ids_graph, ids_direct, ids_again = run(False), run(True), run(False)
    om = oracle.OracleModel(path, B, 64)
    om.kv_reset()
    for b, p in enumerate(prompts):
        om.forward(p, np.arange(len(p)), np.full(len(p), b, np.int32))
    cur, pos, oids = [int(p[-1]) for p in prompts], [len(p) for p in prompts], []
    for _ in range(steps):
        lg = om.forward(cur, pos, None)
        cur, pos = [int(r.argmax()) for r in lg], [q + 1 for q in pos]
        oids.append(cur)
    om.close()
    assert np.array_equal(ids_graph, ids_direct)
    assert np.array_equal(ids_graph, ids_again)
    assert np.array_equal(ids_graph, np.array(oids))


def test_graph_recaptured_across_position_buckets(make_model):
    """Decode positions 1000..1039 cross the 1024 bucket (the graph is captured
    again with a larger attention LDS); two models keep separate graphs."""
    path = make_model("qwen2-long-int8")
    other = make_model("tiny-qwen2-int8")
    with ec.Model(path, 1, 0) as m, ec.Model(other, 1, 0) as m2:
        prompt = prompt_ids(1000, m.vocab, seed=4)
        p2 = prompt_ids(8, m2.vocab, seed=5)
        a2, _ = m2.generate(p2, 16)
        ids, _ = m.generate(prompt, 40)
        b2, _ = m2.generate(p2, 16)
    oids, _ = oracle.OracleModel(path, 1, 0).generate(prompt, 40)
    o2, _ = oracle.OracleModel(other, 1, 0).generate(p2, 16)
    assert np.array_equal(ids, oids)
    assert np.array_equal(a2, o2) and np.array_equal(b2, o2)
