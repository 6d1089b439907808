"""The persistent decode step (decode_step.hip) against the kernel-per-
operation forward it replaces for one-token int8 Qwen2 steps
(src/gpt2.c:667-805 at M = 1).

Both paths run the same arithmetic in the same order, so a greedy decode
through the step must give logits bit-identical to the same decode with the
step turned off (EDGECORE_STEP=0 when the model is loaded), at every step,
and the oracle's tokens.  The model has the Qwen2-0.5B per-layer shapes at 3
layers; the decode crosses positions 505-530 (the attention's first K tile
and a 512-position boundary)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = pytest.mark.gpu

V = 151936


@pytest.fixture(scope="module")
def step_model(model_dir):
    path = model_dir / "qwen2-0.5b-3l-int8.ecm"
    if not path.exists():
        ec.synth(path, name="qwen2-0.5b-3l", arch="qwen2", layers=3, embd=896, heads=14, kv_heads=2, ffn=4864,
                 ctx=32768, vocab=V, precision="int8", tie=1)
    return path


def _families(fn):
    L = ec.lib()
    L.ec_prof_start(b"")
    fn()
    buf = C.create_string_buffer(1 << 16)
    assert L.ec_prof_stop(buf, len(buf)) > 0, ec.last_error()
    return {k["kernel"]: k for k in json.loads(buf.value.decode())}


def _decode(path, prompt, steps, step_on):
    old = os.environ.get("EDGECORE_STEP")
    os.environ["EDGECORE_STEP"] = "1" if step_on else "0"
    try:
        m = ec.Model(path, 1, len(prompt) + steps + 8)
    finally:
        if old is None:
            del os.environ["EDGECORE_STEP"]
        else:
            os.environ["EDGECORE_STEP"] = old
    with m:
        n = len(prompt)
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        cur, pos, out, ids = int(prompt[-1]), n, [], []
        fams = None
        for s in range(steps):
            if s == 0:
                res = {}
                fams = _families(lambda: res.update(r=m.forward([cur], [pos], None, want_logits=True,
                                                              want_argmax=True)))
                lg, am = res["r"]
            else:
                lg, am = m.forward([cur], [pos], None, want_logits=True, want_argmax=True)
            out.append(lg[0])
            cur, pos = int(am[0]), pos + 1
            ids.append(cur)
    return np.stack(out), ids, fams


def test_step_bit_identical_to_kernel_per_op(step_model):
    prompt = prompt_ids(505, V, seed=7)
    lg_s, ids_s, fam_s = _decode(step_model, prompt, 26, True)
    lg_k, ids_k, fam_k = _decode(step_model, prompt, 26, False)
    assert "decode_step" in fam_s and "gemv_qkv" not in fam_s, sorted(fam_s)
    assert "decode_step" not in fam_k and "gemv_qkv" in fam_k, sorted(fam_k)
    assert ids_s == ids_k
    assert np.array_equal(lg_s.view(np.uint32), lg_k.view(np.uint32)), float(np.abs(lg_s - lg_k).max())
    om = oracle.OracleModel(step_model, 1, len(prompt) + 26 + 8)
    oids, olg = om.generate(prompt, 26, want_logits=True)
    om.close()
    assert ids_s == [int(x) for x in oids[len(prompt):]]
    assert float(np.abs(lg_s - olg).max()) <= 2e-2


def test_step_short_context(step_model):
    """Positions 1-12: the first steps after a one-token prompt."""
    prompt = prompt_ids(1, V, seed=9)
    lg_s, ids_s, _ = _decode(step_model, prompt, 12, True)
    lg_k, ids_k, _ = _decode(step_model, prompt, 12, False)
    assert ids_s == ids_k and np.array_equal(lg_s.view(np.uint32), lg_k.view(np.uint32))


def _load(path, ctx, step_on):
    old = os.environ.get("EDGECORE_STEP")
    os.environ["EDGECORE_STEP"] = "1" if step_on else "0"
    try:
        return ec.Model(path, 1, ctx)
    finally:
        if old is None:
            del os.environ["EDGECORE_STEP"]
        else:
            os.environ["EDGECORE_STEP"] = old


def test_generate_greedy_equals_step_loop(step_model):
    """ec_generate_greedy (steps chained on the device, one HIP graph per
    512-position bucket) gives the ids of the host-driven greedy loop, across
    the 512-position boundary; in two calls (the second continuing from the
    first's last id); then a host-driven step after it; and through the
    kernel-per-op fallback (no persistent step)."""
    prompt = prompt_ids(505, V, seed=7)
    n = len(prompt)
    _, ids_s, _ = _decode(step_model, prompt, 26, True)
    for step_on in (True, False):
        with _load(step_model, n + 26 + 8, step_on) as m:
            m.kv_reset()
            m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
            ids = m.generate_greedy(int(prompt[-1]), n, 0, 26)
            assert [int(x) for x in ids] == ids_s, step_on
            m.kv_reset()
            m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
            a = m.generate_greedy(int(prompt[-1]), n, 0, 10)
            b = m.generate_greedy(int(a[-1]), n + 10, 0, 15)
            _, am = m.forward([int(b[-1])], [n + 25], None, want_logits=False, want_argmax=True)
            assert [int(x) for x in a] + [int(x) for x in b] + [int(am[0])] == ids_s, step_on


def test_generate_greedy_rejects_bad_arguments(step_model):
    with _load(step_model, 64, True) as m:
        for args in ((V, 0, 0, 4), (-1, 0, 0, 4), (5, 60, 0, 8), (5, -1, 0, 2), (5, 0, -1, 2)):
            with pytest.raises(ec.EdgeCoreError):
                m.generate_greedy(*args)
        with pytest.raises(ec.EdgeCoreError):
            m.generate_greedy(5, 0, 0, 0)


_CHILD = r"""
import json, sys
import numpy as np
import edgecore_amd as ec
from tests.conftest import prompt_ids
path, mode = sys.argv[1], sys.argv[2]
prompt = prompt_ids(300, 151936, seed=11)
n = len(prompt)
with ec.Model(path, 1, n + 40) as m:
    m.kv_reset()
    m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
    if mode == "chain":
        ids = [int(x) for x in m.generate_greedy(int(prompt[-1]), n, 0, 24)]
    else:
        cur, ids = int(prompt[-1]), []
        for k in range(24):
            _, am = m.forward([cur], [n + k], None, want_logits=False, want_argmax=True)
            cur = int(am[0])
            ids.append(cur)
print(json.dumps(ids))
"""


def _child_ids(path, mode, env):
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    e = dict(os.environ)
    e.update(env)
    r = subprocess.run([sys.executable, "-c", _CHILD, str(path), mode], cwd=root, env=e, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1]), r.stderr


def test_step_launch_modes_and_timeout_switch(step_model):
    """The persistent step as a plain launch (the default) and as a
    cooperative launch give the same ids, host-driven and chained; and a step
    that reports a timed-out wait while plain (forced from the host) switches
    the library to cooperative launches and is redone with the same result."""
    plain, _ = _child_ids(step_model, "loop", {})
    coop, _ = _child_ids(step_model, "loop", {"EDGECORE_STEP_COOP": "1"})
    chain, _ = _child_ids(step_model, "chain", {})
    chain_coop, _ = _child_ids(step_model, "chain", {"EDGECORE_STEP_COOP": "1"})
    assert plain == coop == chain == chain_coop
    for mode in ("loop", "chain"):
        ids, err = _child_ids(step_model, mode, {"EDGECORE_STEP_TEST_FAIL": "1"})
        assert ids == plain, mode
        assert "cooperative launches from now on" in err, (mode, err[-500:])


def _step_vs_kernel_per_op_and_oracle(path, prompt, steps):
    lg_s, ids_s, fam_s = _decode(path, prompt, steps, True)
    lg_k, ids_k, fam_k = _decode(path, prompt, steps, False)
    assert "decode_step" in fam_s and "gemv_qkv" not in fam_s, sorted(fam_s)
    assert "decode_step" not in fam_k, sorted(fam_k)
    assert ids_s == ids_k
    assert np.array_equal(lg_s.view(np.uint32), lg_k.view(np.uint32)), float(np.abs(lg_s - lg_k).max())
    om = oracle.OracleModel(path, 1, len(prompt) + steps + 8)
    oids, olg = om.generate(prompt, steps, want_logits=True)
    om.close()
    assert ids_s == [int(x) for x in oids[len(prompt):]]
    err = float(np.abs(lg_s - olg).max())
    assert err <= 2e-2, err
    return err


def test_step_long_context_crosses_2048(step_model):
    """A 2040-token prompt, then 16 steps at positions 2040-2055: the K rows
    of the first tile come from the prefetch, the later K tiles (positions
    512 and on, including the tile loop past the second tile) are loaded by
    the attention body, and V no longer fits the step's V tile (the product
    threads load it themselves); the decode crosses the 2048-position
    bucket boundary."""
    err = _step_vs_kernel_per_op_and_oracle(step_model, prompt_ids(2040, V, seed=13), 16)
    print(f"step at positions 2040-2055: max-abs logits diff to the oracle {err:.3e}")


@pytest.fixture(scope="module")
def window_model(model_dir):
    path = model_dir / "qwen2-0.5b-3l-w700-int8.ecm"
    if not path.exists():
        ec.synth(path, name="qwen2-0.5b-3l-w700", arch="qwen2", layers=3, embd=896, heads=14, kv_heads=2,
                 ffn=4864, ctx=32768, vocab=V, precision="int8", tie=1, sliding_window=700)
    return path


def test_step_sliding_window(window_model):
    """The Qwen2-0.5B per-layer shapes with a 700-position sliding window
    (src/gpt2.c:753-754): a 1000-token prompt, then 16 steps, so every step
    attends to positions [pos - 699, pos] -- the window branch (lo > 0) of
    the K and V prefetch, with more rows than the first K tile holds."""
    err = _step_vs_kernel_per_op_and_oracle(window_model, prompt_ids(1000, V, seed=17), 16)
    print(f"windowed step: max-abs logits diff to the oracle {err:.3e}")


def test_generate_greedy_timed(step_model):
    """ec_generate_greedy_timed: the ids of ec_generate_greedy, and per-step
    times from the GPU clock that are positive and add up to no more than the
    host's wall time around the call (and to most of it)."""
    import time

    prompt = prompt_ids(300, V, seed=21)
    n = len(prompt)
    with _load(step_model, n + 48, True) as m:
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        want = m.generate_greedy(int(prompt[-1]), n, 0, 40)
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        ec.lib().ec_sync()
        t0 = time.perf_counter()
        ids, ms = m.generate_greedy_timed(int(prompt[-1]), n, 0, 40)
        wall = (time.perf_counter() - t0) * 1e3
    assert [int(x) for x in ids] == [int(x) for x in want]
    assert (ms > 0).all(), ms
    assert ms.sum() <= wall, (ms.sum(), wall)
    assert ms.sum() >= 0.5 * wall, (ms.sum(), wall)
    assert float(np.median(ms)) < 5.0, ms
