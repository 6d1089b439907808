"""The persistent decode step of the fp16 GPT-2 forward (decode_step_gpt2.hip)
against the kernel-per-operation forward it replaces for one-token steps
(src/gpt2.c:470-581 at M = 1), and against the oracle.

The GPT-2 small per-layer shapes (d_model 768, 12 heads of head_dim 64, GELU
FFN 3072, LayerNorm, biases, learned positions) at 3 layers, fp16 weights.
The step's fp16 dots are fp32 sums in an order of their own, so its logits
equal the kernel-per-op path's within a small tolerance (2e-3) rather than
bit for bit; both must give the oracle's greedy tokens and stay within the
fp16 bar (max-abs 1e-2) of its logits.  The decode crosses position 512 (a
512-position graph bucket, and the step's attention's second position per
thread) and runs up to position 1009 of the 1024 the step holds."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = pytest.mark.gpu

V = 50257


@pytest.fixture(scope="module")
def g2_model(model_dir):
    path = model_dir / "gpt2-small-3l-fp16.ecm"
    if not path.exists():
        ec.synth(path, name="gpt2-small-3l", arch="gpt2", layers=3, embd=768, heads=12, ffn=3072, ctx=1024,
                 vocab=V, precision="fp16")
    return path


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


def _families(fn):
    L = ec.lib()
    L.ec_prof_start(b"")
    fn()
    buf = C.create_string_buffer(1 << 16)
    assert L.ec_prof_stop(buf, len(buf)) > 0, ec.last_error()
    return {k["kernel"]: k for k in json.loads(buf.value.decode())}


def _decode(path, prompt, steps, step_on):
    with _load(path, len(prompt) + steps + 8, step_on) as m:
        n = len(prompt)
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        cur, pos, out, ids, fams = int(prompt[-1]), n, [], [], None
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


@pytest.mark.parametrize("n,steps", [(500, 24), (1, 12), (990, 20)])
def test_gpt2_step_against_kernel_per_op_and_oracle(g2_model, n, steps):
    prompt = prompt_ids(n, V, seed=21)
    lg_s, ids_s, fam_s = _decode(g2_model, prompt, steps, True)
    lg_k, ids_k, fam_k = _decode(g2_model, prompt, steps, False)
    assert "decode_step" in fam_s and "gemv_qkv" not in fam_s, sorted(fam_s)
    assert "decode_step" not in fam_k and "gemv_qkv" in fam_k, sorted(fam_k)
    err_k = float(np.abs(lg_s - lg_k).max())
    print(f"GPT-2 step vs kernel-per-op: max-abs {err_k:.3e}")
    assert ids_s == ids_k
    assert err_k <= 2e-3, err_k
    om = oracle.OracleModel(g2_model, 1, n + steps + 8)
    oids, olg = om.generate(prompt, steps, want_logits=True)
    om.close()
    assert ids_s == [int(x) for x in oids[n:]]
    err_o = float(np.abs(lg_s - olg).max())
    print(f"GPT-2 step vs oracle: max-abs {err_o:.3e}")
    assert err_o <= 1e-2, err_o


def test_gpt2_generate_greedy_equals_step_loop(g2_model):
    """ec_generate_greedy (steps chained on the device through the GPT-2 step,
    one HIP graph per 512-position bucket) gives the host-driven loop's ids
    across the 512-position boundary, in one call and in two."""
    prompt = prompt_ids(500, V, seed=21)
    n = len(prompt)
    _, ids_s, _ = _decode(g2_model, prompt, 24, True)
    with _load(g2_model, n + 24 + 8, True) as m:
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        assert [int(x) for x in m.generate_greedy(int(prompt[-1]), n, 0, 24)] == ids_s
        m.kv_reset()
        m.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n, want_logits=False)
        a = m.generate_greedy(int(prompt[-1]), n, 0, 10)
        b = m.generate_greedy(int(a[-1]), n + 10, 0, 14)
        assert [int(x) for x in a] + [int(x) for x in b] == ids_s
