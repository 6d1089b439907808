"""The batched decode's layer tail (decode_tail.hip): layer l's o projection,
RMSNorm, gate/up + SiLU and down, then layer l + 1's RMSNorm and q|k|v, in
one launch between two attentions, for up to 4 tokens in their own slots
(src/gpt2.c:667-805 at M = batch, src/runtime_main.c:336-345).

The tail repeats the batched GEMVs' arithmetic (the same norms, codes, exact
int32 dots and epilogues), so its logits must equal the kernel-per-op path's
(EDGECORE_TAIL=0) bit for bit, and its greedy ids the oracle's.  Cases: d_model
256 with FFN 5120 and 1040 (the widest FFN exchange; pair blocks past the last
row) and the Qwen2-0.5B layer shape (d_model 896, FFN 4864, 14 / 2 heads) at
2 layers, M = 1-4 (the one-token persistent step off, so that M = 1 runs the
tail too), direct launches and graph replays; and a forward whose tail reports
a timed-out wait (forced from the host) is redone through the GEMVs with the
same ids."""
import json
import os

import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests.conftest import prompt_ids

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q05_model(model_dir):
    path = model_dir / "qwen2-0.5b-2l-int8.ecm"
    if not path.exists():
        ec.synth(path, name="qwen2-0.5b-2l", arch="qwen2", layers=2, embd=896, heads=14, kv_heads=2,
                 ffn=4864, ctx=32768, vocab=151936, precision="int8", tie=1)
    return path


def _load(path, slots, ctx, tail):
    saved = {k: os.environ.get(k) for k in ("EDGECORE_TAIL", "EDGECORE_STEP")}
    os.environ["EDGECORE_TAIL"] = "1" if tail else "0"
    os.environ["EDGECORE_STEP"] = "0"
    try:
        return ec.Model(path, slots, ctx)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _families(m, fn):
    import ctypes as C
    L = ec.lib()
    L.ec_prof_start(b"")
    fn()
    buf = C.create_string_buffer(1 << 16)
    assert L.ec_prof_stop(buf, len(buf)) > 0, ec.last_error()
    return {k["kernel"] for k in json.loads(buf.value.decode())}


def _decode(path, B, steps, tail, prompt_len=12):
    """Per-slot prefills, then `steps` greedy steps at M = B: logits of every
    step (direct launches) and the ids of a second run of the same steps
    through graph replays (argmax only)."""
    with _load(path, B, prompt_len + B + 2 * steps + 8, tail) as m:
        V = m.vocab
        prompts = [prompt_ids(prompt_len + b, V, seed=40 + b) for b in range(B)]

        def prefill():
            m.kv_reset()
            for b, p in enumerate(prompts):
                n = len(p)
                m.forward(p, np.arange(n), np.full(n, b, np.int32), lm_from=n, want_logits=False)
            return [int(p[-1]) for p in prompts], [len(p) for p in prompts]

        cur, pos = prefill()
        lgs, ids, fams = [], [], None
        for s in range(steps):
            res = {}
            call = lambda: res.update(r=m.forward(cur, pos, None, want_logits=True, want_argmax=True))
            if s == 0:
                fams = _families(m, call)
            else:
                call()
            lg, am = res["r"]
            lgs.append(lg)
            cur, pos = [int(x) for x in am], [p + 1 for p in pos]
            ids.append(cur)
        cur, pos = prefill()
        gids = []
        for s in range(steps):
            _, am = m.forward(cur, pos, None, want_logits=False, want_argmax=True)
            cur, pos = [int(x) for x in am], [p + 1 for p in pos]
            gids.append(cur)
    return np.stack(lgs), ids, gids, fams, prompts


@pytest.mark.parametrize("name", ["qwen2-ffn5120-int8", "qwen2-ffn1040-int8"])
@pytest.mark.parametrize("B", [1, 2, 3, 4])
def test_tail_equals_kernel_per_op(make_model, name, B):
    path = make_model(name)
    lg_t, ids_t, gids_t, fam_t, prompts = _decode(path, B, 6, True)
    lg_k, ids_k, gids_k, fam_k, _ = _decode(path, B, 6, False)
    assert "decode_tail" in fam_t and "gemv_o" not in fam_t and "gemv_down" not in fam_t, sorted(fam_t)
    assert "decode_tail" not in fam_k and "gemv_o" in fam_k, sorted(fam_k)
    assert np.array_equal(lg_t.view(np.uint32), lg_k.view(np.uint32)), float(np.abs(lg_t - lg_k).max())
    assert ids_t == ids_k == gids_t == gids_k
    # and the oracle's greedy ids
    om = oracle.OracleModel(path, B, 64)
    om.kv_reset()
    for b, p in enumerate(prompts):
        om.forward(p, np.arange(len(p)), np.full(len(p), b, np.int32))
    cur, pos = [int(p[-1]) for p in prompts], [len(p) for p in prompts]
    for s in range(len(ids_t)):
        want = om.forward(cur, pos, None)
        assert np.abs(lg_t[s] - want).max() <= 2e-2
        assert [int(r.argmax()) for r in want] == ids_t[s], s
        cur, pos = ids_t[s], [p + 1 for p in pos]
    om.close()


@pytest.mark.parametrize("B", [1, 4])
def test_tail_qwen2_05b_shape(q05_model, B):
    """d_model 896, FFN 4864, q|k|v 1152 rows: 56 o/down, 76 gate/up and 72
    q|k|v blocks of the 256."""
    lg_t, ids_t, gids_t, fam_t, _ = _decode(q05_model, B, 4, True)
    lg_k, ids_k, gids_k, _, _ = _decode(q05_model, B, 4, False)
    assert "decode_tail" in fam_t, sorted(fam_t)
    assert np.array_equal(lg_t.view(np.uint32), lg_k.view(np.uint32)), float(np.abs(lg_t - lg_k).max())
    assert ids_t == ids_k == gids_t == gids_k


_CHILD = r"""
import json, os, sys
import numpy as np
import edgecore_amd as ec
from tests.conftest import prompt_ids
path = sys.argv[1]
os.environ["EDGECORE_STEP"] = "0"
with ec.Model(path, 3, 64) as m:
    prompts = [prompt_ids(12 + b, m.vocab, seed=40 + b) for b in range(3)]
    m.kv_reset()
    for b, p in enumerate(prompts):
        m.forward(p, np.arange(len(p)), np.full(len(p), b, np.int32), lm_from=len(p), want_logits=False)
    cur, pos, ids = [int(p[-1]) for p in prompts], [len(p) for p in prompts], []
    for s in range(5):
        _, am = m.forward(cur, pos, None, want_logits=s % 2 == 0, want_argmax=True)
        cur, pos = [int(x) for x in am], [p + 1 for p in pos]
        ids.append(cur)
print(json.dumps(ids))
"""


def test_tail_timeout_falls_back_to_gemvs(make_model):
    """A tail that reports a timed-out wait (forced from the host: no kernel
    is made to wait) is redone through the GEMVs, which are used from then
    on; the ids equal those of a run without the failure."""
    import subprocess
    import sys
    from pathlib import Path

    path = make_model("qwen2-ffn5120-int8")
    root = Path(__file__).resolve().parents[1]

    def child(env):
        e = dict(os.environ)
        e.update(env)
        r = subprocess.run([sys.executable, "-c", _CHILD, str(path)], cwd=root, env=e, capture_output=True,
                           text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        return json.loads(r.stdout.strip().splitlines()[-1]), r.stderr

    ok, _ = child({})
    failed, err = child({"EDGECORE_TAIL_TEST_FAIL": "1"})
    assert failed == ok
    assert "separate kernels from now on" in err, err[-500:]
