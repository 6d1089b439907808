"""The reference-signature forward entry points (src/edgecore.h:259-264)
called through the C ABI as a reference-built caller would: gpt2_forward and
qwen2_forward write every row's logits, equal to gpt2_forward_ex's on the same
inputs, and exit with status 1 and a message where the reference would
overrun (bad token, position past the cache) or run the wrong architecture."""
import ctypes as C
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import edgecore_amd as ec
from tests.conftest import REPO, prompt_ids

pytestmark = pytest.mark.gpu


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.mark.parametrize("name,entry", [("tiny-gpt2-int8", "gpt2_forward"), ("tiny-qwen2-int8", "gpt2_forward"),
                                        ("tiny-qwen2-int8", "qwen2_forward"), ("tiny-qwen2-bf16", "qwen2_forward")])
def test_reference_signature_forward_equals_forward_ex(make_model, name, entry):
    path = make_model(name)
    L = ec.lib()
    fn = getattr(L, entry)
    fn.restype = None
    fn.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_void_p]
    with ec.Model(path, 2, 64) as m:
        V = m.vocab
        toks = np.array(prompt_ids(12, V, seed=5), np.int32)
        pos = np.arange(12, dtype=np.int32)
        slot = np.ones(12, np.int32)
        m.kv_reset()
        want, _ = m.forward(toks, pos, slot)
        nxt_want, _ = m.forward([int(want[-1].argmax())], [12], [1])
        m.kv_reset()
        got = np.full((12, V), np.nan, np.float32)
        fn(C.byref(m.g), _ptr(toks), _ptr(pos), _ptr(slot), 12, _ptr(got))
        assert np.array_equal(got, want)
        # the KV cache it left behind is the same: the next step agrees too
        nxt = np.full((1, V), np.nan, np.float32)
        t1, p1, s1 = (np.array([x], np.int32) for x in (int(want[-1].argmax()), 12, 1))
        fn(C.byref(m.g), _ptr(t1), _ptr(p1), _ptr(s1), 1, _ptr(nxt))
        assert np.array_equal(nxt, nxt_want)


_CHILD = textwrap.dedent("""
    import ctypes as C, sys
    import numpy as np
    sys.path.insert(0, {repo!r})
    import edgecore_amd as ec
    L = ec.lib()
    fn = getattr(L, {entry!r})
    fn.restype = None
    fn.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_void_p]
    m = ec.Model({path!r}, 1, 32)
    t = np.array([{tok}], np.int32); p = np.array([{pos}], np.int32)
    out = np.zeros((1, m.vocab), np.float32)
    print("calling", flush=True)
    fn(C.byref(m.g), t.ctypes.data_as(C.c_void_p), p.ctypes.data_as(C.c_void_p), None, 1,
       out.ctypes.data_as(C.c_void_p))
    print("returned", flush=True)
""")


@pytest.mark.parametrize("name,entry,tok,pos,msg", [
    ("tiny-gpt2-int8", "gpt2_forward", 50257, 0, "token"),      # token == vocab
    ("tiny-gpt2-int8", "gpt2_forward", 5, 32, "position"),      # position == eff_ctx (--max-ctx 32)
    ("tiny-gpt2-int8", "qwen2_forward", 5, 0, "not a qwen2"),   # wrong architecture
])
def test_reference_signature_forward_exits_1(make_model, name, entry, tok, pos, msg):
    code = _CHILD.format(repo=str(REPO), entry=entry, path=str(make_model(name)), tok=tok, pos=pos)
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert p.returncode == 1, (p.returncode, p.stdout, p.stderr)
    assert "calling" in p.stdout and "returned" not in p.stdout
    assert msg in p.stderr, p.stderr
