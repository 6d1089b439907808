"""The GPU path against the golden fixtures written by the reference CPU
runtime itself (tests/golden/make_golden.py, reference src/ built from
source): kernel vectors and greedy decoding of seeded models, including the
Qwen2-0.5B shape with its 256-token prompt.

int8 GEMM vectors: bit-exact.  fp16/bf16 GEMM vectors: within 2K*2^-24*sum|ab|.
Models: the 32 greedy ids identical, every step's top-5 logits within 2e-2
(int8) / 1e-2 (16-bit) of the reference's.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import edgecore_amd as ec

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_kernel_vectors():
    g = np.load(GOLDEN / "kernels.npz")
    i = 0
    while f"i8_{i}_A" in g.files:
        C = ec.gemm_int8(g[f"i8_{i}_A"], g[f"i8_{i}_as"], g[f"i8_{i}_B"],
                         g[f"i8_{i}_bs"] if f"i8_{i}_bs" in g.files else None,
                         g[f"i8_{i}_bias"] if f"i8_{i}_bias" in g.files else None)
        assert np.array_equal(C.view(np.uint32), g[f"i8_{i}_C"].view(np.uint32)), i
        i += 1
    for kind, fn in (("f16", ec.gemm_fp16_fp32), ("bf16", ec.gemm_bf16_fp32)):
        i = 0
        while f"{kind}_{i}_A" in g.files:
            A, B, Cref = g[f"{kind}_{i}_A"], g[f"{kind}_{i}_B"], g[f"{kind}_{i}_C"]
            Bf = (B.astype(np.uint32) << 16).view(np.float32) if kind == "bf16" else B.view(np.float16).astype(np.float32)
            bound = 2 * A.shape[1] * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(Bf).astype(np.float64).T)
            assert np.all(np.abs(fn(A, B) - Cref) <= bound + 1e-30), (kind, i)
            i += 1


@pytest.mark.parametrize("name", ["tiny-gpt2-int8", "tiny-gpt2-fp16", "tiny-qwen2-int8", "tiny-qwen2-bf16",
                                  "qwen2-0.5b-int8"])
def test_greedy_decode_matches_reference(name, tmp_path):
    g = json.loads((GOLDEN / "models.json").read_text())[name]
    path = tmp_path / f"{name}.ecm"
    ec.synth(path, name=name, **g["synth"])
    assert hashlib.sha256(path.read_bytes()).hexdigest() == g["file_sha256"]
    prompt = np.array(g["prompt"], np.int32)
    with ec.Model(path, 1, g["max_ctx"]) as m:
        tol = 2e-2 if m.precision == 0 else 1e-2
        ids, steps = m.generate(prompt, 32, want_logits=True)
    assert [int(x) for x in ids[len(prompt):]] == g["ids"]
    err = 0.0
    for s, top in enumerate(g["top5"]):
        for j, v in top:
            err = max(err, abs(float(steps[s, j]) - v))
    print(f"{name}: max |logit - reference| over the top-5 of 32 steps = {err:.3e}")
    assert err <= tol
