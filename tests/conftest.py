import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds")


# Synthetic model shapes used by the tests, as ecm_synth arguments.
MODEL_SPECS = {
    # the reference's CPU-runnable case: tiny GPT-2 (L2 E64 H2 FFN256 ctx128 V50257) int8
    "tiny-gpt2-int8": dict(preset="tiny-gpt2"),
    "tiny-gpt2-fp16": dict(preset="tiny-gpt2", precision="fp16"),
    "tiny-qwen2-int8": dict(preset="tiny-qwen2"),
    "tiny-qwen2-fp16": dict(preset="tiny-qwen2", precision="fp16"),
    "tiny-qwen2-bf16": dict(preset="tiny-qwen2", precision="bf16"),
    "tiny-qwen2-tied": dict(preset="tiny-qwen2", tie=1, vocab=3000),
    # hd 128, GQA 6:1, an odd vocabulary and intermediate size
    "qwen2-hd128-int8": dict(arch="qwen2", layers=3, embd=768, heads=6, kv_heads=1, ffn=1000,
                             ctx=512, vocab=4099, precision="int8", tie=1),
    # sliding window 48 and YaRN RoPE (factor 4 over an original 64 positions)
    "qwen2-window-yarn-int8": dict(arch="qwen2", layers=2, embd=256, heads=4, kv_heads=2, ffn=384,
                                   ctx=256, vocab=1000, precision="int8", sliding_window=48,
                                   rope_type="yarn", yarn_factor=4.0, yarn_orig_max=64,
                                   yarn_attention_factor=1.1),
    # intermediate sizes past 1024: the batched down GEMV's wide quantizing
    # prologue (one wave per row up to 5120) and its clamped strips
    "qwen2-ffn5120-int8": dict(arch="qwen2", layers=2, embd=256, heads=4, kv_heads=2, ffn=5120,
                               ctx=128, vocab=1000, precision="int8"),
    "qwen2-ffn1040-int8": dict(arch="qwen2", layers=2, embd=256, heads=4, kv_heads=2, ffn=1040,
                               ctx=128, vocab=1000, precision="int8"),
    # long context: decode crosses 512-position boundaries
    "qwen2-long-int8": dict(arch="qwen2", layers=2, embd=128, heads=4, kv_heads=2, ffn=256,
                            ctx=1536, vocab=1000, precision="int8"),
    # reference smoke-test shape (scripts/make_synthetic.py defaults), byte vocab
    "smoke-gpt2-int8": dict(arch="gpt2", layers=2, embd=32, heads=2, ctx=64, vocab=256,
                            precision="int8"),
    "smoke-gpt2-fp16": dict(arch="gpt2", layers=2, embd=32, heads=2, ctx=64, vocab=256,
                            precision="fp16"),
}


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


@pytest.fixture(scope="session")
def make_model(model_dir):
    import edgecore_amd as ec

    cache = {}

    def _make(name: str) -> Path:
        if name not in cache:
            out = model_dir / f"{name}.ecm"
            ec.synth(out, name=name, **MODEL_SPECS[name])
            cache[name] = out
        return cache[name]

    return _make


def prompt_ids(n: int, vocab: int, seed: int = 1):
    """Prompt ids uniform in [0, vocab) from the generator's prompt stream."""
    import tempfile

    import edgecore_amd as ec

    with tempfile.TemporaryDirectory() as d:
        p = Path(d) / "p.txt"
        ec.synth(None, prompt_out=p, prompt_len=n, prompt_seed=seed, vocab=vocab)
        return ec.read_ids(p)
