"""The edgecore-runtime CLI contract on the GPU, as pinned by the reference's
scripts/smoke_test.sh:26-86 and consumed by edgecore/bench.py:147-151 and
edgecore/verify.py:126-136."""
import json
import subprocess

import numpy as np
import pytest

import edgecore_amd as ec
import oracle

pytestmark = pytest.mark.gpu


def run(*args, check=True):
    p = subprocess.run([str(ec.RUNTIME), *map(str, args)], capture_output=True, text=True, timeout=300)
    if check and p.returncode != 0:
        raise AssertionError(f"rc={p.returncode}\n{p.stderr}")
    return p


def test_logits_json_int8(make_model):
    path = make_model("smoke-gpt2-int8")
    d = json.loads(run("--model", path, "--mode", "logits", "--prompt", "hello world").stdout)
    assert d["precision"] == "int8"
    assert d["n_tokens"] == 11 and len(d["logits"]) == 11
    assert all(len(r) == 256 for r in d["logits"])
    assert d["tokens"] == list(b"hello world")


def test_logits_json_fp16_and_affinity_key(make_model):
    path = make_model("smoke-gpt2-fp16")
    d = json.loads(run("--model", path, "--mode", "logits", "--prompt", "hello world").stdout)
    assert d["precision"] == "fp16" and len(d["logits"]) == 11
    assert "affinity_cpus" in d


def test_logits_bin_layout_matches_oracle(make_model, tmp_path):
    path = make_model("smoke-gpt2-int8")
    (tmp_path / "t.txt").write_text("0 1 2 3 4 5 6 7 8 9 10\n")
    run("--model", path, "--mode", "logits", "--tokens-file", tmp_path / "t.txt",
        "--logits-bin", tmp_path / "l.bin", "--logits-limit", 64)
    raw = (tmp_path / "l.bin").read_bytes()
    n, V = np.frombuffer(raw[:8], np.int32)
    toks = np.frombuffer(raw[8:8 + 4 * n], np.int32)
    lg = np.frombuffer(raw[8 + 4 * n:], np.float32).reshape(n, V)
    assert n == 11 and V == 256 and list(toks) == list(range(11))
    om = oracle.OracleModel(path)
    want = om.forward(toks, np.arange(n), np.zeros(n, np.int32))
    assert np.abs(lg - want).max() <= 2e-2


def test_generate_keys_and_sampling(make_model):
    path = make_model("smoke-gpt2-int8")
    d = json.loads(run("--model", path, "--mode", "generate", "--prompt", "hello world",
                       "--n-tokens", 16, "--temp", 0.7, "--top-k", 40, "--seed", 1,
                       "--no-print").stdout)
    assert d["n_generated_tokens"] == 16
    assert d["ttft_ms"] >= 0 and d["tpot_avg_ms"] > 0
    assert d["tokens_per_sec"] > 0 and d["p50_ms"] > 0
    assert d["affinity_requested"] == "none"


def test_generate_greedy_ids_match_oracle(make_model, tmp_path):
    path = make_model("tiny-gpt2-int8")
    from tests.conftest import prompt_ids
    prompt = prompt_ids(8, 50257, seed=1)
    (tmp_path / "p.txt").write_text(" ".join(map(str, prompt)))
    d = json.loads(run("--model", path, "--mode", "generate", "--tokens-file", tmp_path / "p.txt",
                       "--n-tokens", 32, "--max-ctx", 48, "--no-print").stdout)
    om = oracle.OracleModel(path, 1, 48)
    ids, _ = om.generate(prompt, 32)
    assert d["token_ids"] == [int(x) for x in ids[8:]]


def test_bench_keys_batch2(make_model):
    path = make_model("smoke-gpt2-fp16")
    d = json.loads(run("--model", path, "--mode", "bench", "--prompt", "hello world", "--n-tokens", 16,
                       "--warmup", 1, "--iters", 3, "--batch", 2, "--threads", 2,
                       "--affinity", "physical").stdout)
    assert d["n_generated_tokens"] == 32
    # the mean may exceed the 95th percentile when one step is slow; the
    # percentiles themselves are ordered
    assert d["avg_token_ms"] > 0 and 0 < d["p50_ms"] <= d["p95_ms"] <= d["p99_ms"]
    assert d["tokens_per_sec"] > 0 and d["tokens_per_sec_aggregate"] > 0
    assert d["affinity_applied"] is True and len(d["affinity_cpus"]) >= 1
    assert "ttft_p95_ms" in d and "ttft_p99_ms" in d
    for k in ("avg_token_ms", "ttft_avg_ms", "p50_ms", "p95_ms", "p99_ms", "tokens_per_sec",
              "peak_rss_gb", "n_generated_tokens", "iterations"):
        assert k in d


def test_exit_codes(make_model, tmp_path):
    path = make_model("smoke-gpt2-int8")
    assert run("--model", path, "--precision", "fp16", "--mode", "logits", check=False).returncode == 2
    assert run("--model", path, "--mode", "nope", check=False).returncode == 2
    assert run("--model", tmp_path / "missing.ecm", check=False).returncode == 1
    # prompt + n-tokens beyond the context is refused instead of overrunning the cache
    assert run("--model", path, "--mode", "generate", "--prompt", "hello world", "--n-tokens", 60,
               "--no-print", check=False).returncode == 2


@pytest.fixture(scope="module")
def step_model(model_dir):
    """Qwen2-0.5B per-layer shapes at 3 layers: its one-token greedy steps run
    through the persistent decode step"""
    path = model_dir / "qwen2-0.5b-3l-int8.ecm"
    if not path.exists():
        ec.synth(path, name="qwen2-0.5b-3l", arch="qwen2", layers=3, embd=896, heads=14, kv_heads=2, ffn=4864,
                 ctx=32768, vocab=151936, precision="int8", tie=1)
    return path


def test_greedy_batch1_chained_with_gpu_clock(step_model, tmp_path):
    """At batch 1 with greedy decoding the driver chains the steps on the GPU
    (ec_generate_greedy_timed) and times them with the GPU's clock: the same
    ids as the oracle's greedy loop, in generate and in bench mode."""
    from tests.conftest import prompt_ids
    prompt = prompt_ids(200, 151936, seed=3)
    (tmp_path / "p.txt").write_text(" ".join(map(str, prompt)))
    d = json.loads(run("--model", step_model, "--mode", "generate", "--tokens-file", tmp_path / "p.txt",
                       "--n-tokens", 24, "--max-ctx", 240, "--no-print").stdout)
    assert d["step_timing"] == "gpu-clock"
    om = oracle.OracleModel(step_model, 1, 240)
    ids, _ = om.generate(prompt, 24)
    om.close()
    assert d["token_ids"] == [int(x) for x in ids[200:]]
    assert 0 < d["p50_ms"] <= d["p95_ms"] and d["tokens_per_sec"] > 0
    b = json.loads(run("--model", step_model, "--mode", "bench", "--tokens-file", tmp_path / "p.txt",
                       "--n-tokens", 24, "--warmup", 1, "--iters", 2, "--max-ctx", 240).stdout)
    assert b["step_timing"] == "gpu-clock" and b["n_generated_tokens"] == 24
    assert 0 < b["p50_ms"] <= b["p95_ms"] <= b["p99_ms"] and b["tokens_per_sec"] > 0
