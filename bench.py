#!/usr/bin/env python3
"""Decode benchmark of the EdgeCore MI355X path on the Qwen2-0.5B int8 shape.

Workload (bs=1): Qwen2-0.5B architecture (24 layers, d_model 896, 14/2 heads,
head_dim 64, SwiGLU 4864, vocab 151936 tied), int8 per-output-channel weights
N(0, 0.02) from seed 0 (synthetic, bin/ecm_synth), a 256-token prompt of ids
uniform in [0, 151936) from seed 1, greedy decoding.  One step is one decode
token: the forward at M=1 plus the GPU argmax.  The steps run through
ec_generate_greedy, which chains them on the device (each argmax id becomes
the next step's token there; the K ids come back to the host at the end;
runs of 16 steps inside one 512-position bucket are one HIP graph launch).
The prompt is prefilled first (reported as prefill tok/s, untimed), then W
warmup steps, then the K steps once untimed (their graphs are captured on
first use), then the same K steps timed, bracketed by stream
synchronisation; both runs give the same ids.

Two passes of the same K steps run, each after the same prefill and warmup.
In the first, every kernel launch records its own dispatch start and stop on
HIP events (hipExtLaunchKernel on the library's stream, ec_prof_*; with the
profiler on, ec_generate_greedy runs one host-driven step per token): that
gives the per-kernel table and the launch durations of the roofline object
(the family with the largest total time: the persistent decode step, which
runs every layer; int8_weight_stream: the layers' int8 weights and scales per
step over that kernel's time; roofline_lm_head: the fp16 LM head;
roofline_int8_gemv: the largest separate int8 GEMV family, when the step is
off).  The second is the timed region
proper (value, ms_per_step), with nothing but the work.  The launch durations
agree with rocprofv3's kernel trace of the same command (profiles/), and
both passes must produce the same tokens.  roofline.traffic is the HBM bytes
per launch measured with rocprofv3 counters (profiles/traffic.json).  The
CPU baseline is the reference runtime built from its own sources
(oracle/_ref/edgecore-runtime) on the same model file and prompt, timed on
the host cores.

prefill_4x2048 is the prefill-heavy workload on the same model: 4 prompts of
2048 ids, prefilled one slot at a time, then 32 decode steps at M=4, with the
matrix-core GEMMs' TOP/s against the int8 dense peak.  It is reported beside
the decode line, not as its value.

gpt2_small_fp16: GPT-2 small with fp16 weights, a 128-token prompt prefilled
on the 16-bit matrix-core GEMM (TFLOP/s against the fp16 dense peak), then
128 greedy decode steps; the step's bytes (about 254 MB) fit in the 256 MiB
Infinity Cache, which the line flags.  qwen25_1.5b_int8_m16: the
Qwen2.5-1.5B shape in int8, 16 prompts of 1024 ids each prefilled into its
own slot, then 256 greedy steps at M=16 (GB/s of the skinny int8 GEMMs).
Both are reported beside the decode line.

Prints one JSON line.
"""
import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "decode tok/s + int8 GEMV HBM GB/s (% of peak), Qwen2-0.5B-shape int8 bs=1"
HBM_PEAK_GBPS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix-core peak, TOP/s
PROMPT = 256
# prefill-heavy workload: 4 prompts of 2048 ids (seeds 1..4), one slot each,
# prefilled one at a time as the reference driver does, then 32 decode steps at M=4
C4_PROMPT, C4_SEQS, C4_DECODE = 2048, 4, 32


def ensure_inputs(cache: Path):
    import edgecore_amd as ec

    cache.mkdir(parents=True, exist_ok=True)
    model = cache / "qwen2-0.5b-int8.ecm"
    prompt = cache / "prompt256.txt"
    if not model.exists():
        tmp = cache / "qwen2-0.5b-int8.ecm.tmp"
        ec.synth(tmp, preset="qwen2-0.5b")
        tmp.rename(model)
    if not prompt.exists():
        ec.synth(None, prompt_out=prompt, prompt_len=PROMPT, prompt_seed=1, vocab=151936)
    return model, prompt


def prefill_c4(ec, np, model: Path, cache: Path):
    """4 x 2048-token prefills into slots 0..3 (each with the LM head on its
    last row and the device argmax, i.e. time to first token), then 2 untimed
    and 32 timed greedy decode steps at M=4.  A second pass of one prefill records every launch's
    dispatch timestamps: the per-family table and the matrix-core GEMMs'
    TOP/s (2*M*N*K per launch)."""
    E, F, kv = 896, 4864, 128
    prompts = []
    for b in range(C4_SEQS):
        f = cache / f"prompt{C4_PROMPT}_s{b + 1}.txt"
        if not f.exists():
            ec.synth(None, prompt_out=f, prompt_len=C4_PROMPT, prompt_seed=b + 1, vocab=151936)
        prompts.append(ec.read_ids(f))
    m = ec.Model(model, C4_SEQS, C4_PROMPT + C4_DECODE + 8)
    L = ec.lib()
    n = C4_PROMPT
    pos = np.arange(n)

    def prefill(b):
        _, am = m.forward(prompts[b], pos, np.full(n, b, np.int32), lm_from=n - 1, want_logits=False,
                          want_argmax=True)
        return int(am[0])

    m.kv_reset()
    prefill(0)  # warm
    m.kv_reset()
    L.ec_sync()
    t0 = time.perf_counter()
    first = [prefill(b) for b in range(C4_SEQS)]
    L.ec_sync()
    t_prefill = time.perf_counter() - t0

    cur, p = list(first), [n] * C4_SEQS

    def decode(k):
        nonlocal cur, p
        for _ in range(k):
            _, am = m.forward(cur, p, None, want_logits=False, want_argmax=True)
            cur, p = [int(x) for x in am], [x + 1 for x in p]

    # two untimed steps first: the first step at M=4 in a 512-position bucket
    # captures that bucket's graph
    decode(2)
    L.ec_sync()
    t0 = time.perf_counter()
    decode(C4_DECODE)
    L.ec_sync()
    t_decode = time.perf_counter() - t0
    # four more M=4 steps with per-launch timestamps (launched directly, not
    # as the graph: the per-family table of a decode step)
    dec_kernels = _prof(L, lambda: decode(4))

    # one more prefill of slot 0 with per-launch timestamps
    L.ec_prof_start(b"")
    prefill(0)
    L.ec_sync()
    buf = __import__("ctypes").create_string_buffer(1 << 16)
    kernels = json.loads(buf.value.decode()) if L.ec_prof_stop(buf, len(buf)) > 0 else []
    m.close()
    shapes = {"gemm_qkv": (E + 2 * kv, E), "gemm_o": (E, E), "gemm_gateup": (2 * F, E), "gemm_down": (E, F)}
    tot = sum(k["total_us"] for k in kernels) or 1.0
    for k in kernels:
        k["share"] = round(k["total_us"] / tot, 4)
        if k["kernel"] in shapes:
            N_, K_ = shapes[k["kernel"]]
            k["tops"] = round(2.0 * n * N_ * K_ / (k["avg_us"] * 1e6), 1)
            k["int8_mfma_frac"] = round(k["tops"] / INT8_PEAK_TOPS, 4)
    gemms = [k for k in kernels if k["kernel"] in shapes]
    gflop = sum(2.0 * n * shapes[k["kernel"]][0] * shapes[k["kernel"]][1] * k["launches"] for k in gemms)
    gus = sum(k["total_us"] for k in gemms)
    dom = max(gemms, key=lambda k: k["total_us"]) if gemms else None
    return {
        "workload": f"Qwen2-0.5B-shape int8, {C4_SEQS} x {C4_PROMPT}-token prompts (seeds 1-{C4_SEQS}), "
                    f"one slot each, prefilled one at a time; then {C4_DECODE} greedy steps at M={C4_SEQS}",
        "prefill_tok_s": round(C4_SEQS * n / t_prefill, 1),
        "ms_per_prompt": round(t_prefill / C4_SEQS * 1e3, 3),
        "batched_decode_tok_s": round(C4_SEQS * C4_DECODE / t_decode, 1),
        "batched_decode_ms_per_step": round(t_decode / C4_DECODE * 1e3, 4),
        "gemm_roofline": None if not dom else {
            "kernel": dom["kernel"], "bound": "mfma", "achieved": dom["tops"], "peak": INT8_PEAK_TOPS,
            "unit": "TOP/s (int8)", "frac": dom["int8_mfma_frac"], "avg_us": dom["avg_us"]},
        "gemm_all_tops": round(gflop / (gus * 1e6), 1) if gus else None,
        "kernels": kernels,
        "decode_kernels": dec_kernels,
    }


FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix-core peak, TFLOP/s
MALL_BYTES = 256 * 2 ** 20  # MI355X Infinity Cache (last-level, memory-side)


def _prompts(ec, cache: Path, n: int, count: int, vocab: int):
    out = []
    for b in range(count):
        f = cache / f"prompt{n}_v{vocab}_s{b + 1}.txt"
        if not f.exists():
            ec.synth(None, prompt_out=f, prompt_len=n, prompt_seed=b + 1, vocab=vocab)
        out.append(ec.read_ids(f))
    return out


def _prof(L, fn):
    """run fn with per-launch dispatch timestamps; the per-family table"""
    L.ec_sync()
    L.ec_prof_start(b"")
    fn()
    L.ec_sync()
    buf = __import__("ctypes").create_string_buffer(1 << 16)
    return json.loads(buf.value.decode()) if L.ec_prof_stop(buf, len(buf)) > 0 else []


def _batched_leg(ec, np, model: Path, prompts, n_decode: int, prof_steps: int):
    """prefill every prompt into its own slot (one at a time, LM head on the
    last row and device argmax: time to first token), then n_decode greedy
    steps with one token per slot; then a pass with per-launch timestamps of
    one prefill and of prof_steps more decode steps"""
    B, n = len(prompts), len(prompts[0])
    m = ec.Model(model, B, n + n_decode + prof_steps + 8)
    L = ec.lib()
    pos = np.arange(n)

    def prefill(b):
        _, am = m.forward(prompts[b], pos, np.full(n, b, np.int32), lm_from=n - 1, want_logits=False,
                          want_argmax=True)
        return int(am[0])

    m.kv_reset()
    prefill(0)  # warm
    m.kv_reset()
    L.ec_sync()
    t0 = time.perf_counter()
    cur = [prefill(b) for b in range(B)]
    L.ec_sync()
    t_prefill = time.perf_counter() - t0
    p = [n] * B

    def decode(k):
        nonlocal cur, p
        for _ in range(k):
            _, am = m.forward(cur, p, None, want_logits=False, want_argmax=True)
            cur, p = [int(x) for x in am], [x + 1 for x in p]

    decode(2)  # warm the decode path (graph capture at M=1)
    L.ec_sync()
    t0 = time.perf_counter()
    decode(n_decode)
    L.ec_sync()
    t_decode = time.perf_counter() - t0
    dec_kernels = _prof(L, lambda: decode(prof_steps))
    pre_kernels = _prof(L, lambda: prefill(0))
    m.close()
    return t_prefill, t_decode, pre_kernels, dec_kernels


def _gemm_rates(kernels, shapes, rows, peak, unit):
    """TFLOP/s (TOP/s) of the matrix-core GEMM families over a prefill of rows
    tokens: 2 * rows * N * K per launch"""
    out = []
    for k in kernels:
        if k["kernel"] in shapes:
            N_, K_ = shapes[k["kernel"]]
            r = 2.0 * rows * N_ * K_ / (k["avg_us"] * 1e6)
            out.append({"kernel": k["kernel"], "avg_us": k["avg_us"], "launches": k["launches"],
                        "achieved": round(r, 1), "peak": peak, "unit": unit, "frac": round(r / peak, 4)})
    return sorted(out, key=lambda x: -x["avg_us"] * x["launches"])


def leg_gpt2_small_fp16(ec, np, cache: Path):
    """GPT-2 small, fp16 weights N(0, 0.02) from seed 0: a 128-token prompt
    (ids uniform in [0, 50257), seed 1) prefilled on the 16-bit matrix-core
    path, then 128 greedy decode steps (positions 128-255)."""
    E, F, L_, V, n, steps = 768, 3072, 12, 50257, 128, 128
    model = cache / "gpt2-small-fp16.ecm"
    if not model.exists():
        tmp = cache / "gpt2-small-fp16.ecm.tmp"
        ec.synth(tmp, preset="gpt2-small")
        tmp.rename(model)
    prompts = _prompts(ec, cache, n, 1, V)
    t_pre, t_dec, pre_k, dec_k = _batched_leg(ec, np, model, prompts, steps, 16)
    # bytes of one decode step: fp16 weights, fp32 biases and LayerNorm
    # parameters, the tied fp16 LM head, and the fp16 K/V read at the mean position
    w = L_ * ((4 * E * E + 2 * E * F) * 2 + (6 * E + F) * 4 + 4 * E * 4) + V * E * 2 + 2 * E * 4
    mean_pos = n + (steps - 1) / 2.0 + 2
    kv = L_ * (mean_pos + 1) * E * 2 * 2
    step_bytes = w + kv
    shapes = {"gemm_qkv": (3 * E, E), "gemm_o": (E, E), "gemm_fc": (F, E), "gemm_down": (E, F)}
    gem = _gemm_rates(pre_k, shapes, n, FP16_PEAK_TFLOPS, "TFLOP/s (fp16)")
    dom_dec = max(dec_k, key=lambda k: k["total_us"]) if dec_k else None
    return {
        "workload": f"GPT-2 small fp16 bs1: {n}-token prompt, then {steps} greedy decode steps",
        "prefill_tok_s": round(n / t_pre, 1), "ttft_ms": round(t_pre * 1e3, 3),
        "decode_tok_s": round(steps / t_dec, 1), "ms_per_step": round(t_dec / steps * 1e3, 4),
        "decode_bytes_per_step": int(step_bytes),
        "decode_effective_gbps": round(step_bytes * steps / t_dec / 1e9, 1),
        "decode_hbm_frac": round(step_bytes * steps / t_dec / 1e9 / HBM_PEAK_GBPS, 4),
        "fits_in_mall": step_bytes < MALL_BYTES,
        "mall_note": "the step's weights, LM head and KV cache total less than the 256 MiB Infinity Cache, "
                     "so repeated steps may be served partly from it: effective GB/s is not an HBM figure",
        "prefill_gemms": gem,
        "decode_dominant_kernel": None if not dom_dec else {
            "kernel": dom_dec["kernel"], "avg_us": dom_dec["avg_us"], "gbps": dom_dec["gbps"]},
        "prefill_kernels": pre_k, "decode_kernels": dec_k,
    }


def leg_qwen25_15b_int8_m16(ec, np, cache: Path, n=1024, steps=256):
    """Qwen2.5-1.5B shape, int8 per-channel weights N(0, 0.02) from seed 0:
    16 prompts of 1024 ids (seeds 1-16), each prefilled into its own slot, then
    256 greedy decode steps at M=16 (one token per slot): the skinny M=16
    int8 matrix-core GEMMs."""
    E, F, kvd, L_, V, B = 1536, 8960, 256, 28, 151936, 16
    model = cache / "qwen2.5-1.5b-int8.ecm"
    if not model.exists():
        tmp = cache / "qwen2.5-1.5b-int8.ecm.tmp"
        ec.synth(tmp, preset="qwen2.5-1.5b")
        tmp.rename(model)
    prompts = _prompts(ec, cache, n, B, V)
    t_pre, t_dec, pre_k, dec_k = _batched_leg(ec, np, model, prompts, steps, 8)
    lin = E * (E + 2 * kvd) + E * E + 3 * F * E
    rows = (E + 2 * kvd) + E + 2 * F + E
    w = L_ * (lin + 4 * rows + 2 * E * 4 + (E + 2 * kvd) * 4) + V * E * 2
    mean_pos = n + (steps - 1) / 2.0 + 2
    kv = B * L_ * (mean_pos + 1) * kvd * 2 * 2
    step_bytes = w + kv
    shapes = {"gemm_qkv": (E + 2 * kvd, E), "gemm_o": (E, E), "gemm_gateup": (2 * F, E), "gemm_down": (E, F)}
    dec_gemms = []
    for k in dec_k:
        if k["kernel"] in shapes:
            dec_gemms.append({"kernel": k["kernel"], "avg_us": k["avg_us"], "launches": k["launches"],
                              "achieved": k["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                              "frac": round(k["gbps"] / HBM_PEAK_GBPS, 4)})
    dec_gemms.sort(key=lambda x: -x["avg_us"] * x["launches"])
    return {
        "workload": f"Qwen2.5-1.5B-shape int8: {B} prompts of {n} ids, one slot each, prefilled one at a "
                    f"time; then {steps} greedy decode steps at M={B}",
        "prefill_tok_s": round(B * n / t_pre, 1), "ms_per_prompt": round(t_pre / B * 1e3, 3),
        "decode_tok_s": round(B * steps / t_dec, 1), "ms_per_step": round(t_dec / steps * 1e3, 4),
        "decode_bytes_per_step": int(step_bytes),
        "decode_effective_gbps": round(step_bytes * steps / t_dec / 1e9, 1),
        "decode_hbm_frac": round(step_bytes * steps / t_dec / 1e9 / HBM_PEAK_GBPS, 4),
        "decode_m16_gemms": dec_gemms,
        "prefill_gemms": _gemm_rates(pre_k, shapes, n, INT8_PEAK_TOPS, "TOP/s (int8)"),
        "prefill_kernels": pre_k, "decode_kernels": dec_k,
    }


def cpu_info():
    """(model name, physical cores of socket 0 among the CPUs this process may
    run on, the cgroup CPU quota in whole CPUs or None)"""
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    allowed = os.sched_getaffinity(0)
    phys = 0
    try:
        out = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], capture_output=True, text=True).stdout
        cores = set()
        for l in out.splitlines():
            if not l or l.startswith("#"):
                continue
            cpu, core, sock = l.split(",")[:3]
            if sock == "0" and int(cpu) in allowed:
                cores.add(core)
        phys = len(cores)
    except Exception:
        pass
    quota = None
    try:
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(per)))
    except Exception:
        pass
    return model, phys or len(allowed), quota


def cpu_baseline(model: Path, prompt: Path, n_tokens: int):
    """The reference CPU runtime (built from its sources) on a bounded sample
    of the same workload: the same 256-token prefill, then n_tokens greedy
    decode steps; once with one thread and once with one socket's physical
    cores (capped by the cgroup CPU quota, where one is set, since threads
    beyond it would time-share).  tok/s is the reference's own bench-mode
    figure: decode tokens over decode time."""
    sys.path.insert(0, str(REPO))
    import oracle

    cpu_model, phys, quota = cpu_info()
    threads_p = min(phys, quota) if quota else phys

    def run(threads):
        cmd = [str(oracle.REF_RUNTIME), "--model", str(model), "--mode", "bench", "--tokens-file",
               str(prompt), "--n-tokens", str(n_tokens), "--warmup", "0", "--iters", "1",
               "--threads", str(threads), "--affinity", "physical", "--max-ctx",
               str(PROMPT + n_tokens + 8), "--no-print"]
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
        if p.returncode != 0:
            raise RuntimeError(f"reference runtime exited {p.returncode}: {p.stderr[-300:]}")
        return json.loads(p.stdout)

    if oracle.REF_RUNTIME.exists():
        d1 = run(1)
        dp = run(threads_p) if threads_p > 1 else d1
        sample = (f"reference runtime_main.c/gpt2.c/kernels.c built with gcc -O3 -mavx2 -mfma -mf16c; "
                  f"same model and 256-token prompt; {n_tokens} greedy decode steps after the prefill; "
                  f"--affinity physical; CPU {cpu_model!r}; socket 0 has {phys} physical cores among the "
                  f"allowed CPUs; cgroup CPU quota {quota if quota else 'none'}")
        return {"value": dp["tokens_per_sec"], "unit": "tok/s", "cores": threads_p, "kind": "reference",
                "sample": sample, "cpu_model": cpu_model, "threads": threads_p,
                "ttft_ms": dp.get("ttft_avg_ms"), "avg_token_ms": dp.get("avg_token_ms"),
                "single_thread": {"value": d1["tokens_per_sec"], "unit": "tok/s", "cores": 1,
                                  "ttft_ms": d1.get("ttft_avg_ms"), "avg_token_ms": d1.get("avg_token_ms")}}
    # the C restatement (oracle port) when the reference build is absent
    import numpy as np

    om = oracle.OracleModel(model, 1, PROMPT + n_tokens + 8)
    ids = [int(x) for x in Path(prompt).read_text().split()]
    om.kv_reset()
    om.forward(ids, list(range(PROMPT)), [0] * PROMPT)
    cur, pos, t = ids[-1], PROMPT, 0.0
    for _ in range(n_tokens):
        t0 = time.perf_counter()
        lg = om.forward([cur], [pos], None)
        t += time.perf_counter() - t0
        cur, pos = int(np.argmax(lg[0])), pos + 1
    om.close()
    return {"value": n_tokens / t, "unit": "tok/s", "cores": 1, "kind": "port", "cpu_model": cpu_model,
            "sample": f"oracle/ec_oracle.c (one thread); same model and prompt; {n_tokens} greedy decode steps"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=248)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cache", default=os.environ.get("EDGECORE_BENCH_DIR", "/tmp/edgecore_bench"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=16)
    ap.add_argument("--no-prefill", action="store_true", help="skip the 4 x 2048-token prefill leg")
    ap.add_argument("--no-gpt2", action="store_true", help="skip the GPT-2 small fp16 leg")
    ap.add_argument("--no-m16", action="store_true", help="skip the Qwen2.5-1.5B M=16 batched-decode leg")
    ap.add_argument("--only", choices=("c4", "c2", "c5"),
                    help="run only this leg beside nothing else (4 x 2048 prefill + M=4 decode, GPT-2 small fp16, "
                         "Qwen2.5-1.5B M=16) and print its JSON: a profiling entry")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="also run the plain copy kernel (ec_device_math op 6) 8 times on this many "
                         "bytes: the reference for HBM traffic counters and achievable bandwidth")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(independent sequences would shard as pure data parallelism: one process per GPU, each with its own model copy and slots)",
              file=sys.stderr)
        return 2

    import numpy as np

    import edgecore_amd as ec

    copy = None
    if args.copy_bytes:
        n = args.copy_bytes // 16 * 4  # floats, a multiple of 4
        src, dst = ec.DeviceBuffer(n * 4), ec.DeviceBuffer(n * 4)
        L0 = ec.lib()
        L0.ec_prof_start(b"copy")
        for _ in range(8):
            if L0.ec_device_math(6, src.ptr, dst.ptr, n):
                raise SystemExit(f"bench.py: copy kernel failed: {ec.last_error()}")
        buf = __import__("ctypes").create_string_buffer(1 << 12)
        L0.ec_prof_stop(buf, len(buf))
        row = json.loads(buf.value.decode())[0]
        copy = {"bytes_per_launch": 8 * n, "avg_us": row["avg_us"], "gbps": round(8 * n / (row["avg_us"] * 1e3), 1)}
        src.close()
        dst.close()

    model, prompt_file = ensure_inputs(Path(args.cache))
    if args.only:
        legs = {"c4": lambda: prefill_c4(ec, np, model, Path(args.cache)),
                "c2": lambda: leg_gpt2_small_fp16(ec, np, Path(args.cache)),
                "c5": lambda: leg_qwen25_15b_int8_m16(ec, np, Path(args.cache))}
        print(json.dumps({"leg": args.only, **legs[args.only]()}))
        return 0
    prompt = ec.read_ids(prompt_file)
    K, W = args.steps, args.warmup
    max_ctx = PROMPT + W + K + 8
    m = ec.Model(model, 1, max_ctx)
    L = ec.lib()

    def prefill():
        m.kv_reset()
        t0 = time.perf_counter()
        _, am = m.forward(prompt, np.arange(PROMPT), np.zeros(PROMPT, np.int32), lm_from=PROMPT - 1,
                          want_logits=False, want_argmax=True)
        return time.perf_counter() - t0

    prefill()  # first call warms code paths
    ttft = prefill()

    def decode_pass(prof_filter):
        """prefill + W warmup steps, then K timed steps; prof_filter: None (no
        events), "" (events on every launch) or a kernel family name"""
        m.kv_reset()
        m.forward(prompt, np.arange(PROMPT), np.zeros(PROMPT, np.int32), lm_from=PROMPT, want_logits=False)
        cur, pos = int(prompt[-1]), PROMPT
        if W > 0:
            cur, pos = int(m.generate_greedy(cur, pos, 0, W)[-1]), pos + W
        L.ec_sync()
        # the same K steps once, untimed: graph capture and instantiation of
        # the steps' buckets happen here (the timed run rewrites the same
        # cache rows with the same values)
        first = [int(x) for x in m.generate_greedy(cur, pos, 0, K)]
        L.ec_sync()
        if prof_filter is not None:
            L.ec_prof_start(prof_filter.encode())
        L.ec_sync()
        t0 = time.perf_counter()
        ids = [int(x) for x in m.generate_greedy(cur, pos, 0, K)]
        L.ec_sync()
        elapsed = time.perf_counter() - t0
        if ids != first:
            raise SystemExit("bench.py: the untimed and timed decode runs produced different tokens")
        kern = []
        if prof_filter is not None:
            buf = __import__("ctypes").create_string_buffer(1 << 16)
            n = L.ec_prof_stop(buf, len(buf))
            kern = json.loads(buf.value.decode()) if n > 0 else []
        return elapsed, kern, ids

    # 1. K steps with every launch recording its own dispatch timestamps
    #    (per-kernel table and the roofline's launch durations)
    elapsed_ev, kernels, ids_ev = decode_pass("")
    # 2. the timed region: the same K steps, nothing but the work
    elapsed, _, ids = decode_pass(None)
    if ids != ids_ev:
        raise SystemExit("bench.py: the two decode passes produced different tokens")
    m.close()

    tot = sum(k["total_us"] for k in kernels) or 1.0
    for k in kernels:
        k["share"] = round(k["total_us"] / tot, 4)
        k["hbm_frac"] = round(k["gbps"] / HBM_PEAK_GBPS, 4)
    dom = max(kernels, key=lambda k: k["total_us"]) if kernels else None
    # the int8-weight GEMVs: inside the persistent decode step (decode_step,
    # all layers), or separate kernels when the step is off (EDGECORE_STEP=0)
    int8 = [k for k in kernels if k["kernel"] in ("gemv_qkv", "gemv_o", "gemv_gateup", "gemv_down")]
    dom_i8 = max(int8, key=lambda k: k["total_us"]) if int8 else None
    lmh = next((k for k in kernels if k["kernel"] == "gemv_lmhead"), None)

    # HBM bytes per launch measured with rocprofv3 counters on this workload
    # (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE of the decode launches,
    # scaled by the copy kernel's counter-to-true-bytes factor)
    traffic = {}
    tpath = REPO / "profiles" / "traffic.json"
    if tpath.exists():
        traffic = json.loads(tpath.read_text()).get("families", {})

    def roof(k):
        if not k:
            return None
        ach = k["bytes_per_launch"] / (k["avg_us"] * 1e3)
        t = traffic.get(k["kernel"], {}).get("hbm_bytes_per_launch")
        return {"kernel": k["kernel"], "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4), "traffic": t,
                "bytes_per_launch": k["bytes_per_launch"], "avg_us": k["avg_us"]}

    # algorithmic bytes of one decode step (weights once + fp16 KV read), mean position
    E, F, kv, V, Lyr = 896, 4864, 128, 151936, 24
    lin = E * E * 2 + 2 * kv * E + 3 * F * E
    mean_pos = PROMPT + W + (K - 1) / 2.0
    step_bytes = Lyr * (lin + 4 * (lin // E) + (mean_pos + 1) * kv * 4) + V * E * 2
    value = K / elapsed
    # the int8 weight stream of the decode GEMVs: int8 weights and row scales
    # of every layer per step, over the time of the kernel(s) that stream them
    # (the persistent step, which also holds the attention; or the separate
    # GEMV kernels)
    i8_bytes = Lyr * (lin + 4 * (lin // E))
    i8_kernels = [k for k in kernels if k["kernel"] == "decode_step"] or int8
    i8_us = sum(k["total_us"] for k in i8_kernels) / K if i8_kernels else 0.0
    i8_stream = None if not i8_us else {
        "kernels": [k["kernel"] for k in i8_kernels], "bytes_per_step": i8_bytes, "us_per_step": round(i8_us, 3),
        "achieved": round(i8_bytes / (i8_us * 1e3), 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
        "frac": round(i8_bytes / (i8_us * 1e3) / HBM_PEAK_GBPS, 4)}
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(elapsed / K * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Qwen2-0.5B-shape int8 bs1 greedy decode after a 256-token prompt",
                   "layers": Lyr, "d_model": E, "heads": 14, "kv_heads": 2, "ffn": F, "vocab": V,
                   "prompt_tokens": PROMPT, "decode_positions": [PROMPT + W, PROMPT + W + K - 1],
                   "batch": 1},
        "roofline": roof(dom),
        "int8_weight_stream": i8_stream,
        "roofline_lm_head": roof(lmh),
        "roofline_int8_gemv": roof(dom_i8),
        "decode_bytes_per_step": int(step_bytes),
        "decode_effective_gbps": round(step_bytes * value / 1e9, 1),
        "ms_per_step_with_kernel_timestamps": round(elapsed_ev / K * 1e3, 4),
        "prefill_tok_s": round(PROMPT / ttft, 1), "ttft_ms": round(ttft * 1e3, 3),
        "copy_kernel": copy,
        "kernels": kernels,
        "kernels_note": "per-launch dispatch start/stop timestamps of every kernel, second pass of the same K steps",
        "device": ec.device_info(),
    }
    if not args.no_prefill:
        out["prefill_4x2048"] = prefill_c4(ec, np, model, Path(args.cache))
    if not args.no_gpt2:
        out["gpt2_small_fp16"] = leg_gpt2_small_fp16(ec, np, Path(args.cache))
    if not args.no_m16:
        out["qwen25_1.5b_int8_m16"] = leg_qwen25_15b_int8_m16(ec, np, Path(args.cache))
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(model, prompt_file, args.cpu_tokens)
        except Exception as e:  # the GPU figure stands on its own
            out["cpu_baseline"] = {"error": str(e)}
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
