"""Pins of the CPU oracle (oracle/ec_oracle.c), independent of the GPU.

Each oracle function is checked against something that would catch a
plausible mistake in it: the host's F16C instruction (exhaustively), closed
forms and invariants, brute force, the golden vectors written by the
reference's own C code (tests/golden/), and -- where the reference build
oracle/_ref exists -- the reference live, bit for bit.
"""
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import edgecore_amd as ec
import oracle

REPO = Path(__file__).resolve().parent.parent
GOLDEN = REPO / "tests" / "golden"


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------- conversions

def test_f32_to_f16_exhaustive_vs_f16c():
    L = oracle.olib()
    if not hasattr(L, "or_check_f16c"):
        pytest.skip("oracle built without F16C")
    assert L.or_check_f16c(0, 0xFFFFFFFF) == 0
    assert L.or_check_f16c_widen() == 0


def _compile_and_run(src: str, tmp_path, *args, extra=()) -> subprocess.CompletedProcess:
    exe = tmp_path / "chk"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fopenmp", "-mf16c",
                    f"-I{REPO / 'include'}", f"-I{REPO / 'edgecore_amd' / 'csrc'}",
                    str(REPO / "tests" / "c" / src), *[str(REPO / e) for e in extra], "-o", str(exe), "-lm"],
                   check=True)
    return subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True)


def test_bf16_packers_exhaustive(tmp_path):
    """edgecore/ecm.py:27-41 restated twice (the generator's ec_f32_to_bf16 and
    the oracle's or_f32_to_bf16) against round-to-nearest-even written as a
    distance comparison, on all 2^32 inputs."""
    p = _compile_and_run("bf16_exhaustive.c", tmp_path,
                         extra=("edgecore_amd/csrc/ecm.c", "oracle/ec_oracle.c"))
    assert p.returncode == 0 and "mismatches 0, or_f32_to_bf16 mismatches 0" in p.stdout, p.stdout


def test_library_header_f16_exhaustive(tmp_path):
    """include/edgecore.h's host conversions (used by the generator) vs F16C."""
    p = _compile_and_run("f16_header_check.c", tmp_path)
    assert p.returncode == 0, p.stdout + p.stderr


def test_device_expf_source_exhaustive(tmp_path):
    """edgecore_amd/csrc/ec_expf.h (the kernels' expf) vs the host libm on all 2^32 inputs."""
    p = _compile_and_run("expf_exhaustive.c", tmp_path)
    assert p.returncode == 0 and "mismatches 0" in p.stdout, p.stdout


def test_reciprocal_quantizer_equals_division(tmp_path):
    """edgecore_amd/csrc/ec_quant.h: the kernels' division-free activation
    quantizer (reciprocal + Markstein correction) gives the reference's
    rint(a / s) code, and the same quotient, around every half-integer."""
    p = _compile_and_run("quant_rcp_check.c", tmp_path)
    assert p.returncode == 0 and "ec_quant1_rcp == ec_quant1" in p.stdout, p.stdout


# ---------------------------------------------------------------- quantizers

@pytest.mark.parametrize("packer", ["oracle", "library"])
def test_weight_packer_closed_forms(packer):
    pack = oracle.quantize_int8_symmetric if packer == "oracle" else ec.quantize_int8_symmetric
    w = np.zeros((4, 8), np.float32)
    w[1] = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -127]     # scale exactly 1.0: ties to even
    w[2] = [1, 0, 0, 0, 0, 0, 0, -1]                          # scale 1/127 stored as float32
    w[3] = [0.3, -0.7, 0.1, 0.0, 0.69999, -0.25, 0.7, 0.05]   # max |w| element -> +-127
    q, s = pack(w)
    assert s[0] == 1.0 and not q[0].any()                     # zero row: scale 1, codes 0
    assert list(q[1]) == [127, 0, 2, 2, 0, -2, -2, -127] and s[1] == 1.0
    assert s[2] == np.float32(1.0 / 127.0) and q[2, 0] == 127 and q[2, 7] == -127
    assert q[3, 1] == -127 and q[3, 6] == 127 and s[3] == np.float32(0.7 / 127.0)


def _packer_golden():
    return np.load(GOLDEN / "packer.npz")


@pytest.mark.parametrize("packer", ["oracle", "library"])
def test_weight_packer_golden(packer):
    """edgecore/ecm.py:50-59 on tests/golden/packer.npz, whose codes and scales
    come from exact rational arithmetic on the float64 definition
    (make_packer_golden.py): adversarial near-half-integer quotients, ties,
    +-maxabs, zero / NaN / infinite / subnormal rows, seeded N(0, 0.02) rows."""
    pack = oracle.quantize_int8_symmetric if packer == "oracle" else ec.quantize_int8_symmetric
    g = _packer_golden()
    q, s = pack(g["w"])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(s.view(np.uint32), g["s"].view(np.uint32)) or np.array_equal(
        np.isnan(s), np.isnan(g["s"])) and np.array_equal(s[~np.isnan(s)], g["s"][~np.isnan(g["s"])])


def test_weight_packer_golden_catches_mistakes():
    """The fixture tells the float64 packer from plausible wrong ones: float32
    arithmetic throughout, dividing by the float32-rounded scale, and
    multiplying by 127 / maxabs each give other codes on its adversarial rows."""
    g = _packer_golden()
    w, want = g["w"][: int(g["n_adversarial"])], g["q"][: int(g["n_adversarial"])]

    def f32(w):
        m = np.max(np.abs(w), axis=1).astype(np.float32)
        s = m / np.float32(127.0)
        return np.clip(np.rint(w / s[:, None]), -128, 127).astype(np.int8)

    def f32_scale(w):
        s = np.max(np.abs(w.astype(np.float64)), axis=1) / 127.0
        return np.clip(np.rint(w.astype(np.float64) / s.astype(np.float32).astype(np.float64)[:, None]),
                       -128, 127).astype(np.int8)

    def recip(w):
        r = 127.0 / np.max(np.abs(w.astype(np.float64)), axis=1)
        return np.clip(np.rint(w.astype(np.float64) * r[:, None]), -128, 127).astype(np.int8)

    for wrong in (f32, f32_scale, recip):
        assert not np.array_equal(wrong(w), want), wrong.__name__


def test_weight_packer_library_equals_oracle():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (64, 896)).astype(np.float32)
    w[3] *= 0
    qa, sa = ec.quantize_int8_symmetric(w)
    qb, sb = oracle.quantize_int8_symmetric(w)
    assert np.array_equal(qa, qb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))


def test_activation_quantizer_closed_forms():
    x = np.zeros((3, 8), np.float32)
    x[0] = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -127]
    x[2] = [1, -1, 0.5, 0.25, 0, 0, 0, 0]
    q, s = oracle.quantize_rows(x)
    assert list(q[0]) == [127, 0, 2, 2, 0, -2, -2, -127] and s[0] == 1.0
    assert s[1] == 1.0 and not q[1].any()
    assert s[2] == np.float32(np.float32(1.0) / np.float32(127.0)) and q[2, 0] == 127 and q[2, 1] == -127


# ---------------------------------------------------------------- GEMMs

def test_gemm_int8_bruteforce():
    rng = np.random.default_rng(1)
    for M, K, N in [(3, 4864, 7), (2, 37, 5), (1, 896, 64)]:
        A = rng.integers(-128, 128, (M, K)).astype(np.int8)
        B = rng.integers(-128, 128, (N, K)).astype(np.int8)
        A[0, :] = -128
        B[0, :] = -128
        a_s = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
        b_s = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
        C = oracle.gemm_int8(A, a_s, B, b_s, None)
        dots = A.astype(np.int64) @ B.astype(np.int64).T
        assert dots[0, 0] == 128 * 128 * K
        want = (dots.astype(np.float32) * a_s[:, None]) * b_s[None, :]
        assert np.array_equal(C.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_w16_within_fp32_bound(bf16):
    rng = np.random.default_rng(2)
    M, K, N = 3, 901, 17
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    if bf16:
        u = W.view(np.uint32).astype(np.uint64)
        B = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        Bf = (B.astype(np.uint32) << 16).view(np.float32)
    else:
        B = W.astype(np.float16).view(np.uint16)
        Bf = B.view(np.float16).astype(np.float32)
    C = oracle.gemm_w16(A, B, bf16)
    exact = A.astype(np.float64) @ Bf.astype(np.float64).T
    bound = 2 * K * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(Bf).astype(np.float64).T)
    assert np.all(np.abs(C - exact) <= bound)


def test_gemm_golden_vectors_from_reference():
    g = np.load(GOLDEN / "kernels.npz")
    n_i8 = len({k.split("_")[1] for k in g.files if k.startswith("i8_")})
    for i in range(n_i8):
        C = oracle.gemm_int8(g[f"i8_{i}_A"], g[f"i8_{i}_as"], g[f"i8_{i}_B"],
                             g[f"i8_{i}_bs"] if f"i8_{i}_bs" in g.files else None,
                             g[f"i8_{i}_bias"] if f"i8_{i}_bias" in g.files else None)
        assert np.array_equal(C.view(np.uint32), g[f"i8_{i}_C"].view(np.uint32)), i
    for kind, bf in (("f16", False), ("bf16", True)):
        i = 0
        while f"{kind}_{i}_A" in g.files:
            C = oracle.gemm_w16(g[f"{kind}_{i}_A"], g[f"{kind}_{i}_B"], bf)
            assert np.array_equal(C.view(np.uint32), g[f"{kind}_{i}_C"].view(np.uint32)), (kind, i)
            i += 1


# ---------------------------------------------------------------- row ops

def _rms(x, g, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    oracle.olib().or_rmsnorm_rows(out.ctypes.data, x.ctypes.data, np.ascontiguousarray(g, np.float32).ctypes.data,
                                  x.shape[0], x.shape[1], eps)
    return out


def _ln(x, g, b, eps):
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(g, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(x)
    oracle.olib().or_layernorm_rows(out.ctypes.data, x.ctypes.data, g.ctypes.data, b.ctypes.data,
                                    x.shape[0], x.shape[1], eps)
    return out


def test_norm_invariants():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (4, 896)).astype(np.float32)
    g = np.ones(896, np.float32)
    # scaling by a power of two is exact in every step when eps = 0
    assert np.array_equal(_rms(x, g, 0.0), _rms(x * 8, g, 0.0))
    assert np.array_equal(_ln(x, g, 0 * g, 0.0), _ln(x * 0.25, g, 0 * g, 0.0))
    # gamma enters as one exact multiply (doubling), beta as one add
    assert np.array_equal(_rms(x, 2 * g, 1e-6), 2 * _rms(x, g, 1e-6))
    # a constant row normalizes to beta exactly
    c = np.full((1, 64), 3.25, np.float32)
    beta = rng.normal(0, 1, 64).astype(np.float32)
    assert np.array_equal(_ln(c, np.ones(64, np.float32), beta, 1e-5)[0], beta)
    # rms of a row of ones is 1/sqrt(1 + eps) in double, rounded once
    assert _rms(np.ones((1, 16), np.float32), np.ones(16, np.float32), 0.0)[0, 0] == 1.0


def test_rope_inverse_frequencies():
    import ctypes as C
    f = np.zeros(32, np.float64)
    oracle.olib().or_rope_inv_freq(f.ctypes.data, 32, 1e6, 0, 1.0, 32768.0)
    assert f[0] == 1.0                        # pos * inv_freq[0] = pos: pins the layout
    assert abs(f[16] - 1e6 ** -0.5) < 1e-15   # theta^(-2i/dim) at i = dim/4
    assert np.all(np.diff(f) < 0)
    y = np.zeros(32, np.float64)
    oracle.olib().or_rope_inv_freq(y.ctypes.data, 32, 1e6, 1, 1.0, 32768.0)
    assert np.allclose(f, y, rtol=1e-15, atol=0)  # YaRN with factor 1: f*ramp + f*(1-ramp) ~ f
    oracle.olib().or_rope_inv_freq(y.ctypes.data, 32, 1e6, 1, 4.0, 32768.0)
    assert y[0] == f[0] and abs(y[-1] - f[-1] / 4) < 1e-20   # high-frequency kept, low interpolated
    del C


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def test_attention_rows_closed_forms():
    """or_attention_rows (the forward's per-row attention over given caches):
    a single position returns its V row exactly (pins the slot and KV-head
    mapping, h * KVH / H); positions outside [lo, pos] are never read (NaN
    there stays out); random rows agree with a float64 softmax attention
    within float rounding (pins the 1/sqrt(hd) scale and the operand roles)."""
    rng = np.random.default_rng(11)
    H, KVH, hd, C, ns = 6, 2, 16, 40, 3
    kv = KVH * hd
    kc = _f16(rng.normal(0, 1, (ns, C, kv)))
    vc = _f16(rng.normal(0, 1, (ns, C, kv)))
    q = rng.normal(0, 1, (ns, H * hd)).astype(np.float32)
    out = oracle.attention_rows(q, kc, vc, np.zeros(ns), np.arange(ns), H, KVH)
    vf = vc.view(np.float16).astype(np.float32)
    for m in range(ns):
        for h in range(H):
            g = h * KVH // H
            assert np.array_equal(out[m, h * hd:(h + 1) * hd], vf[m, 0, g * hd:(g + 1) * hd])
    # causality and the sliding window: NaN outside [pos - window + 1, pos]
    pos = np.array([5, 20, 39], np.int32)
    for window in (0, 4):
        k2, v2 = kc.copy(), vc.copy()
        for m, p in enumerate(pos):
            lo = max(0, p - window + 1) if window else 0
            k2[m, :lo] = k2[m, p + 1:] = v2[m, :lo] = v2[m, p + 1:] = 0x7e00
        o2 = oracle.attention_rows(q, k2, v2, pos, np.arange(ns), H, KVH, window=window)
        assert np.isfinite(o2).all()
        kf, vf2 = k2.view(np.float16).astype(np.float64), v2.view(np.float16).astype(np.float64)
        for m, p in enumerate(pos):
            lo = max(0, p - window + 1) if window else 0
            for h in range(H):
                g = h * KVH // H
                K = kf[m, lo:p + 1, g * hd:(g + 1) * hd]
                V = vf2[m, lo:p + 1, g * hd:(g + 1) * hd]
                s = K @ q[m, h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
                w = np.exp(s - s.max())
                want = (w / w.sum()) @ V
                np.testing.assert_allclose(o2[m, h * hd:(h + 1) * hd], want, rtol=1e-4, atol=1e-5)
    # only the listed rows are computed
    part = oracle.attention_rows(q, kc, vc, pos, np.arange(ns), H, KVH, rows=[1])
    assert np.isnan(part[0]).all() and np.isfinite(part[1]).all()


def test_forward_from_equals_full_rows(make_model):
    """or_forward_from (LM head from row lm_from on) = the full forward's rows,
    and leaves the same KV cache (the next step's logits agree)."""
    path = make_model("tiny-qwen2-int8")
    a, b = oracle.OracleModel(path, 1, 32), oracle.OracleModel(path, 1, 32)
    toks = [3, 14, 15, 92, 65, 35]
    full = a.forward(toks, np.arange(6), np.zeros(6, np.int32))
    part = b.forward(toks, np.arange(6), np.zeros(6, np.int32), lm_from=4)
    assert np.array_equal(full[4:], part)
    assert b.forward(toks, np.arange(6), np.zeros(6, np.int32), lm_from=6).shape == (0, a.vocab)
    assert np.array_equal(a.forward([7], [6], [0]), b.forward([7], [6], [0]))
    a.close()
    b.close()


def test_elementwise_map_matches_scalars():
    x = np.array([-3.0, -0.5, 0.0, 0.75, 5.0], np.float32)
    L = oracle.olib()
    assert np.array_equal(oracle.map_op(1, x), np.array([L.or_silu(float(v)) for v in x], np.float32))
    assert np.array_equal(oracle.map_op(2, x), np.array([L.or_gelu_new(float(v)) for v in x], np.float32))


# ---------------------------------------------------------------- end to end

def _golden():
    return json.loads((GOLDEN / "models.json").read_text())


@pytest.mark.parametrize("name", ["tiny-gpt2-int8", "tiny-gpt2-fp16", "tiny-qwen2-int8", "tiny-qwen2-bf16"])
def test_oracle_reproduces_reference_golden(name, tmp_path):
    g = _golden()[name]
    path = tmp_path / f"{name}.ecm"
    ec.synth(path, name=name, **g["synth"])
    assert _sha(np.fromfile(path, np.uint8)) == g["file_sha256"], "generator output changed"
    om = oracle.OracleModel(path, 1, g["max_ctx"])
    prompt = np.array(g["prompt"], np.int32)
    ids, steps = om.generate(prompt, 32, want_logits=True)
    assert [int(x) for x in ids[len(prompt):]] == g["ids"]
    assert [_sha(r) for r in steps] == g["step_logits_sha256"]
    om.kv_reset()
    n = len(prompt)
    pre = om.forward(prompt, np.arange(n), np.zeros(n, np.int32))
    assert _sha(pre) == g["prefill_logits_sha256"]


@pytest.mark.slow
def test_oracle_reproduces_reference_golden_qwen2_05b(tmp_path):
    g = _golden()["qwen2-0.5b-int8"]
    path = tmp_path / "c3.ecm"
    ec.synth(path, name="qwen2-0.5b-int8", **g["synth"])
    om = oracle.OracleModel(path, 1, g["max_ctx"])
    prompt = np.array(g["prompt"], np.int32)
    ids, steps = om.generate(prompt, 32, want_logits=True)
    assert [int(x) for x in ids[len(prompt):]] == g["ids"]
    assert [_sha(r) for r in steps] == g["step_logits_sha256"]


@pytest.mark.skipif(not oracle.ref_available(), reason="reference build oracle/_ref absent")
@pytest.mark.parametrize("spec", [dict(preset="tiny-qwen2", tie=1, vocab=3000),
                                  dict(arch="qwen2", layers=2, embd=96, heads=6, kv_heads=2, ffn=160, ctx=96,
                                       vocab=700, precision="fp16"),
                                  dict(arch="gpt2", layers=3, embd=48, heads=3, ctx=80, vocab=300,
                                       precision="int8"),
                                  # sliding window 16 (positions reach 31) and YaRN RoPE
                                  dict(arch="qwen2", layers=2, embd=128, heads=4, kv_heads=2, ffn=192, ctx=96,
                                       vocab=600, precision="int8", sliding_window=16, rope_type="yarn",
                                       yarn_factor=4.0, yarn_orig_max=24, yarn_attention_factor=1.1)])
def test_oracle_equals_reference_live(spec, tmp_path):
    path = tmp_path / "m.ecm"
    ec.synth(path, name="m", **spec)
    rm = oracle.RefModel(path, 2, 64)
    om = oracle.OracleModel(path, 2, 64)
    prompt = np.arange(5, 17, dtype=np.int32) % rm.vocab
    a = rm.generate(prompt, 20, want_logits=True)
    b = om.generate(prompt, 20, want_logits=True)
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    # batched decode through two slots
    rm.kv_reset()
    om.kv_reset()
    for slot in (0, 1):
        rm.forward(prompt, np.arange(12), np.full(12, slot, np.int32))
        om.forward(prompt, np.arange(12), np.full(12, slot, np.int32))
    x = rm.forward([3, 4], [12, 12], None)
    y = om.forward([3, 4], [12, 12], None)
    assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
