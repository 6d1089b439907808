"""EdgeCore on MI355X: Python access to the C ABI of libedgecore_hip.so.

The product is native: ``lib/libedgecore_hip.so`` (HIP kernels for gfx950 and
the C host runtime behind ``include/edgecore.h``), ``bin/edgecore-runtime``
(the command-line driver with the reference's CLI contract) and
``bin/ecm_synth`` (seeded synthetic model generator).  This module only binds
them with ctypes so that tests and the benchmark can call the same entry
points a C host calls.  There is no fallback: if the library has not been
built, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
LIB_PATH = PKG_DIR / "lib" / "libedgecore_hip.so"
RUNTIME = PKG_DIR / "bin" / "edgecore-runtime"
SYNTH = PKG_DIR / "bin" / "ecm_synth"
HEADER = REPO_DIR / "include" / "edgecore.h"

__all__ = [
    "EdgeCoreError", "lib", "GPT2", "Model", "gemm_int8", "gemm_fp16_fp32",
    "gemm_bf16_fp32", "quantize_int8_symmetric", "synth", "sample_full", "sample_candidates", "topk_dev", "PKG_DIR", "LIB_PATH",
    "RUNTIME", "SYNTH", "HEADER",
]


class EdgeCoreError(RuntimeError):
    """A failing call into libedgecore_hip.so (message from ec_last_error)."""


class Tokenizer(C.Structure):
    _fields_ = [
        ("id_to_token", C.c_void_p), ("byte_to_id", C.c_void_p), ("cp_to_byte", C.c_void_p),
        ("merge_l", C.c_void_p), ("merge_r", C.c_void_p), ("merge_m", C.c_void_p),
        ("n_merges", C.c_int), ("vocab_size", C.c_int), ("variant", C.c_int), ("eos_id", C.c_int),
        ("sp_tok", C.c_void_p), ("sp_len", C.c_void_p), ("sp_id", C.c_void_p), ("n_sp", C.c_int),
    ]


class GPT2(C.Structure):
    """Mirror of ``GPT2`` in include/edgecore.h (pointer fields are device pointers)."""

    _fields_ = [
        ("model_name", C.c_char * 64),
        ("n_layer", C.c_int), ("n_head", C.c_int), ("n_embd", C.c_int), ("n_ctx", C.c_int),
        ("vocab", C.c_int), ("n_kv_head", C.c_int), ("n_kv_embd", C.c_int),
        ("intermediate", C.c_int), ("head_dim", C.c_int), ("arch", C.c_int),
        ("n_params", C.c_size_t), ("eps", C.c_double),
        ("rope_theta", C.c_double), ("rope_type", C.c_int),
        ("yarn_factor", C.c_double), ("yarn_orig_max", C.c_double),
        ("yarn_attention_factor", C.c_double),
        ("sliding_window", C.c_int), ("tie_word_embeddings", C.c_int), ("eos_token_id", C.c_int),
        ("wte", C.c_void_p), ("wpe", C.c_void_p), ("lw", C.c_void_p),
        ("lnf_g", C.c_void_p), ("lnf_b", C.c_void_p), ("lm_head", C.c_void_p),
        ("precision", C.c_int),
        ("k_cache", C.c_void_p), ("v_cache", C.c_void_p),
        ("batch_cap", C.c_int), ("max_ctx", C.c_int),
        ("ws_x", C.c_void_p), ("ws_tmp", C.c_void_p), ("ws_qkv", C.c_void_p),
        ("ws_attn", C.c_void_p), ("ws_scores", C.c_void_p),
        ("ws_q", C.c_void_p), ("ws_qs", C.c_void_p), ("ws_q_cols", C.c_size_t),
        ("tok", Tokenizer),
        ("file_data", C.c_void_p), ("file_size", C.c_size_t), ("file_mapped", C.c_int),
    ]


_LIB: Optional[C.CDLL] = None

_P = C.c_void_p
_I = C.c_int
_SIG = {
    "gemm_fp16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
    "gemm_bf16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
    "gemm_int8": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "ec_gemm_fp16_fp32_dev": (_I, [_P, _P, _P, _I, _I, _I]),
    "ec_gemm_bf16_fp32_dev": (_I, [_P, _P, _P, _I, _I, _I]),
    "ec_gemm_int8_dev": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "ec_gemm_int8_epi_dev": (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "ec_gemm_w16_epi_dev": (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I]),
    "ec_quantize_rows_dev": (_I, [_P, _I, _I, _P, _P]),
    "gpt2_load": (_I, [_P, C.c_char_p, _I, _I]),
    "gpt2_free": (None, [_P]),
    "gpt2_forward": (None, [_P, _P, _P, _P, _I, _P]),
    "qwen2_forward": (None, [_P, _P, _P, _P, _I, _P]),
    "gpt2_forward_ex": (_I, [_P, _P, _P, _P, _I, _I, _P, _P]),
    "gpt2_forward_topk": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _P, _P]),
    "ec_topk_max": (_I, []),
    "ec_generate_greedy": (_I, [_P, _I, _I, _I, _I, _P]),
    "ec_generate_greedy_timed": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "ec_last_logits": (_I, [_P, _I, _P]),
    "ec_topk_dev": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "ec_topk_dev_noalloc": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "ec_attention_dev": (_I, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _I, _P, _I, _I]),
    "ec_rng_next": (C.c_uint, [C.POINTER(C.c_ulonglong)]),
    "ec_sample_full": (_I, [_P, _I, C.c_float, _I, C.POINTER(C.c_ulonglong)]),
    "ec_sample_candidates": (_I, [_P, _P, _I, _I, C.c_float, _I, C.POINTER(C.c_ulonglong)]),
    "gpt2_kv_reset": (_I, [_P]),
    "ecm_parse": (_I, [_P, C.c_size_t, _P, _I, _P]),
    "ec_last_error": (C.c_char_p, []),
    "ec_init": (_I, []),
    "ec_release": (_I, []),
    "ec_alloc_count": (C.c_long, []),
    "ec_device_info": (_I, [C.c_char_p, _I]),
    "ec_stream": (_P, []),
    "ec_sync": (_I, []),
    "ec_dev_alloc": (_P, [C.c_size_t]),
    "ec_dev_free": (_I, [_P]),
    "ec_memcpy_h2d": (_I, [_P, _P, C.c_size_t]),
    "ec_memcpy_d2h": (_I, [_P, _P, C.c_size_t]),
    "ec_memset_dev": (_I, [_P, _I, C.c_size_t]),
    "ec_prof_start": (_I, [C.c_char_p]),
    "ec_prof_stop": (_I, [C.c_char_p, _I]),
    "ec_quantize_int8_symmetric": (None, [_P, _I, _I, _P, _P]),
    "ec_gpt2_sizeof": (C.c_size_t, []),
    "ec_device_math": (_I, [_I, _P, _P, C.c_size_t]),
    "tokenizer_encode": (_I, [_P, C.c_char_p, _P, _I]),
    "tokenizer_load": (_I, [_P, C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, _I, _I]),
    "tokenizer_free": (None, [_P]),
    "tokenizer_decode": (_P, [_P, _P, _I]),
    "now_sec": (C.c_double, []),
    "peak_rss_gb": (C.c_float, []),
}


def lib() -> C.CDLL:
    """Load libedgecore_hip.so (built in-tree by ``make``); raise if it is missing."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise EdgeCoreError(f"{LIB_PATH} is not built; run `make` (or __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def last_error() -> str:
    return (lib().ec_last_error() or b"").decode(errors="replace")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise EdgeCoreError(f"{what} failed ({rc}): {last_error()}")


def device_info() -> dict:
    import json
    buf = C.create_string_buffer(1024)
    n = lib().ec_device_info(buf, len(buf))
    if n < 0:
        raise EdgeCoreError(f"ec_device_info failed: {last_error()}")
    return json.loads(buf.value.decode())


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


# ---------------------------------------------------------------------------
# kernel ABI (host pointers, like the reference src/kernels.c)
# ---------------------------------------------------------------------------

def gemm_int8(A: np.ndarray, a_scale: np.ndarray, B: np.ndarray,
              b_scale: Optional[np.ndarray] = None, bias: Optional[np.ndarray] = None) -> np.ndarray:
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    a_scale = np.ascontiguousarray(a_scale, np.float32)
    b_scale = None if b_scale is None else np.ascontiguousarray(b_scale, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    M, K = A.shape
    N = B.shape[0]
    assert B.shape[1] == K and a_scale.shape == (M,)
    Cm = np.empty((M, N), np.float32)
    lib().gemm_int8(_ptr(Cm), _ptr(A), _ptr(a_scale), _ptr(B), _ptr(b_scale), _ptr(bias), M, K, N)
    return Cm


def _gemm_w16(fn, A: np.ndarray, B: np.ndarray) -> np.ndarray:
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.uint16)
    M, K = A.shape
    N = B.shape[0]
    assert B.shape[1] == K
    Cm = np.empty((M, N), np.float32)
    fn(_ptr(Cm), _ptr(A), _ptr(B), M, K, N)
    return Cm


def gemm_fp16_fp32(A: np.ndarray, B_fp16_bits: np.ndarray) -> np.ndarray:
    return _gemm_w16(lib().gemm_fp16_fp32, A, B_fp16_bits)


def gemm_bf16_fp32(A: np.ndarray, B_bf16_bits: np.ndarray) -> np.ndarray:
    return _gemm_w16(lib().gemm_bf16_fp32, A, B_bf16_bits)


def quantize_int8_symmetric(w: np.ndarray):
    """The library's weight packer (edgecore/ecm.py:50-59 semantics)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().ec_quantize_int8_symmetric(_ptr(w), rows, cols, _ptr(q), _ptr(s))
    return q, s


def gemm_w16_epi(wt: int, epi: int, bm: int, A: np.ndarray, B: np.ndarray, B2: Optional[np.ndarray] = None,
                 bias: Optional[np.ndarray] = None, C0: Optional[np.ndarray] = None) -> np.ndarray:
    """ec_gemm_w16_epi_dev on host arrays copied to the device: the 16-bit
    weight matrix-core GEMM (wt 1 fp16, 2 bf16; B and B2 as uint16 bit
    patterns) with epilogue epi (0 store, 1 residual onto C0, 2 GELU, 3 SwiGLU
    with B2, 4-6 the same with bias) and row tile bm (0 = the library's
    choice)."""
    M, K = A.shape
    N = B.shape[0]
    arrs = [np.ascontiguousarray(A, np.float32), np.ascontiguousarray(B, np.uint16)]
    opt = [None if B2 is None else np.ascontiguousarray(B2, np.uint16),
           None if bias is None else np.ascontiguousarray(bias, np.float32)]
    c0 = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    bufs = [DeviceBuffer.from_array(x) for x in arrs]
    obufs = [None if x is None else DeviceBuffer.from_array(x) for x in opt]
    cb = DeviceBuffer.from_array(c0)
    try:
        p = [b.ptr for b in bufs] + [None if b is None else b.ptr for b in obufs]
        _check(lib().ec_gemm_w16_epi_dev(int(wt), int(epi), int(bm), cb.ptr, p[0], p[1], p[2], p[3], M, K, N),
               "ec_gemm_w16_epi_dev")
        _check(lib().ec_sync(), "ec_sync")
        return cb.to_array(np.float32, (M, N))
    finally:
        for b in bufs + [x for x in obufs if x is not None] + [cb]:
            b.close()


def gemm_int8_epi(epi: int, bm: int, A: np.ndarray, a_scale: np.ndarray, B: np.ndarray,
                  b_scale: Optional[np.ndarray] = None, B2: Optional[np.ndarray] = None,
                  b2_scale: Optional[np.ndarray] = None, bias: Optional[np.ndarray] = None,
                  C0: Optional[np.ndarray] = None) -> np.ndarray:
    """ec_gemm_int8_epi_dev on host arrays copied to the device: the int8
    matrix-core GEMM with epilogue epi (0 store, 1 residual onto C0, 2 GELU,
    3 SwiGLU with B2) and row tile bm (0 = the library's choice)."""
    M, K = A.shape
    N = B.shape[0]
    arrs = [np.ascontiguousarray(A, np.int8), np.ascontiguousarray(a_scale, np.float32),
            np.ascontiguousarray(B, np.int8)]
    opt = [b_scale, B2, b2_scale, bias]
    opt = [None if x is None else np.ascontiguousarray(x, np.int8 if i == 1 else np.float32)
           for i, x in enumerate(opt)]
    c0 = np.zeros((M, N), np.float32) if C0 is None else np.ascontiguousarray(C0, np.float32)
    bufs = [DeviceBuffer.from_array(x) for x in arrs]
    obufs = [None if x is None else DeviceBuffer.from_array(x) for x in opt]
    cb = DeviceBuffer.from_array(c0)
    try:
        p = [b.ptr for b in bufs] + [None if b is None else b.ptr for b in obufs]
        _check(lib().ec_gemm_int8_epi_dev(int(epi), int(bm), cb.ptr, p[0], p[1], p[2], p[3], p[4], p[5], p[6],
                                          M, K, N), "ec_gemm_int8_epi_dev")
        _check(lib().ec_sync(), "ec_sync")
        return cb.to_array(np.float32, (M, N))
    finally:
        for b in bufs + [x for x in obufs if x is not None] + [cb]:
            b.close()


class DeviceBuffer:
    """A device allocation from ec_dev_alloc, freed on close()."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = lib().ec_dev_alloc(self.nbytes)
        if not self.ptr:
            raise EdgeCoreError(f"ec_dev_alloc({nbytes}) failed: {last_error()}")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 1))
        if a.nbytes:
            _check(lib().ec_memcpy_h2d(b.ptr, _ptr(a), a.nbytes), "ec_memcpy_h2d")
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        _check(lib().ec_memcpy_d2h(_ptr(out), self.ptr, out.nbytes), "ec_memcpy_d2h")
        return out

    def close(self) -> None:
        if self.ptr:
            lib().ec_dev_free(self.ptr)
            self.ptr = None


# ---------------------------------------------------------------------------
# model
# ---------------------------------------------------------------------------

class Model:
    """A model loaded by gpt2_load (weights, KV cache and workspaces in HBM)."""

    def __init__(self, path: str | os.PathLike, batch_cap: int = 1, max_ctx: int = 0):
        L = lib()
        if C.sizeof(GPT2) != L.ec_gpt2_sizeof():
            raise EdgeCoreError("GPT2 ctypes mirror does not match the library")
        self.g = GPT2()
        rc = L.gpt2_load(C.byref(self.g), str(path).encode(), int(batch_cap), int(max_ctx))
        if rc != 0:
            raise EdgeCoreError(f"gpt2_load({path}) failed: {last_error()}")
        self._open = True

    @property
    def vocab(self) -> int:
        return self.g.vocab

    @property
    def eff_ctx(self) -> int:
        g = self.g
        return g.max_ctx if 0 < g.max_ctx < g.n_ctx else g.n_ctx

    @property
    def precision(self) -> int:
        return self.g.precision

    def kv_reset(self) -> None:
        _check(lib().gpt2_kv_reset(C.byref(self.g)), "gpt2_kv_reset")

    def forward(self, tokens: Sequence[int], positions: Sequence[int],
                seqs: Optional[Sequence[int]] = None, lm_from: int = 0,
                want_logits: bool = True, want_argmax: bool = False):
        """gpt2_forward_ex; returns (logits [M - lm_from, V] or None, argmax or None)."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(positions, np.int32)
        s = None if seqs is None else np.ascontiguousarray(seqs, np.int32)
        M = len(t)
        rows = M - lm_from
        lg = np.empty((rows, self.vocab), np.float32) if want_logits and rows > 0 else None
        am = np.empty(rows, np.int32) if want_argmax and rows > 0 else None
        rc = lib().gpt2_forward_ex(C.byref(self.g), _ptr(t), _ptr(p), _ptr(s), M, lm_from,
                                   _ptr(lg), _ptr(am))
        _check(rc, "gpt2_forward_ex")
        return lg, am

    def forward_topk(self, tokens: Sequence[int], positions: Sequence[int],
                     seqs: Optional[Sequence[int]] = None, lm_from: int = 0, top_k: int = 40):
        """gpt2_forward_topk; returns (vals, idx [M - lm_from, top_k + 1], status [M - lm_from])."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(positions, np.int32)
        s = None if seqs is None else np.ascontiguousarray(seqs, np.int32)
        M = len(t)
        rows = M - lm_from
        vals = np.empty((rows, top_k + 1), np.float32)
        idx = np.empty((rows, top_k + 1), np.int32)
        status = np.empty(rows, np.int32)
        rc = lib().gpt2_forward_topk(C.byref(self.g), _ptr(t), _ptr(p), _ptr(s), M, lm_from, top_k,
                                     _ptr(vals), _ptr(idx), _ptr(status))
        _check(rc, "gpt2_forward_topk")
        return vals, idx, status

    def generate_greedy(self, token: int, pos: int, slot: int, n: int) -> np.ndarray:
        """ec_generate_greedy: the ids of n greedy steps from `token` at `pos` in `slot`."""
        out = np.empty(n, np.int32)
        _check(lib().ec_generate_greedy(C.byref(self.g), int(token), int(pos), int(slot), int(n), _ptr(out)),
               "ec_generate_greedy")
        return out

    def generate_greedy_timed(self, token: int, pos: int, slot: int, n: int):
        """ec_generate_greedy_timed: (ids, per-step ms) of n greedy steps."""
        out = np.empty(n, np.int32)
        ms = np.empty(n, np.float64)
        _check(lib().ec_generate_greedy_timed(C.byref(self.g), int(token), int(pos), int(slot), int(n), _ptr(out),
                                              _ptr(ms)), "ec_generate_greedy_timed")
        return out, ms

    def last_logits(self, row: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        _check(lib().ec_last_logits(C.byref(self.g), row, _ptr(out)), "ec_last_logits")
        return out

    def generate(self, prompt: Sequence[int], n_gen: int, want_logits: bool = False):
        """gen_and_measure at batch 1, greedy (src/runtime_main.c:293-362):
        returns (ids, [n_gen, V] step logits or None)."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        n = len(prompt)
        self.kv_reset()
        self.forward(prompt, np.arange(n), np.zeros(n, np.int32), lm_from=n,
                     want_logits=False)
        ids = list(int(x) for x in prompt)
        cur, pos = int(prompt[-1]), n
        steps = []
        for _ in range(n_gen):
            lg, am = self.forward([cur], [pos], None, want_logits=want_logits, want_argmax=True)
            if want_logits:
                steps.append(lg[0])
            cur = int(am[0])
            ids.append(cur)
            pos += 1
        return np.array(ids, np.int32), (np.stack(steps) if want_logits else None)

    def close(self) -> None:
        if getattr(self, "_open", False):
            lib().gpt2_free(C.byref(self.g))
            self._open = False

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# sampling (src/runtime_main.c:205-248)
# ---------------------------------------------------------------------------

def sample_full(logits: np.ndarray, temp: float, top_k: int, state: int) -> tuple[int, int]:
    """ec_sample_full on one row; returns (token, new LCG state)."""
    row = np.ascontiguousarray(logits, np.float32)
    st = C.c_ulonglong(state)
    tok = lib().ec_sample_full(_ptr(row), len(row), temp, top_k, C.byref(st))
    return tok, st.value


def sample_candidates(vals: np.ndarray, idx: np.ndarray, vocab: int, temp: float, top_k: int,
                      state: int) -> tuple[int, int]:
    """ec_sample_candidates on a row's top_k + 1 candidates; returns (token, new state)."""
    v = np.ascontiguousarray(vals, np.float32)
    i = np.ascontiguousarray(idx, np.int32)
    st = C.c_ulonglong(state)
    tok = lib().ec_sample_candidates(_ptr(v), _ptr(i), len(v), vocab, temp, top_k, C.byref(st))
    return tok, st.value


def topk_dev(logits: np.ndarray, top_k: int):
    """ec_topk_dev on host rows (copied to the device): (vals, idx, status)."""
    L = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    rows, V = L.shape
    buf = DeviceBuffer.from_array(L)
    try:
        vals = np.empty((rows, top_k + 1), np.float32)
        idx = np.empty((rows, top_k + 1), np.int32)
        status = np.empty(rows, np.int32)
        _check(lib().ec_topk_dev(buf.ptr, rows, V, V, top_k, _ptr(vals), _ptr(idx), _ptr(status)), "ec_topk_dev")
        return vals, idx, status
    finally:
        buf.close()


def attention_dev(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos, slot, H: int, KVH: int,
                  window: int = 0, path: int = 0) -> np.ndarray:
    """ec_attention_dev on host arrays (copied to the device): q [M][H*hd]
    fp32, kc / vc [nslots][C][KVH*hd] fp16 bits (uint16), pos / slot [M];
    returns out [M][H*hd] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.uint16)
    vc = np.ascontiguousarray(vc, np.uint16)
    pos = np.ascontiguousarray(pos, np.int32)
    slot = np.ascontiguousarray(slot, np.int32)
    M, E = q.shape
    nslots, C, kv = kc.shape
    hd = E // H
    bufs = [DeviceBuffer.from_array(a) for a in (q, kc, vc)] + [DeviceBuffer(q.nbytes)]
    try:
        _check(lib().ec_attention_dev(bufs[0].ptr, E, bufs[1].ptr, bufs[2].ptr, nslots, C, H, KVH, hd,
                                      _ptr(pos), _ptr(slot), M, window, bufs[3].ptr, E, path),
               "ec_attention_dev")
        return bufs[3].to_array(np.float32, (M, E))
    finally:
        for b in bufs:
            b.close()


# ---------------------------------------------------------------------------
# tools
# ---------------------------------------------------------------------------

def synth(out: str | os.PathLike | None, preset: Optional[str] = None, prompt_out=None,
          prompt_len: int = 0, prompt_seed: int = 1, **shape) -> None:
    """Run bin/ecm_synth (seeded synthetic .ecm model and/or prompt ids)."""
    if not SYNTH.exists():
        raise EdgeCoreError(f"{SYNTH} is not built; run `make`")
    cmd = [str(SYNTH)]
    if out is not None:
        cmd += ["--out", str(out)]
    if preset:
        cmd += ["--preset", preset]
    for k, v in shape.items():
        cmd += ["--" + k.replace("_", "-"), str(v)]
    if prompt_out is not None:
        cmd += ["--prompt-out", str(prompt_out), "--prompt-len", str(prompt_len),
                "--prompt-seed", str(prompt_seed)]
    subprocess.run(cmd, check=True)


def read_ids(path: str | os.PathLike) -> np.ndarray:
    return np.array(Path(path).read_text().split(), dtype=np.int32)
