"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

ctypes binding of ``oracle/liboracle.so`` (our C restatement of the reference
CPU path, ec_oracle.c) and, where it was built, ``oracle/_ref/libref.so`` (the
reference's own C sources behind ref_harness.c).  Only tests/,
``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg use this module;
the product never does.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Optional

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "liboracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libref.so"
REF_RUNTIME = ORACLE_DIR / "_ref" / "edgecore-runtime"
REF_SAMPLE = ORACLE_DIR / "_ref" / "libref_sample.so"

_P, _I = C.c_void_p, C.c_int
_O: Optional[C.CDLL] = None
_R: Optional[C.CDLL] = None


def olib() -> C.CDLL:
    global _O
    if _O is None:
        if not ORACLE_LIB.exists():
            raise RuntimeError(f"{ORACLE_LIB} not built (make -C oracle)")
        L = C.CDLL(str(ORACLE_LIB))
        sig = {
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [C.c_float]),
            "or_quantize_int8_symmetric": (None, [_P, _I, _I, _P, _P]),
            "or_quantize_rows": (None, [_P, _I, _I, _P, _P]),
            "or_gemm_fp16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
            "or_gemm_bf16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
            "or_gemm_int8": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I]),
            "or_layernorm_rows": (None, [_P, _P, _P, _P, _I, _I, C.c_double]),
            "or_rmsnorm_rows": (None, [_P, _P, _P, _I, _I, C.c_double]),
            "or_gelu_new": (C.c_float, [C.c_float]),
            "or_silu": (C.c_float, [C.c_float]),
            "or_rope_inv_freq": (None, [_P, _I, C.c_double, _I, C.c_double, C.c_double]),
            "or_load": (_P, [C.c_char_p, _I, _I]),
            "or_free": (None, [_P]),
            "or_kv_reset": (None, [_P]),
            "or_vocab": (_I, [_P]),
            "or_eff_ctx": (_I, [_P]),
            "or_precision": (_I, [_P]),
            "or_arch": (_I, [_P]),
            "or_forward": (_I, [_P, _P, _P, _P, _I, _P]),
            "or_forward_from": (_I, [_P, _P, _P, _P, _I, _I, _P]),
            "or_argmax": (_I, [_P, _I]),
            "or_generate": (_I, [_P, _P, _I, _I, _P, _P]),
            "or_map": (None, [_I, _P, _P, C.c_size_t]),
            "or_attention_rows": (_I, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P, _I]),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, k)
            f.restype, f.argtypes = r, a
        if hasattr(L, "or_check_f16c"):
            L.or_check_f16c.restype, L.or_check_f16c.argtypes = C.c_uint64, [C.c_uint32, C.c_uint32]
            L.or_check_f16c_widen.restype, L.or_check_f16c_widen.argtypes = C.c_uint64, []
        _O = L
    return _O


def ref_available() -> bool:
    return REF_LIB.exists()


_RS: Optional[C.CDLL] = None


def ref_sample_available() -> bool:
    return REF_SAMPLE.exists()


def ref_sample(logits: np.ndarray, temp: float, top_k: int, state: int) -> tuple[int, int]:
    """The reference driver's own sample_token (src/runtime_main.c:213-248, built
    from that file by ref_sample.c) on one row, with its LCG state set to
    `state` first; returns (token, state after)."""
    global _RS
    if _RS is None:
        L = C.CDLL(str(REF_SAMPLE))
        L.ref_sample_token.restype = _I
        L.ref_sample_token.argtypes = [_P, _I, C.c_float, _I]
        L.ref_rng_set.restype = None
        L.ref_rng_set.argtypes = [C.c_ulonglong]
        L.ref_rng_get.restype = C.c_ulonglong
        L.ref_rng_get.argtypes = []
        _RS = L
    row = np.ascontiguousarray(logits, np.float32)
    _RS.ref_rng_set(state)
    tok = _RS.ref_sample_token(row.ctypes.data, len(row), temp, top_k)
    return tok, _RS.ref_rng_get()


def rlib() -> C.CDLL:
    global _R
    if _R is None:
        L = C.CDLL(str(REF_LIB))
        sig = {
            "refh_open": (_I, [C.c_char_p, _I, _I]),
            "refh_close": (None, [_I]),
            "refh_vocab": (_I, [_I]),
            "refh_eff_ctx": (_I, [_I]),
            "refh_precision": (_I, [_I]),
            "refh_forward": (None, [_I, _P, _P, _P, _I, _P]),
            "refh_kv_reset": (None, [_I]),
            "refh_logits": (_I, [_I, _P, _I, _P]),
            "refh_generate": (_I, [_I, _P, _I, _I, _P, _P]),
            "gemm_int8": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I]),
            "gemm_fp16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
            "gemm_bf16_fp32": (None, [_P, _P, _P, _I, _I, _I]),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, k)
            f.restype, f.argtypes = r, a
        _R = L
    return _R


def _p(a):
    return None if a is None else a.ctypes.data


# ---- kernels ---------------------------------------------------------------

def gemm_int8(A, a_scale, B, b_scale=None, bias=None, impl: str = "oracle") -> np.ndarray:
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    a_scale = np.ascontiguousarray(a_scale, np.float32)
    b_scale = None if b_scale is None else np.ascontiguousarray(b_scale, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.float32)
    fn = olib().or_gemm_int8 if impl == "oracle" else rlib().gemm_int8
    fn(_p(out), _p(A), _p(a_scale), _p(B), _p(b_scale), _p(bias), M, K, N)
    return out


def gemm_w16(A, B, bf16: bool = False, impl: str = "oracle") -> np.ndarray:
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.uint16)
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.float32)
    if impl == "oracle":
        fn = olib().or_gemm_bf16_fp32 if bf16 else olib().or_gemm_fp16_fp32
    else:
        fn = rlib().gemm_bf16_fp32 if bf16 else rlib().gemm_fp16_fp32
    fn(_p(out), _p(A), _p(B), M, K, N)
    return out


def quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    olib().or_quantize_rows(_p(x), M, K, _p(q), _p(s))
    return q, s


def quantize_int8_symmetric(w) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, np.float32)
    r, c = w.shape
    q = np.empty((r, c), np.int8)
    s = np.empty(r, np.float32)
    olib().or_quantize_int8_symmetric(_p(w), r, c, _p(q), _p(s))
    return q, s


def map_op(op: int, x: np.ndarray) -> np.ndarray:
    """Reference elementwise arithmetic (op codes of ec_device_math)."""
    x = np.ascontiguousarray(x)
    out = np.empty(x.shape, {3: np.uint16, 5: np.int8}.get(op, np.float32))
    olib().or_map(op, _p(x), _p(out), x.size)
    return out


def attention_rows(q, kc, vc, pos, slot, H: int, KVH: int, rows=None, window: int = 0) -> np.ndarray:
    """Reference attention (or_attention_rows) of the listed rows (all if
    None): q [M][H*hd] fp32, kc / vc [nslots][C][KVH*hd] fp16 bits, pos /
    slot [M].  Rows not listed come back as NaN."""
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.uint16)
    vc = np.ascontiguousarray(vc, np.uint16)
    pos = np.ascontiguousarray(pos, np.int32)
    slot = np.ascontiguousarray(slot, np.int32)
    M, E = q.shape
    nslots, C, _ = kc.shape
    rows = np.arange(M, dtype=np.int32) if rows is None else np.ascontiguousarray(rows, np.int32)
    out = np.full((M, E), np.nan, np.float32)
    rc = olib().or_attention_rows(_p(q), E, _p(kc), _p(vc), nslots, C, H, KVH, E // H, _p(pos), _p(slot),
                                  _p(rows), rows.size, window, _p(out), E)
    if rc:
        raise ValueError("or_attention_rows: arguments outside the caches")
    return out


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    L = olib()
    return np.array([L.or_f32_to_f16(float(v)) for v in x], np.uint16)


# ---- models ----------------------------------------------------------------

class OracleModel:
    def __init__(self, path, batch_cap: int = 1, max_ctx: int = 0):
        self.h = olib().or_load(str(path).encode(), batch_cap, max_ctx)
        if not self.h:
            raise RuntimeError(f"oracle could not load {path}")
        self.vocab = olib().or_vocab(self.h)
        self.eff_ctx = olib().or_eff_ctx(self.h)

    def kv_reset(self):
        olib().or_kv_reset(self.h)

    def forward(self, tokens, positions, seqs=None, lm_from: int = 0) -> np.ndarray:
        """Logits of rows [lm_from, M) (the LM head skips the rows before)."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(positions, np.int32)
        s = None if seqs is None else np.ascontiguousarray(seqs, np.int32)
        out = np.empty((len(t) - lm_from, self.vocab), np.float32)
        rc = olib().or_forward_from(self.h, _p(t), _p(p), _p(s), len(t), lm_from, _p(out))
        if rc:
            raise RuntimeError("oracle forward rejected its inputs")
        return out

    def generate(self, prompt, n_gen: int, want_logits: bool = False):
        prompt = np.ascontiguousarray(prompt, np.int32)
        ids = np.empty(len(prompt) + n_gen, np.int32)
        lg = np.empty((n_gen, self.vocab), np.float32) if want_logits else None
        rc = olib().or_generate(self.h, _p(prompt), len(prompt), n_gen, _p(ids), _p(lg))
        if rc:
            raise RuntimeError("oracle generate failed")
        return ids, lg

    def close(self):
        if self.h:
            olib().or_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class RefModel:
    """The reference's own gpt2_load/gpt2_forward (only where oracle/_ref exists)."""

    def __init__(self, path, batch_cap: int = 1, max_ctx: int = 0):
        self.h = rlib().refh_open(str(path).encode(), batch_cap, max_ctx)
        if self.h < 0:
            raise RuntimeError(f"reference could not load {path}")
        self.vocab = rlib().refh_vocab(self.h)

    def logits(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((len(t), self.vocab), np.float32)
        rlib().refh_logits(self.h, _p(t), len(t), _p(out))
        return out

    def forward(self, tokens, positions, seqs=None) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(positions, np.int32)
        s = None if seqs is None else np.ascontiguousarray(seqs, np.int32)
        out = np.empty((len(t), self.vocab), np.float32)
        rlib().refh_forward(self.h, _p(t), _p(p), _p(s), len(t), _p(out))
        return out

    def kv_reset(self):
        rlib().refh_kv_reset(self.h)

    def generate(self, prompt, n_gen: int, want_logits: bool = False):
        prompt = np.ascontiguousarray(prompt, np.int32)
        ids = np.empty(len(prompt) + n_gen, np.int32)
        lg = np.empty((n_gen, self.vocab), np.float32) if want_logits else None
        rc = rlib().refh_generate(self.h, _p(prompt), len(prompt), n_gen, _p(ids), _p(lg))
        if rc:
            raise RuntimeError("reference generate failed")
        return ids, lg

    def close(self):
        if self.h is not None and self.h >= 0:
            rlib().refh_close(self.h)
            self.h = -1

    def __del__(self):
        self.close()
