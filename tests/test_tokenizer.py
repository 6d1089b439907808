"""Byte-level BPE tokenizer of the library (tokenizer.c) against the
reference tokenizer (src/tokenizer.c) -- CPU only.

A synthetic vocabulary (tests/tok_vocab.py: trained merges, merges the loader
must drop, a duplicated text, <|...|> specials) is loaded by both.  Token ids
and decoded bytes must be identical for the GPT-2 (0) and Qwen2 (1)
pre-tokenizers: on the committed fixture tests/golden/tokenizer.json (written
from the reference by tests/golden/make_tokenizer_golden.py, inputs from the
reference's tests/tokenizer/test_cases.json plus edge cases), and live on
random strings where the reference build oracle/_ref exists.
"""
import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

import edgecore_amd as ec
import oracle
from tests import tok_vocab

GOLDEN = Path(__file__).resolve().parent / "golden" / "tokenizer.json"


class Tok:
    def __init__(self, L, vb, mb, n_vocab, variant):
        self.L, self.t = L, ec.Tokenizer()
        assert L.tokenizer_load(C.byref(self.t), vb, len(vb), mb, len(mb), n_vocab, variant) == 0

    def encode(self, s):
        buf = (C.c_int * 8192)()
        n = self.L.tokenizer_encode(C.byref(self.t), s.encode("utf-8"), buf, 8192)
        return list(buf[:n]) if n >= 0 else None

    def decode(self, ids):
        arr = (C.c_int * max(len(ids), 1))(*ids)
        p = self.L.tokenizer_decode(C.byref(self.t), arr, len(ids))
        return C.string_at(p)


def _ref_lib():
    L = C.CDLL(str(oracle.REF_LIB))
    L.tokenizer_load.restype = C.c_int
    L.tokenizer_load.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, C.c_int, C.c_int]
    L.tokenizer_encode.restype = C.c_int
    L.tokenizer_encode.argtypes = [C.c_void_p, C.c_char_p, C.c_void_p, C.c_int]
    L.tokenizer_decode.restype = C.c_void_p
    L.tokenizer_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    return L


@pytest.fixture(scope="module")
def vocab_blobs():
    vocab, merges = tok_vocab.build()
    vb, mb = tok_vocab.blobs(vocab, merges)
    return vb, mb, len(vocab)


@pytest.mark.parametrize("variant", [0, 1])
def test_tokenizer_equals_reference_fixture(vocab_blobs, variant):
    vb, mb, nv = vocab_blobs
    g = json.loads(GOLDEN.read_text())
    assert g["n_vocab"] == nv, "vocabulary builder changed; regenerate the fixture"
    tok = Tok(ec.lib(), vb, mb, nv, variant)
    for s, want in zip(g["inputs"], g[f"variant{variant}"]):
        ids = tok.encode(s)
        assert ids == want["ids"], s
        assert tok.decode(ids).hex() == want["decoded_hex"], s
        if "<|" not in s:
            assert tok.decode(ids) == s.encode("utf-8")  # byte tokens cover every byte: round trip


def test_tokenizer_drops_bad_merges_and_finds_specials(vocab_blobs):
    vb, mb, nv = vocab_blobs
    tok = Tok(ec.lib(), vb, mb, nv, 0)
    vocab, merges = tok_vocab.build()
    assert tok.t.n_merges == len(merges) - 2
    assert tok.t.n_sp == 4 and tok.t.eos_id == vocab.index("<|endoftext|>")
    assert tok.encode("<|im_start|>x|>y") == [vocab.index("<|im_start|>x|>"), vocab.index("y")]  # longest first
    assert tok.encode("<|endoftext|>") == [vocab.index("<|endoftext|>")]
    assert tok.encode("abc", ) is not None and tok.encode("a" * 10000) is None  # overflow of max_out


@pytest.mark.skipif(not oracle.ref_available(), reason="reference build oracle/_ref absent")
@pytest.mark.parametrize("variant", [0, 1])
def test_tokenizer_equals_reference_live(vocab_blobs, variant):
    vb, mb, nv = vocab_blobs
    ours, ref = Tok(ec.lib(), vb, mb, nv, variant), Tok(_ref_lib(), vb, mb, nv, variant)
    rng = np.random.default_rng(variant)
    alphabet = list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789") + \
        list(" \t\n\r\x0b\x0c'!?.,;:-()[]{}<>|/\\\"") + ["é", "ö", "世", "界", "😀", "ñ", "<|im_end|>", "<|endoftext|>",
                                                         "'s", "'LL", "'re", "  ", "\n\n", "123456"]
    for _ in range(400):
        s = "".join(rng.choice(alphabet, size=int(rng.integers(0, 60))))
        a, b = ours.encode(s), ref.encode(s)
        assert a == b, repr(s)
        assert ours.decode(a) == ref.decode(b), repr(s)
