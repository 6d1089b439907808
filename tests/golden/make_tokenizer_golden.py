"""Writes tests/golden/tokenizer.json: token ids and decoded bytes of the
reference tokenizer (src/tokenizer.c, compiled into oracle/_ref/libref.so)
for the synthetic vocabulary of tests/tok_vocab.py, variants 0 (GPT-2) and
1 (Qwen2).  Inputs: the strings of the reference's tests/tokenizer/
test_cases.json (chat cases rendered with <|im_start|> / <|im_end|>) and
tests/tok_vocab.py's EXTRA_INPUTS.  Run from the repository root after
`make` (needs /root/reference and oracle/_ref)."""
import ctypes as C
import json
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))

from tests import tok_vocab  # noqa: E402
import edgecore_amd as ec  # noqa: E402
import oracle  # noqa: E402


def ref_lib():
    L = C.CDLL(str(oracle.REF_LIB))
    L.tokenizer_load.restype = C.c_int
    L.tokenizer_load.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, C.c_int, C.c_int]
    L.tokenizer_encode.restype = C.c_int
    L.tokenizer_encode.argtypes = [C.c_void_p, C.c_char_p, C.c_void_p, C.c_int]
    L.tokenizer_decode.restype = C.c_void_p
    L.tokenizer_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    return L


def run(L, vocab_blob, merges_blob, n_vocab, variant, texts):
    t = ec.Tokenizer()
    assert L.tokenizer_load(C.byref(t), vocab_blob, len(vocab_blob), merges_blob, len(merges_blob), n_vocab,
                            variant) == 0
    out = []
    for s in texts:
        buf = (C.c_int * 4096)()
        n = L.tokenizer_encode(C.byref(t), s.encode("utf-8"), buf, 4096)
        ids = list(buf[:n]) if n >= 0 else None
        dec = None
        if ids is not None:
            arr = (C.c_int * max(len(ids), 1))(*ids)
            p = L.tokenizer_decode(C.byref(t), arr, len(ids))
            dec = C.string_at(p).hex()
        out.append({"ids": ids, "decoded_hex": dec})
    return out


def main():
    cases = json.loads(Path("/root/reference/tests/tokenizer/test_cases.json").read_text())
    texts = [c["input"] if "input" in c else tok_vocab.chat(c["messages"]) for c in cases]
    texts += tok_vocab.EXTRA_INPUTS
    vocab, merges = tok_vocab.build()
    vb, mb = tok_vocab.blobs(vocab, merges)
    L = ref_lib()
    res = {"inputs": texts, "n_vocab": len(vocab),
           "variant0": run(L, vb, mb, len(vocab), 0, texts), "variant1": run(L, vb, mb, len(vocab), 1, texts)}
    (REPO / "tests" / "golden" / "tokenizer.json").write_text(json.dumps(res, ensure_ascii=False, indent=0))


if __name__ == "__main__":
    main()
