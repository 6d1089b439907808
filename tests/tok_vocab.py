"""A synthetic byte-level BPE vocabulary in the .ecm tokenizer blob format
(edgecore/ecm.py:127-171 layout), for tokenizer tests.

Token texts use GPT-2's bytes_to_unicode alphabet.  Merges are learned by a
plain most-frequent-pair BPE on a fixed corpus (deterministic), and the list
also holds merges the loader must drop (a half or the concatenation not in
the vocabulary), a duplicated text, and <|...|> special tokens.
"""
import collections
import struct

CORPUS = (
    "The rapid adoption of small language models has created a need for efficient deployment on "
    "diverse computing environments. Hello world. What is 2 + 2? Explain CPU cache locality! "
    "system You are Qwen, created by Alibaba Cloud. You are a helpful assistant. user assistant "
    "don't won't it's we'll they've I'm you're 12345 67890 the the the and and of of to to in in "
    "café naïve 世界"
)


def bytes_to_unicode():
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cps, extra = {}, 0
    for b in range(256):
        if b in keep:
            cps[b] = chr(b)
        else:
            cps[b] = chr(256 + extra)
            extra += 1
    return cps


def build(n_merges=300):
    b2u = bytes_to_unicode()
    words = collections.Counter()
    for w in CORPUS.replace("\n", " ").split(" "):
        if w:
            words[tuple(b2u[b] for b in (" " + w).encode())] += 1
            words[tuple(b2u[b] for b in w.encode())] += 1
    vocab = [b2u[b] for b in range(256)]
    merges = []
    for _ in range(n_merges):
        pairs = collections.Counter()
        for w, c in words.items():
            for a, b in zip(w, w[1:]):
                pairs[(a, b)] += c
        if not pairs:
            break
        (a, b), _ = max(pairs.items(), key=lambda kv: (kv[1], kv[0]))
        merges.append((a, b))
        vocab.append(a + b)
        nw = collections.Counter()
        for w, c in words.items():
            out, i = [], 0
            while i < len(w):
                if i + 1 < len(w) and w[i] == a and w[i + 1] == b:
                    out.append(a + b)
                    i += 2
                else:
                    out.append(w[i])
                    i += 1
            nw[tuple(out)] += c
        words = nw
    # merges to drop: unknown half, unknown concatenation
    merges.insert(5, ("zzq", "e"))
    merges.insert(9, ("Q", "ĠQ"))
    specials = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|im_start|>x|>"]
    vocab += specials
    vocab.append(vocab[300])  # a duplicated text (the first id must win in lookups)
    return vocab, merges


def blobs(vocab, merges):
    v = bytearray(struct.pack("<I", len(vocab)))
    for i, t in enumerate(vocab):
        e = t.encode("utf-8")
        v += struct.pack("<II", i, len(e)) + e
    m = bytearray(struct.pack("<I", len(merges)))
    for a, b in merges:
        ea, eb = a.encode("utf-8"), b.encode("utf-8")
        m += struct.pack("<I", len(ea)) + ea + struct.pack("<I", len(eb)) + eb
    return bytes(v), bytes(m)


def chat(messages):
    s = ""
    for msg in messages:
        s += "<|im_start|>" + msg["role"] + "\n" + msg["content"] + "<|im_end|>\n"
    return s + "<|im_start|>assistant\n"


EXTRA_INPUTS = [
    "", " ", "     ", "x   ", "   y", "a\n\nb\r\n c  \t d   ", "don't I'll we've they're", "A'S IT'LL 'RE",
    "1234567 89 0", "<|im_start|>user\nhi<|im_end|>", "<|im_sta", "<|im_start|>x|>y <|im_start|>x", "<|endoftext|>", "a<|endoftext|>b",
    "héllo wörld 日本語 😀", "the the the and of", "?!... --- ;;", "\t\n\r\x0b\x0c",
]
