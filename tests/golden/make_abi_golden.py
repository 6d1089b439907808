#!/usr/bin/env python3
"""Writes tests/golden/abi_layout.json: the struct layout of the reference's
src/edgecore.h (GPT2, struct LayerW, Tokenizer, EcmTensor), which
include/edgecore.h must reproduce so that a caller compiled against the
reference header can pass its structs to this library."""
import json
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))
from abi_layout import layout  # noqa: E402

REF = Path("/root/reference/src/edgecore.h")
OUT = Path(__file__).resolve().parent / "abi_layout.json"

if __name__ == "__main__":
    d = layout(REF)
    OUT.write_text(json.dumps(d, indent=1) + "\n")
    print(f"wrote {OUT}: sizeof(GPT2) {d['GPT2']['sizeof']}")
