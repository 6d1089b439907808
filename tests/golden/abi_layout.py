"""Field offsets and sizes of the ABI structs (GPT2, struct LayerW, Tokenizer,
EcmTensor), printed by a C program compiled against a given edgecore.h.

make_abi_golden.py runs it on the reference's src/edgecore.h and writes
abi_layout.json; tests/test_abi.py runs it on include/edgecore.h and compares.
"""
import json
import subprocess
import tempfile
from pathlib import Path

STRUCTS = {
    "GPT2": ["model_name", "n_layer", "n_head", "n_embd", "n_ctx", "vocab", "n_kv_head", "n_kv_embd",
             "intermediate", "head_dim", "arch", "n_params", "eps", "rope_theta", "rope_type", "yarn_factor",
             "yarn_orig_max", "yarn_attention_factor", "sliding_window", "tie_word_embeddings", "eos_token_id",
             "wte", "wpe", "lw", "lnf_g", "lnf_b", "lm_head", "precision", "k_cache", "v_cache", "batch_cap",
             "max_ctx", "ws_x", "ws_tmp", "ws_qkv", "ws_attn", "ws_scores", "ws_q", "ws_qs", "ws_q_cols", "tok",
             "file_data", "file_size", "file_mapped"],
    "struct LayerW": ["ln1_g", "ln1_b", "attn_w", "attn_s", "attn_b", "proj_w", "proj_s", "proj_b", "ln2_g",
                      "ln2_b", "fc_w", "fc_s", "fc_b", "fc2_w", "fc2_s", "fc2_b", "q_w", "k_w", "v_w", "o_w",
                      "q_s", "k_s", "v_s", "o_s", "q_b", "k_b", "v_b", "o_b", "gate_w", "up_w", "down_w",
                      "gate_s", "up_s", "down_s", "gate_b", "up_b", "down_b"],
    "Tokenizer": [],
    "EcmTensor": ["name", "dtype", "nelems", "bytes", "offset", "dims", "ndims"],
}


def layout(header: Path, cflags=()) -> dict:
    lines = ["#include <immintrin.h>", "#include <stddef.h>", "#include <stdio.h>", f'#include "{header}"',
             "int main(void) {", '  printf("{");']
    first = True
    for st, fields in STRUCTS.items():
        key = st.replace("struct ", "")
        sep = "" if first else ", "
        first = False
        lines.append(f'  printf("{sep}\\"{key}\\": {{\\"sizeof\\": %zu", sizeof({st}));')
        for f in fields:
            lines.append(f'  printf(", \\"{f}\\": %zu", offsetof({st}, {f}));')
        lines.append('  printf("}");')
    lines += ['  printf("}\\n");', "  return 0;", "}"]
    with tempfile.TemporaryDirectory() as d:
        src, exe = Path(d) / "l.c", Path(d) / "l"
        src.write_text("\n".join(lines) + "\n")
        subprocess.run(["gcc", "-std=c11", "-mavx2", "-mf16c", *cflags, str(src), "-o", str(exe)], check=True,
                       capture_output=True)
        return json.loads(subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout)
