"""Writes the golden fixtures in tests/golden/ from the reference's own C code.

Needs /root/reference (this container only). Builds the reference engine's C
sources with oracle/Makefile (target ``ref``), runs the harness
tests/golden/ref_golden.c, and packs what it prints into ref_vectors.npz. It
also records the reference's struct layout (offsetof / sizeof of every member
the boundary passes) into ref_layout.json, by compiling a probe against the
reference's headers.

    python tests/golden/make_golden.py
"""
import json
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.environ.get("VITNA_REF", "/root/reference")

# Members of the engine's structs whose placement the boundary depends on.
LAYOUT = {
    "vitna_llama_config_t": ["n_layers", "hidden", "intermediate", "n_heads", "n_kv_heads", "head_dim", "vocab",
                             "max_positions", "rms_eps", "rope_theta", "tied_embeddings", "qk_norm",
                             "qk_norm_per_head", "n_experts", "n_experts_used", "renormalize", "qwen3"],
    "vitna_matrix_t": ["data", "dtype", "rows", "cols"],
    "vitna_expert_t": ["gate", "up", "down"],
    "vitna_llama_layer_t": ["attn_norm", "mlp_norm", "q", "k", "v", "o", "gate", "up", "down", "q_norm", "k_norm",
                            "router", "experts"],
    "vitna_llama_t": ["cfg", "shards", "shard_paths", "n_shards", "embed", "lm_head", "final_norm", "layers",
                      "inv_freq", "ctx", "seqs", "past", "k_cache", "v_cache", "x", "xn", "q", "k", "v", "att",
                      "proj", "gate", "up", "scores", "cos_t", "sin_t", "router_logits", "expert_out", "stream",
                      "pred_xn", "pred_logits", "predicted", "predicted_layer", "predicted_right",
                      "predicted_total", "trace_logits", "trace_chosen", "trace_positions", "pin", "pin_positions",
                      "cuda", "rows_max", "rows_logits", "rows_next", "rows_weights", "rows_order", "rows_pred",
                      "rows_chunk", "rows_outs", "no_rows", "gpu_kv_layers", "gpu_fast", "device_lost",
                      "device_error", "fail_armed", "fail_loses", "fail_at"],
}


def layout_probe_source(header):
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "%s"' % header, "int main(void) {",
             '  printf("{");']
    first = True
    for typ, members in LAYOUT.items():
        sep = "" if first else ","
        first = False
        lines.append('  printf("%s\\"%s\\": {\\"sizeof\\": %%zu", sizeof(%s));' % (sep, typ, typ))
        for mem in members:
            lines.append('  printf(", \\"%s\\": %%zu", offsetof(%s, %s));' % (mem, typ, mem))
        lines.append('  printf("}");')
    lines.append('  printf("}\\n"); return 0; }')
    return "\n".join(lines)


def probe_layout(header, include_dirs):
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        with open(src, "w") as f:
            f.write(layout_probe_source(header))
        cmd = ["gcc", "-O0", src, "-o", exe] + ["-I" + i for i in include_dirs]
        subprocess.run(cmd, check=True)
        return json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)


def read_records(path):
    recs = {}
    with open(path, "rb") as f:
        data = f.read()
    off = 0
    while off < len(data):
        (n,) = struct.unpack_from("<I", data, off)
        off += 4
        name = data[off:off + n].decode()
        off += n
        kind = chr(data[off])
        off += 1
        (count,) = struct.unpack_from("<Q", data, off)
        off += 8
        dt = {"f": np.float32, "i": np.int32, "u": np.uint8}[kind]
        size = count * np.dtype(dt).itemsize
        recs[name] = np.frombuffer(data[off:off + size], dtype=dt).copy()
        off += size
    return recs


def main():
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "ref", "REF=" + REF, "-j8"], check=True)
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "golden.bin")
        run = subprocess.run([os.path.join(ROOT, "oracle", "_ref", "ref_golden"), out], check=True,
                             capture_output=True, text=True)
        recs = read_records(out)
    meta = {"matvec_path": run.stderr.strip(), "gcc": subprocess.run(["gcc", "--version"], capture_output=True,
                                                                     text=True).stdout.splitlines()[0],
            "glibc": os.confstr("CS_GNU_LIBC_VERSION")}
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **recs)
    with open(os.path.join(HERE, "ref_vectors.meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    layout = probe_layout("model.h", [os.path.join(REF, "engine", "include")])
    with open(os.path.join(HERE, "ref_layout.json"), "w") as f:
        json.dump(layout, f, indent=1)
    print("wrote %d records; %s" % (len(recs), meta))


if __name__ == "__main__":
    sys.exit(main())
