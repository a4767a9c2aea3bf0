"""Writes tests/golden/gguf_ref_dump.json: what the reference's own GGUF reader
and loader (compiled from /root/reference by oracle/Makefile target ref, run
as oracle/_ref/ref_gguf_dump) make of one fixed synthetic checkpoint, with the
checkpoint's SHA-256, so that the GGUF reader's test can compare against the
reference where the reference is not present.

    python tests/golden/make_gguf_fixture.py
"""
import hashlib
import json
import os
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "vitna-anchor_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import vitna_amd as va  # noqa: E402
from test_gguf import FIXED, REF_DUMP, FIXTURE, make  # noqa: E402


def main():
    spec, seed, norm_dtype, alignment, ctx, seqs = FIXED
    with tempfile.TemporaryDirectory() as tmp:
        path = make(tmp, spec, seed, norm_dtype, alignment)
        with open(path, "rb") as f:
            sha = hashlib.sha256(f.read()).hexdigest()
        r = subprocess.run([REF_DUMP, tmp, str(ctx), str(seqs)], capture_output=True, text=True, check=True)
    out = {"about": "oracle/_ref/ref_gguf_dump on the checkpoint tests/test_gguf.py FIXED describes "
                    "(vitna_synth_write_gguf of that seeded model)", "sha256": sha, "reference": json.loads(r.stdout)}
    with open(FIXTURE, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", FIXTURE, "sha256", sha)


if __name__ == "__main__":
    main()
