"""Builds libvitna_hip's native parts in-tree, for gfx950.

    python vitna-anchor_amd/build.py          # HIP library + synthetic-model library
    python vitna-anchor_amd/build.py --all    # also the CPU checker (oracle/)
    python vitna-anchor_amd/build.py --incremental   # recompile only what changed

Outputs (git-ignored, carried to the GPU box with the tree):
  vitna-anchor_amd/libvitna_hip.so          the HIP kernels and the C ABI (include/vitna_hip.h)
  vitna-anchor_amd/synth/libvitna_synth.so  seeded synthetic models (workload generation)
"""
import concurrent.futures
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # no multiply fused into an add unless the code says fmaf: the exact paths rely on it
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed fp32 instructions stay off (they are not trusted on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s%s" % (" ".join(cmd), r.stdout, r.stderr))
    return r


def build_hip(incremental=False):
    srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")))
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    # every object depends on its source and on every header it may include
    deps = glob.glob(os.path.join(PKG, "csrc", "*.h")) + glob.glob(os.path.join(ROOT, "include", "*.h"))
    newest_dep = max((os.path.getmtime(d) for d in deps), default=0.0)
    jobs, objs = [], []
    for s in srcs:
        o = os.path.join(objdir, os.path.basename(s) + ".o")
        objs.append(o)
        if incremental and os.path.exists(o) and os.path.getmtime(o) > max(os.path.getmtime(s), newest_dep):
            continue
        jobs.append((s, o))
    # host-only C++ (the GGUF reader) compiles with the host compiler
    for s in sorted(glob.glob(os.path.join(PKG, "csrc", "*.cpp"))):
        o = os.path.join(objdir, os.path.basename(s) + ".o")
        objs.append(o)
        if not (incremental and os.path.exists(o) and os.path.getmtime(o) > max(os.path.getmtime(s), newest_dep)):
            jobs.append((s, o))
    if jobs:
        def compile_one(so):
            if so[0].endswith(".cpp"):
                return _run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-c", so[0], "-o", so[1]])
            return _run([HIPCC] + HIP_FLAGS + ["-c", so[0], "-o", so[1]])
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
            list(ex.map(compile_one, jobs))
    out = os.path.join(PKG, "libvitna_hip.so")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out] + objs)
    return out


def build_synth():
    out = os.path.join(PKG, "synth", "libvitna_synth.so")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", os.path.join(PKG, "synth", "vitna_synth.c"),
          os.path.join(PKG, "synth", "gguf_write.c"), "-o", out, "-lm", "-lpthread"])
    return out


def build_oracle():
    """The CPU checker (test infrastructure), and the compiled reference when its sources are here."""
    _run(["make", "-C", os.path.join(ROOT, "oracle")])
    if os.path.isdir("/root/reference/engine/src"):
        _run(["make", "-C", os.path.join(ROOT, "oracle"), "ref", "-j8"])


def main(argv):
    build_synth()
    # --incremental (a developer's rebuild): objects newer than their source and every header are kept
    build_hip(incremental="--incremental" in argv)
    if "--all" in argv:
        build_oracle()


if __name__ == "__main__":
    main(sys.argv[1:])
