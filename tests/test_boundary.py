"""The drop-in boundary, checked without a GPU.

* include/vitna_model.h lays out the engine's structs exactly as the
  reference's model.h does (offsets recorded from the reference's own header
  by tests/golden/make_golden.py into ref_layout.json), and the ctypes mirror
  in vitna_amd agrees with both.
* libvitna_hip.so loads and exports every function include/vitna_hip.h
  declares.
* The host-side refusals the reference makes are made (no compute call runs
  without a GPU).
"""
import ctypes as C
import json
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import vitna_amd as va

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys_path = os.path.join(ROOT, "tests", "golden")


def probe_ours():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(ROOT, "tests", "golden", "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    return mg.probe_layout(os.path.join(ROOT, "include", "vitna_model.h"), [])


def test_struct_layout_matches_reference():
    with open(os.path.join(ROOT, "tests", "golden", "ref_layout.json")) as f:
        ref = json.load(f)
    ours = probe_ours()
    assert ours == ref


def test_ctypes_mirror_matches_reference():
    with open(os.path.join(ROOT, "tests", "golden", "ref_layout.json")) as f:
        ref = json.load(f)
    mirror = {"vitna_llama_config_t": va.Config, "vitna_matrix_t": va.Matrix, "vitna_expert_t": va.Expert,
              "vitna_llama_layer_t": va.Layer, "vitna_llama_t": va.Llama}
    for name, cls in mirror.items():
        assert C.sizeof(cls) == ref[name]["sizeof"], name
        for field, off in ref[name].items():
            if field != "sizeof":
                assert getattr(cls, field).offset == off, (name, field)


def declared_functions():
    """Every function the library's headers (include/vitna_hip.h, include/vitna_gguf.h) declare."""
    names = set()
    for h in ("vitna_hip.h", "vitna_gguf.h"):
        with open(os.path.join(ROOT, "include", h)) as f:
            text = f.read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(vitna_(?:cuda|hip)_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    assert os.path.exists(va.HIP_LIB), "build first: python vitna-anchor_amd/build.py"
    names = declared_functions()
    assert len(names) >= 39
    out = subprocess.run(["nm", "-D", "--defined-only", va.HIP_LIB], capture_output=True, text=True, check=True).stdout
    exported = set(line.split()[-1] for line in out.splitlines() if " T " in line)
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    lib = va.hip()
    for n in names:
        assert getattr(lib, n) is not None


def test_headers_compile_as_c_and_cpp():
    """The engine's C code includes the ABI header (model.c is C); it compiles as C99 and as C++, warning-free."""
    with tempfile.TemporaryDirectory() as d:
        src_c = os.path.join(d, "t.c")
        with open(src_c, "w") as f:
            f.write('#include "vitna_hip.h"\n#include "vitna_gguf.h"\nint main(void) { return vitna_cuda_probe(0, 0) ? 0 : 0; }\n')
        src_cc = os.path.join(d, "t.cc")
        with open(src_cc, "w") as f:
            f.write('#include "vitna_hip.h"\n#include "vitna_gguf.h"\nint main() { return 0; }\n')
        inc = os.path.join(ROOT, "include")
        for cmd in (["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", inc, "-c", src_c, "-o", os.path.join(d, "c.o")],
                    ["g++", "-std=c++11", "-Wall", "-Wextra", "-Werror", "-I", inc, "-c", src_cc, "-o", os.path.join(d, "cc.o")]):
            r = subprocess.run(cmd, capture_output=True, text=True)
            assert r.returncode == 0, r.stderr


def test_library_is_gfx950():
    """The offload bundle's target ids name gfx950 and nothing else."""
    import re
    data = open(va.HIP_LIB, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}, targets


def test_dense_entry_points_refuse():
    lib = va.hip()
    err = C.create_string_buffer(256)
    lib.vitna_cuda_step.restype = C.c_bool
    assert not lib.vitna_cuda_step(None, 0, 0, 0, None, err, 256)
    assert b"mixture of experts" in err.value
    lib.vitna_cuda_cpu_experts.restype = C.c_bool
    assert not lib.vitna_cuda_cpu_experts(None, 4, err, 256)
    lib.vitna_cuda_prompt_min.restype = C.c_size_t
    assert lib.vitna_cuda_prompt_min(None) == 2 ** 64 - 1


def test_create_refuses_bad_shapes_before_touching_a_device():
    """check_shapes runs before any HIP call: a dense model, and an expert width the kernels do not take."""
    lib = va.hip()
    m = va.Model(va.shape(n_layers=1, hidden=256, intermediate=256, n_experts=8, n_experts_used=2, attention=0,
                          dt_gate_up=va.Q8_0, dt_down=va.Q8_0), 1)
    try:
        err = C.create_string_buffer(256)
        m.m.cfg.n_experts = 0
        assert not lib.vitna_cuda_create(m.ptr, None, None, 0, err, 256)
        assert b"dense" in err.value
        m.m.cfg.n_experts = 8
        m.m.layers[0].router.dtype = va.F16
        assert not lib.vitna_cuda_create(m.ptr, None, None, 0, err, 256)
        assert b"router must be F32" in err.value
        m.m.layers[0].router.dtype = va.F32
        m.m.layers[0].experts[3].down.dtype = va.Q4_K
        assert not lib.vitna_cuda_create(m.ptr, None, None, 0, err, 256)
        assert b"share a dtype" in err.value
    finally:
        m.m.layers[0].experts[3].down.dtype = va.Q8_0
        m.free()


def test_create_refuses_a_context_the_merge_cannot_take():
    """More than 1024 attention chunks of 64 positions is refused by check_shapes, before any HIP call."""
    lib = va.hip()
    m = va.Model(va.shape(n_layers=1, hidden=256, intermediate=256, n_heads=4, n_kv_heads=2, head_dim=64, vocab=300,
                          n_experts=8, n_experts_used=2, dt_gate_up=va.Q8_0, dt_down=va.Q8_0, dt_q=va.Q8_0,
                          dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0, dt_head=va.Q8_0, dt_embed=va.Q8_0, ctx=64), 1)
    try:
        err = C.create_string_buffer(256)
        m.m.ctx = 65537
        assert not lib.vitna_cuda_create(m.ptr, None, None, 0, err, 256)
        assert b"context of 65537 positions" in err.value
    finally:
        m.m.ctx = 64
        m.free()


def test_probe_without_gpu_says_why():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    lib = va.hip()
    err = C.create_string_buffer(256)
    assert not lib.vitna_cuda_probe(err, 256)
    assert err.value


REF_ENGINE = "/root/reference/engine/src"


@pytest.mark.skipif(not os.path.isdir(REF_ENGINE), reason="the reference's sources are not here (the GPU box)")
def test_reference_engine_links_against_library():
    """The drop-in claim: the reference engine's own C sources, compiled with -DVITNA_CUDA=1 as its CUDA build
    compiles them (engine/Makefile:24-52), link against libvitna_hip.so in place of model_cuda.cu with no
    undefined symbol (oracle/Makefile target link), and the linked engine starts."""
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "link", "-j8"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    objs = os.path.join(ROOT, "oracle", "_ref", "cuda_obj")
    need = set()
    for o in os.listdir(objs):
        out = subprocess.run(["nm", "-u", os.path.join(objs, o)], capture_output=True, text=True).stdout
        need |= {l.split()[-1] for l in out.splitlines() if "vitna_cuda_" in l}
    assert len(need) >= 20, sorted(need)
    have = subprocess.run(["nm", "-D", "--defined-only", os.path.join(ROOT, "vitna-anchor_amd", "libvitna_hip.so")],
                          capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in have.splitlines()}
    assert need <= exported, sorted(need - exported)
    run = subprocess.run([os.path.join(ROOT, "oracle", "_ref", "vitna-anchor-hip"), "--help"], capture_output=True,
                         text=True, timeout=60)
    assert "--device cuda" in run.stdout + run.stderr
