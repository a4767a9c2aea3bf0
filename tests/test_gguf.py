"""The GGUF reader (include/vitna_gguf.h, csrc/gguf_reader.cpp) against the
reference's own reader and loader, without a GPU.

A synthetic Qwen3-shaped model is written as a GGUF checkpoint by the
synthetic-model library (synth/gguf_write.c): llama.cpp's tensor names,
expert stacks, metadata the reader must step over. The reference's
vitna_gguf_open (engine/src/gguf.c:229) and vitna_llama_load_ex
(engine/src/model.c:302), compiled from /root/reference by oracle/Makefile,
describe what they read (tests/golden/ref_gguf_dump.c); the library's reader
must describe the same: every tensor's name, dtype, shape and offsets, the
metadata, every matrix's place in the file, the norm weights' bits, the
rotary frequencies, the cache shape. Where the reference is not here (the GPU
box), the reference's description of one fixed file is committed
(tests/golden/gguf_ref_dump.json, with the file's SHA-256) and checked
instead.
"""
import ctypes as C
import hashlib
import json
import os
import struct
import subprocess

import pytest

import vitna_amd as va

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DUMP = os.path.join(ROOT, "oracle", "_ref", "ref_gguf_dump")
FIXTURE = os.path.join(ROOT, "tests", "golden", "gguf_ref_dump.json")

SMALL = dict(n_layers=2, hidden=256, intermediate=256, n_heads=4, n_kv_heads=2, head_dim=64, vocab=300, n_experts=8,
             n_experts_used=2, renormalize=1, norm_std=0.1, ctx=64)
# the fixture's model: the seed and shape the committed reference description was made from
FIXED = (dict(SMALL), 4242, va.F32, 32, 48, 2)


def fnv(b):
    h = 1469598103934665603
    for x in b:
        h = ((h ^ x) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return "%016x" % h


def ours(path, ctx, seqs):
    """What the library's reader makes of the checkpoint, in ref_gguf_dump's form."""
    g = va.GgufModel(path, ctx=ctx, seqs=seqs)
    try:
        i = g.info
        out = {"info": {"arch": i.arch.decode(), "version": i.version, "alignment": i.alignment,
                        "block_count": i.block_count, "embedding_length": i.embedding_length,
                        "feed_forward_length": i.feed_forward_length,
                        "expert_feed_forward_length": i.expert_feed_forward_length, "head_count": i.head_count,
                        "head_count_kv": i.head_count_kv, "key_length": i.key_length,
                        "context_length": i.context_length, "expert_count": i.expert_count,
                        "expert_used_count": i.expert_used_count, "rms_eps": i.rms_eps,
                        "rope_freq_base": i.rope_freq_base, "file_tensors": i.file_tensors,
                        "data_offset": g.data_offset()}}
        ts = g.tensors()
        out["tensors"] = [list(t) for t in ts]
        lib = va.hip()
        t0 = va.GgufTensor()
        assert lib.vitna_hip_gguf_tensor(g.g, 0, C.byref(t0))
        base = t0.data - t0.offset_begin
        m, c = g.m, g.cfg

        def mat(x):
            return [x.dtype, x.rows, x.cols, (x.data - base) if x.data else -1]

        def vec(p, n):
            return [n, fnv(C.string_at(p, 4 * n)) if p else "%016x" % 0]

        d = {"cfg": [c.n_layers, c.hidden, c.intermediate, c.n_heads, c.n_kv_heads, c.head_dim, c.vocab, c.max_positions,
                     float("%.9g" % c.rms_eps), float("%.9g" % c.rope_theta), int(c.tied_embeddings), int(c.qk_norm),
                     int(c.qk_norm_per_head), c.n_experts, c.n_experts_used, int(c.renormalize), int(c.qwen3)],
             "ctx": m.ctx, "seqs": m.seqs, "embed": mat(m.embed), "lm_head": mat(m.lm_head),
             "final_norm": vec(C.cast(m.final_norm, C.c_void_p).value, c.hidden),
             "inv_freq": vec(C.cast(m.inv_freq, C.c_void_p).value, c.head_dim // 2)}
        qn = c.head_dim if c.qk_norm_per_head else c.n_heads * c.head_dim
        kn = c.head_dim if c.qk_norm_per_head else c.n_kv_heads * c.head_dim
        for l in range(c.n_layers):
            L = m.layers[l]
            for nm in ("q", "k", "v", "o", "router"):
                d["%d.%s" % (l, nm)] = mat(getattr(L, nm))
            for nm, n in (("attn_norm", c.hidden), ("mlp_norm", c.hidden), ("q_norm", qn), ("k_norm", kn)):
                d["%d.%s" % (l, nm)] = vec(C.cast(getattr(L, nm), C.c_void_p).value, n)
            for e in range(c.n_experts):
                x = L.experts[e]
                for nm in ("gate", "up", "down"):
                    d["%d.%d.%s" % (l, e, nm)] = mat(getattr(x, nm))
        d["end"] = 0
        out["model"] = d
        return out
    finally:
        g.free()


def theirs(directory, ctx, seqs):
    r = subprocess.run([REF_DUMP, directory, str(ctx), str(seqs)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-1000:] + r.stderr[-1000:]
    return json.loads(r.stdout)


def normalized(d):
    """Floats compared as float32 values where the two sides print them differently."""
    return json.loads(json.dumps(d))


def make(tmp, spec, seed, norm_dtype, alignment):
    model = va.Model(va.shape(**spec), seed)
    try:
        va.write_gguf(model, str(tmp), norm_dtype, alignment)
    finally:
        model.free()
    return os.path.join(str(tmp), "model.gguf")


needs_ref = pytest.mark.skipif(not os.path.exists(REF_DUMP), reason="the compiled reference is not here (oracle/_ref)")


@needs_ref
@pytest.mark.parametrize("variant", ["q4km_f32norm", "q8_f16norm_align64", "q4km_bf16norm_renorm0", "mixed_dtypes"])
def test_reader_matches_reference(tmp_path, variant):
    spec = dict(SMALL)
    norm_dtype, alignment, ctx, seqs = va.F32, 32, 48, 2
    if variant == "q8_f16norm_align64":
        spec.update(dt_gate_up=va.Q8_0, dt_down=va.Q8_0, dt_q=va.Q8_0, dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0,
                    dt_head=va.Q8_0, dt_embed=va.Q8_0)
        norm_dtype, alignment, ctx, seqs = va.F16, 64, 0, 1
    elif variant == "q4km_bf16norm_renorm0":
        # renormalize off with Qwen3's per-head norms: config.json says norm_topk_prob false
        norm_dtype = va.BF16
    elif variant == "mixed_dtypes":
        spec.update(dt_q=va.Q6_K, dt_k=va.Q8_0, dt_o=va.Q6_K, dt_embed=va.Q8_0, n_layers=3)
        ctx, seqs = 100, 3  # ctx beyond max_positions is cut to it, as the reference cuts it
    path = make(tmp_path, spec, 77, norm_dtype, alignment)
    if variant == "q4km_bf16norm_renorm0":
        cfgp = os.path.join(str(tmp_path), "config.json")
        with open(cfgp) as f:
            j = json.load(f)
        j["norm_topk_prob"] = False
        with open(cfgp, "w") as f:
            json.dump(j, f)
    ref = theirs(str(tmp_path), ctx, seqs)
    got = normalized(ours(path, ctx, seqs))
    assert got["info"] == ref["info"]
    assert got["tensors"] == ref["tensors"]
    assert got["model"] == ref["model"]


def test_reader_matches_committed_reference_description(tmp_path):
    """The fixed checkpoint's bytes are the ones the committed description was made from (SHA-256), and the
    library's reader describes it as the reference did."""
    spec, seed, norm_dtype, alignment, ctx, seqs = FIXED
    path = make(tmp_path, spec, seed, norm_dtype, alignment)
    with open(FIXTURE) as f:
        fx = json.load(f)
    with open(path, "rb") as f:
        assert hashlib.sha256(f.read()).hexdigest() == fx["sha256"]
    got = normalized(ours(path, ctx, seqs))
    ref = fx["reference"]
    assert got["info"] == ref["info"]
    assert got["tensors"] == ref["tensors"]
    assert got["model"] == ref["model"]


@needs_ref
def test_committed_description_is_the_reference_s(tmp_path):
    """The fixture is what the compiled reference prints for the fixed checkpoint today."""
    spec, seed, norm_dtype, alignment, ctx, seqs = FIXED
    make(tmp_path, spec, seed, norm_dtype, alignment)
    with open(FIXTURE) as f:
        fx = json.load(f)
    assert theirs(str(tmp_path), ctx, seqs) == fx["reference"]


def _patch(path, off, data):
    with open(path, "r+b") as f:
        f.seek(off)
        f.write(data)


def _find(path, needle):
    with open(path, "rb") as f:
        b = f.read()
    i = b.find(needle)
    assert i >= 0
    return i


@pytest.mark.parametrize("case,needle", [("magic", "not a GGUF file"), ("version", "GGUF version 4"),
                                         ("name", "is not one this engine knows"), ("llama", "permuted"),
                                         ("offset", "off its alignment"), ("dtype", "ggml type 2;"),
                                         ("truncated", "runs past the end"), ("wide", "rows too wide")])
def test_reader_refuses(tmp_path, case, needle):
    """The refusals the reference makes (engine/src/gguf.c:239-440), each on a damaged copy of a good file."""
    path = make(tmp_path, SMALL, 5, va.F32, 32)
    if case == "magic":
        _patch(path, 0, b"GGUX")
    elif case == "version":
        _patch(path, 4, struct.pack("<I", 4))
    elif case == "name":
        i = _find(path, b"blk.1.attn_q.weight")
        _patch(path, i, b"blk.1.attn_z.weight")
    elif case == "llama":
        # general.architecture's 8 bytes become "llama" and three NULs: read as a C string, the architecture is llama
        _patch(path, _find(path, b"qwen3moe"), b"llama\0\0\0")
    elif case == "offset":
        i = _find(path, b"output.weight")
        j = i + len(b"output.weight") + 4 + 16 + 4  # dims, two extents, type
        with open(path, "rb") as f:
            f.seek(j)
            off = struct.unpack("<Q", f.read(8))[0]
        _patch(path, j, struct.pack("<Q", off + 4))
    elif case == "dtype":
        i = _find(path, b"output.weight")
        _patch(path, i + len(b"output.weight") + 4 + 16, struct.pack("<I", 2))  # Q4_0
    elif case == "truncated":
        with open(path, "r+b") as f:
            f.truncate(1000)
    elif case == "wide":
        # a row width of 2^62 Q6_K weights: its byte count (2^54 * 210) wraps a 64-bit product to a small number
        i = _find(path, b"output.weight")
        _patch(path, i + len(b"output.weight") + 4, struct.pack("<Q", 1 << 62))
    with pytest.raises(va.VitnaError, match=needle):
        g = va.GgufModel(path)
        g.free()


def test_reader_survives_damaged_directories(tmp_path):
    """Random damage to the header, metadata and tensor directory of a good file (bit flips, random bytes,
    huge 64-bit values, truncation): the reader either refuses with a message or reads a file whose every tensor
    lies inside the mapping and binds or refuses the model, and never crashes. (An address-sanitized build of the
    reader with a C driver took 18,000 such files without a finding.)"""
    import random
    path = make(tmp_path, SMALL, 5, va.F32, 32)
    with open(path, "rb") as f:
        good = f.read()
    g = va.GgufModel(path)
    head = g.data_offset()
    g.free()
    rng = random.Random(20261202)
    bad_path = str(tmp_path / "damaged" / "model.gguf")
    os.makedirs(os.path.dirname(bad_path))
    os.link(os.path.join(os.path.dirname(path), "config.json"), os.path.join(os.path.dirname(bad_path), "config.json"))
    opened = refused = 0
    for _ in range(300):
        b = bytearray(good)
        for _ in range(rng.randint(1, 4)):
            p = rng.randrange(head)
            kind = rng.randrange(4)
            if kind == 0:
                b[p] ^= 1 << rng.randrange(8)
            elif kind == 1:
                b[p] = rng.randrange(256)
            elif kind == 2:
                b[p:p + 8] = b"\xff" * 7 + b"\x7f"
                del b[len(good):]
            else:
                del b[rng.randrange(1, len(b)):]
                break
        with open(bad_path, "wb") as f:
            f.write(b)
        try:
            m = va.GgufModel(bad_path)
        except va.VitnaError as e:
            assert str(e)
            refused += 1
            continue
        opened += 1
        start = m.data_offset()  # tensor offsets count from the data section
        for name, dt, nd, r, c, lo, hi in m.tensors():
            assert lo <= hi and start + hi <= len(b), name
        m.free()
    assert refused > 0 and opened > 0 and opened + refused == 300
