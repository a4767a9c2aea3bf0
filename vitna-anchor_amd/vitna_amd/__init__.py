"""Python side of vitna-anchor's MoE decode path on MI355X.

ctypes bindings to the C ABI in include/vitna_hip.h (libvitna_hip.so, built
from vitna-anchor_amd/csrc by vitna-anchor_amd/build.py) and to the seeded
synthetic-model generator (synth/libvitna_synth.so). The engine's own caller,
engine/src/model.c, calls the same functions from C; this module is how the
tests and bench.py call them.

Nothing here computes the path's arithmetic: every numeric result comes from
the HIP library. If the library is missing, loading fails loudly.
"""
import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)
HIP_LIB = os.environ.get("VITNA_HIP_LIB") or os.path.join(PKG, "libvitna_hip.so")
SYNTH_LIB = os.path.join(PKG, "synth", "libvitna_synth.so")

# vitna_dtype_t (include/vitna_model.h; engine/include/safetensors.h:23-45)
F32, F16, BF16 = 1, 2, 3
Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 14, 15, 16, 17, 18, 19
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), F32: (1, 4), F16: (1, 2), BF16: (1, 2)}


def row_bytes(dtype, cols):
    be, bb = BLOCK[dtype]
    assert cols % be == 0
    return cols // be * bb


class Config(C.Structure):
    _fields_ = [("n_layers", C.c_size_t), ("hidden", C.c_size_t), ("intermediate", C.c_size_t), ("n_heads", C.c_size_t),
                ("n_kv_heads", C.c_size_t), ("head_dim", C.c_size_t), ("vocab", C.c_size_t),
                ("max_positions", C.c_size_t), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("tied_embeddings", C.c_bool), ("qk_norm", C.c_bool), ("qk_norm_per_head", C.c_bool),
                ("n_experts", C.c_size_t), ("n_experts_used", C.c_size_t), ("renormalize", C.c_bool),
                ("qwen3", C.c_bool)]


class Matrix(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int), ("rows", C.c_size_t), ("cols", C.c_size_t)]

    def bytes(self):
        n = row_bytes(self.dtype, self.cols) * self.rows
        return np.ctypeslib.as_array(C.cast(self.data, C.POINTER(C.c_uint8)), shape=(n,))


class Expert(C.Structure):
    _fields_ = [("gate", Matrix), ("up", Matrix), ("down", Matrix)]


_FP = C.POINTER(C.c_float)


class Layer(C.Structure):
    _fields_ = [("attn_norm", _FP), ("mlp_norm", _FP), ("q", Matrix), ("k", Matrix), ("v", Matrix), ("o", Matrix),
                ("gate", Matrix), ("up", Matrix), ("down", Matrix), ("q_norm", _FP), ("k_norm", _FP),
                ("router", Matrix), ("experts", C.POINTER(Expert))]


class Llama(C.Structure):
    _fields_ = [("cfg", Config), ("shards", C.c_void_p), ("shard_paths", C.c_void_p), ("n_shards", C.c_size_t),
                ("embed", Matrix), ("lm_head", Matrix), ("final_norm", _FP), ("layers", C.POINTER(Layer)),
                ("inv_freq", _FP), ("ctx", C.c_size_t), ("seqs", C.c_size_t), ("past", C.POINTER(C.c_size_t)),
                ("k_cache", _FP), ("v_cache", _FP)] + \
               [(n, _FP) for n in ("x", "xn", "q", "k", "v", "att", "proj", "gate", "up", "scores", "cos_t", "sin_t",
                                   "router_logits", "expert_out")] + \
               [("stream", C.c_void_p), ("pred_xn", _FP), ("pred_logits", _FP), ("predicted", C.c_int32 * 64),
                ("predicted_layer", C.c_int64), ("predicted_right", C.c_uint64), ("predicted_total", C.c_uint64),
                ("trace_logits", _FP), ("trace_chosen", C.POINTER(C.c_int32)), ("trace_positions", C.c_size_t),
                ("pin", C.POINTER(C.c_int32)), ("pin_positions", C.c_size_t), ("cuda", C.c_void_p),
                ("rows_max", C.c_size_t), ("rows_logits", _FP), ("rows_next", _FP), ("rows_weights", _FP),
                ("rows_order", C.POINTER(C.c_int32)), ("rows_pred", C.POINTER(C.c_int32)), ("rows_chunk", C.c_void_p),
                ("rows_outs", C.c_void_p), ("no_rows", C.c_bool), ("gpu_kv_layers", C.c_int), ("gpu_fast", C.c_bool),
                ("device_lost", C.c_bool), ("device_error", C.c_char * 160), ("fail_armed", C.c_bool),
                ("fail_loses", C.c_bool), ("fail_at", C.c_size_t)]


class Shape(C.Structure):
    """vitna_synth_shape_t (synth/vitna_synth.h)."""
    _fields_ = [("n_layers", C.c_size_t), ("hidden", C.c_size_t), ("intermediate", C.c_size_t),
                ("n_heads", C.c_size_t), ("n_kv_heads", C.c_size_t), ("head_dim", C.c_size_t), ("vocab", C.c_size_t),
                ("n_experts", C.c_size_t), ("n_experts_used", C.c_size_t), ("renormalize", C.c_int),
                ("attention", C.c_int), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("dt_gate_up", C.c_int), ("dt_down", C.c_int), ("dt_q", C.c_int), ("dt_k", C.c_int), ("dt_v", C.c_int),
                ("dt_o", C.c_int), ("dt_head", C.c_int), ("dt_embed", C.c_int), ("router_std", C.c_float),
                ("q8_scale", C.c_float), ("k_scale", C.c_float), ("norm_std", C.c_float), ("ctx", C.c_size_t),
                ("seqs", C.c_size_t), ("kv_host", C.c_int)]


def shape(**kw):
    """A synthetic shape; unspecified fields take the Qwen3-30B-A3B-shaped defaults of BASELINE config 2."""
    d = dict(n_layers=48, hidden=2048, intermediate=768, n_heads=32, n_kv_heads=4, head_dim=128, vocab=151936,
             n_experts=128, n_experts_used=8, renormalize=1, attention=1, rms_eps=1e-6, rope_theta=1e6,
             dt_gate_up=Q4_K, dt_down=Q6_K, dt_q=Q4_K, dt_k=Q4_K, dt_v=Q6_K, dt_o=Q4_K, dt_head=Q6_K, dt_embed=Q4_K,
             router_std=0.02, q8_scale=0.02 / 127, k_scale=0.01, norm_std=0.05, ctx=4096, seqs=1, kv_host=0)
    d.update(kw)
    return Shape(**d)


# The five benchmark configurations of BASELINE.json, full size.
CONFIGS = {
    0: dict(n_layers=1, hidden=2048, intermediate=1024, n_experts=64, n_experts_used=8, renormalize=0, attention=0,
            rms_eps=1e-5, dt_gate_up=Q8_0, dt_down=Q8_0, norm_std=0.0),
    1: dict(n_layers=1, hidden=2048, intermediate=768, n_experts=128, n_experts_used=8, renormalize=1, attention=0,
            dt_gate_up=Q4_K, dt_down=Q6_K, norm_std=0.0),
    2: dict(),
    3: dict(seqs=32, ctx=8193),
    4: dict(n_layers=1, intermediate=768, n_experts=128, n_experts_used=8, renormalize=1, attention=0,
            dt_gate_up=Q8_0, dt_down=Q8_0, norm_std=0.0),
}


def _synth():
    if not os.path.exists(SYNTH_LIB):
        raise RuntimeError("%s is not built: run python vitna-anchor_amd/build.py" % SYNTH_LIB)
    lib = C.CDLL(SYNTH_LIB)
    lib.vitna_synth_model.restype = C.POINTER(Llama)
    lib.vitna_synth_model.argtypes = [C.POINTER(Shape), C.c_uint64, C.c_int, C.c_char_p, C.c_size_t]
    lib.vitna_synth_free.argtypes = [C.POINTER(Llama)]
    lib.vitna_synth_normal.argtypes = [C.c_uint64, C.c_uint64, _FP, C.c_size_t]
    lib.vitna_synth_matrix.argtypes = [C.c_int, C.c_uint64, C.c_uint64, C.c_size_t, C.c_size_t, C.c_float, C.c_void_p,
                                       C.c_int]
    lib.vitna_synth_write_gguf.argtypes = [C.POINTER(Llama), C.c_char_p, C.c_int, C.c_uint32, C.c_char_p, C.c_size_t]
    lib.vitna_synth_f32_to_f16.restype = C.c_uint16
    lib.vitna_synth_f32_to_f16.argtypes = [C.c_float]
    return lib


_synth_lib = None


def synth():
    global _synth_lib
    if _synth_lib is None:
        _synth_lib = _synth()
    return _synth_lib


def fptr(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_FP)


def normal(seed, tag, n):
    out = np.empty(n, dtype=np.float32)
    synth().vitna_synth_normal(seed, tag, fptr(out), n)
    return out


def synth_matrix(dtype, seed, tag, rows, cols, scale, threads=8):
    out = np.empty(rows * row_bytes(dtype, cols), dtype=np.uint8)
    rc = synth().vitna_synth_matrix(dtype, seed, tag, rows, cols, scale, out.ctypes.data_as(C.c_void_p), threads)
    if rc:
        raise ValueError("unsupported matrix for the generator")
    return out


class Model:
    """A seeded synthetic model (host memory), laid out as the engine's vitna_llama_t."""

    def __init__(self, shp, seed, threads=16):
        err = C.create_string_buffer(512)
        self.shape = shp
        self.seed = seed
        self.ptr = synth().vitna_synth_model(C.byref(shp), seed, threads, err, 512)
        if not self.ptr:
            raise RuntimeError(err.value.decode(errors="replace"))
        self.m = self.ptr.contents

    @property
    def cfg(self):
        return self.m.cfg

    def rope_tables(self):
        """cos/sin of every position, [ctx][head_dim/2], as engine/src/model.c:1213-1232 computes them (float32 angle, libm)."""
        hd = self.cfg.head_dim
        half = hd // 2
        inv = np.ctypeslib.as_array(self.m.inv_freq, shape=(half,)).copy()
        pos = np.arange(self.m.ctx, dtype=np.float32)[:, None]
        ang = (pos * inv[None, :]).astype(np.float32)
        # libm's cosf/sinf via the C library, element by element, for exactness
        libm = C.CDLL("libm.so.6")
        libm.cosf.restype = C.c_float
        libm.cosf.argtypes = [C.c_float]
        libm.sinf.restype = C.c_float
        libm.sinf.argtypes = [C.c_float]
        flat = ang.ravel()
        cs = np.fromiter((libm.cosf(float(a)) for a in flat), dtype=np.float32, count=flat.size).reshape(ang.shape)
        sn = np.fromiter((libm.sinf(float(a)) for a in flat), dtype=np.float32, count=flat.size).reshape(ang.shape)
        return np.ascontiguousarray(cs), np.ascontiguousarray(sn)

    def free(self):
        if self.ptr:
            synth().vitna_synth_free(self.ptr)
            self.ptr = None


class VitnaError(RuntimeError):
    pass


def write_gguf(model, directory, norm_dtype=F32, alignment=32):
    """model (a synthetic Model) written into directory as model.gguf and config.json."""
    err = C.create_string_buffer(512)
    if synth().vitna_synth_write_gguf(model.ptr, directory.encode(), norm_dtype, alignment, err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return os.path.join(directory, "model.gguf")


class GgufInfo(C.Structure):
    """vitna_hip_gguf_info_t (include/vitna_gguf.h)."""
    _fields_ = [("arch", C.c_char * 64), ("version", C.c_uint32), ("alignment", C.c_uint64)] + \
               [(n, C.c_uint64) for n in ("block_count", "embedding_length", "feed_forward_length",
                                          "expert_feed_forward_length", "head_count", "head_count_kv", "key_length",
                                          "context_length", "expert_count", "expert_used_count")] + \
               [("rms_eps", C.c_double), ("rope_freq_base", C.c_double), ("file_tensors", C.c_size_t),
                ("split_no", C.c_uint16), ("split_count", C.c_uint16), ("split_tensors_count", C.c_uint64)]


class GgufTensor(C.Structure):
    """vitna_hip_gguf_tensor_t (include/vitna_gguf.h)."""
    _fields_ = [("name", C.c_char * 256), ("dtype", C.c_int), ("ndim", C.c_size_t), ("shape", C.c_size_t * 2),
                ("offset_begin", C.c_uint64), ("offset_end", C.c_uint64), ("data", C.c_void_p)]


def config_from_json(path):
    """The engine's config from a checkpoint's config.json, as engine/src/model.c:54-137 (read_config) reads it for
    the mixture-of-experts models (model_type olmoe or qwen3_moe); other model types are refused."""
    import json
    with open(path) as f:
        j = json.load(f)
    mt = j.get("model_type")
    if mt not in ("olmoe", "qwen3_moe"):
        raise VitnaError("config.json: model_type is %s, and only olmoe and qwen3_moe are served" % mt)
    if j.get("hidden_act") != "silu":
        raise VitnaError("config.json: hidden_act is %s, and only silu is supported" % j.get("hidden_act"))
    qwen3 = mt == "qwen3_moe"
    c = Config()
    c.n_layers = j["num_hidden_layers"]
    c.hidden = j["hidden_size"]
    c.intermediate = j["moe_intermediate_size"] if qwen3 else j["intermediate_size"]
    c.n_heads = j["num_attention_heads"]
    c.vocab = j["vocab_size"]
    c.max_positions = j["max_position_embeddings"]
    c.n_kv_heads = j.get("num_key_value_heads", c.n_heads)
    c.head_dim = j.get("head_dim", c.hidden // c.n_heads)
    if c.n_heads % c.n_kv_heads or c.head_dim % 2:
        raise VitnaError("config.json: heads do not divide into key-value groups, or head_dim is odd")
    c.n_experts = j["num_experts"]
    c.n_experts_used = j["num_experts_per_tok"]
    c.rms_eps = float(j.get("rms_norm_eps", 1e-6 if qwen3 else 1e-5))
    c.rope_theta = float(j.get("rope_theta", 10000.0))
    c.tied_embeddings = bool(j.get("tie_word_embeddings", False))
    c.qk_norm = True
    c.qk_norm_per_head = qwen3
    c.qwen3 = qwen3
    c.renormalize = bool(j.get("norm_topk_prob", False))
    return c


class GgufModel:
    """A GGUF checkpoint (model.gguf with its config.json) read by the library's GGUF reader into the engine's
    vitna_llama_t: the same interface as Model (ptr, m, cfg, rope_tables, free), so Device and the checker take it."""

    def __init__(self, path, ctx=0, seqs=1, config=None):
        lib = hip()
        self.err = C.create_string_buffer(512)
        self.info = GgufInfo()
        self.g = lib.vitna_hip_gguf_open(path.encode(), C.byref(self.info), self.err, 512)
        if not self.g:
            raise VitnaError(self.err.value.decode(errors="replace"))
        cfg = config if config is not None else config_from_json(os.path.join(os.path.dirname(path), "config.json"))
        self._llama = Llama()
        if not lib.vitna_hip_gguf_llama(self.g, C.byref(cfg), ctx, seqs, C.byref(self._llama), self.err, 512):
            lib.vitna_hip_gguf_close(self.g)
            self.g = None
            raise VitnaError(self.err.value.decode(errors="replace"))
        self.ptr = C.pointer(self._llama)
        self.m = self._llama

    cfg = Model.cfg
    rope_tables = Model.rope_tables

    def tensors(self):
        """The directory: (name, dtype, ndim, shape0, shape1, offset_begin, offset_end) per tensor."""
        lib = hip()
        out = []
        t = GgufTensor()
        for i in range(lib.vitna_hip_gguf_count(self.g)):
            assert lib.vitna_hip_gguf_tensor(self.g, i, C.byref(t))
            out.append((t.name.decode(), t.dtype, t.ndim, t.shape[0], t.shape[1] if t.ndim > 1 else 0, t.offset_begin,
                        t.offset_end))
        return out

    def data_offset(self):
        return hip().vitna_hip_gguf_data_offset(self.g)

    def free(self):
        if self.g:
            hip().vitna_hip_gguf_llama_free(C.byref(self._llama))
            hip().vitna_hip_gguf_close(self.g)
            self.g = None


class RowT(C.Structure):
    _fields_ = [("token", C.c_int32), ("pos", C.c_int32), ("seq", C.c_int32)]


def _hip():
    if not os.path.exists(HIP_LIB):
        raise RuntimeError("%s is not built: the HIP path has no fallback. Run python vitna-anchor_amd/build.py" % HIP_LIB)
    lib = C.CDLL(HIP_LIB)
    E = (C.c_char_p, C.c_size_t)
    P = C.c_void_p
    sig = {
        "vitna_cuda_probe": (C.c_bool, [*E]),
        "vitna_cuda_create": (P, [C.POINTER(Llama), _FP, _FP, C.c_size_t, *E]),
        "vitna_cuda_free": (None, [P]),
        "vitna_cuda_moe_route": (C.c_bool, [P, C.c_size_t, C.c_int32, C.c_size_t, C.c_size_t, _FP, _FP, *E]),
        "vitna_cuda_moe_experts": (C.c_bool, [P, C.c_size_t, C.POINTER(C.c_int32), _FP, C.c_size_t, C.POINTER(C.c_int32),
                                              *E]),
        "vitna_cuda_moe_head": (C.c_bool, [P, _FP, *E]),
        "vitna_cuda_moe_rows_max": (C.c_size_t, [P]),
        "vitna_cuda_moe_rows_route": (C.c_bool, [P, C.POINTER(RowT), C.c_size_t, C.c_size_t, _FP, _FP, *E]),
        "vitna_cuda_moe_rows_experts": (C.c_bool, [P, C.c_size_t, C.c_size_t, C.POINTER(C.c_int32), _FP, C.c_size_t,
                                                   C.POINTER(C.c_int32), *E]),
        "vitna_cuda_moe_rows_head": (C.c_bool, [P, C.c_size_t, C.POINTER(_FP), *E]),
        "vitna_cuda_widen": (C.c_bool, [C.POINTER(Matrix), _FP, *E]),
        "vitna_cuda_expert_check": (C.c_bool, [C.POINTER(Matrix), C.POINTER(Matrix), C.POINTER(Matrix), _FP, _FP,
                                               C.c_float, _FP, _FP, _FP, *E]),
        "vitna_cuda_lost": (C.c_bool, [P, *E]),
        "vitna_cuda_device_name": (C.c_char_p, [P]),
        "vitna_hip_moe_step": (C.c_bool, [P, C.c_size_t, C.c_int32, C.c_size_t, _FP, *E]),
        "vitna_hip_moe_step_async": (C.c_bool, [P, C.c_size_t, C.c_int32, C.c_size_t, *E]),
        "vitna_hip_moe_ffn": (C.c_bool, [P, C.c_size_t, *E]),
        "vitna_hip_moe_rows_step": (C.c_bool, [P, C.POINTER(RowT), C.c_size_t, C.POINTER(_FP), *E]),
        "vitna_hip_residual": (C.c_bool, [P, C.c_size_t, _FP, C.c_bool, *E]),
        "vitna_hip_rows_project": (C.c_bool, [P, C.c_size_t, C.c_int, _FP, C.c_size_t, _FP, *E]),
        "vitna_hip_routing": (C.c_bool, [P, C.c_size_t, _FP, C.POINTER(C.c_int32), C.POINTER(C.c_int32), _FP, *E]),
        "vitna_hip_step_routing": (C.c_bool, [P, C.c_size_t, C.POINTER(C.c_int32), C.POINTER(C.c_int32), _FP, *E]),
        "vitna_hip_rows_routing": (C.c_bool, [P, C.c_size_t, C.c_size_t, C.POINTER(C.c_int32), C.POINTER(C.c_int32), _FP,
                                              *E]),
        "vitna_cuda_test_fast_rows": (None, [P, C.c_size_t]),
        "vitna_hip_attention_io": (C.c_bool, [P, C.c_size_t, _FP, _FP, *E]),
        "vitna_hip_gguf_open": (P, [C.c_char_p, C.POINTER(GgufInfo), *E]),
        "vitna_hip_gguf_count": (C.c_size_t, [P]),
        "vitna_hip_gguf_tensor": (C.c_bool, [P, C.c_size_t, C.POINTER(GgufTensor)]),
        "vitna_hip_gguf_data_offset": (C.c_uint64, [P]),
        "vitna_hip_gguf_llama": (C.c_bool, [P, C.POINTER(Config), C.c_size_t, C.c_size_t, C.POINTER(Llama), *E]),
        "vitna_hip_gguf_llama_free": (None, [C.POINTER(Llama)]),
        "vitna_hip_gguf_close": (None, [P]),
        "vitna_hip_set_step_kernel": (C.c_bool, [P, C.c_int, C.POINTER(C.c_int), *E]),
        "vitna_hip_set_exact_rows": (C.c_bool, [P, C.c_size_t, *E]),
        "vitna_hip_step_trace": (C.c_bool, [P, C.c_size_t, C.c_int32, C.c_size_t, C.c_int, C.POINTER(C.c_uint64),
                                             C.c_size_t, *E]),
        "vitna_hip_kv": (C.c_bool, [P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, _FP, _FP, C.c_bool, *E]),
        "vitna_hip_kv_fill": (C.c_bool, [P, C.c_uint64, C.POINTER(C.c_size_t), *E]),
        "vitna_hip_sync": (C.c_bool, [P, *E]),
        "vitna_hip_stream": (P, [P]),
        "vitna_hip_moe_prefill": (C.c_bool, [P, C.c_size_t, _FP, C.c_size_t, C.POINTER(C.c_int32), *E]),
        "vitna_hip_moe_prefill_noalloc": (C.c_bool, [P, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p, *E]),
        "vitna_hip_time_prefill": (C.c_bool, [P, C.c_size_t, C.c_size_t, C.c_uint64, C.c_int, C.POINTER(C.c_double),
                                              C.POINTER(C.c_double), *E]),
        "vitna_hip_time_rows": (C.c_bool, [P, C.POINTER(RowT), C.c_size_t, C.c_int, C.POINTER(C.c_double), *E]),
        "vitna_hip_prefill_rows": (C.c_bool, [P, C.c_size_t, _FP, _FP, C.POINTER(C.c_int32), *E]),
        "vitna_hip_route_check": (C.c_bool, [_FP, C.c_int, C.c_int, C.c_bool, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                             _FP, *E]),
        "vitna_hip_host_route": (C.c_bool, [_FP, C.c_int, C.c_int, C.c_bool, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                            _FP, *E]),
        "vitna_hip_expert_cache_state": (C.c_bool, [P, C.POINTER(C.c_int32), C.c_size_t, C.POINTER(C.c_uint64), *E]),
        "vitna_cuda_moe_report": (C.c_char_p, [P, C.c_char_p, C.c_size_t]),
        "vitna_hip_copy_probe": (C.c_bool, [C.c_size_t, C.c_int, C.POINTER(C.c_double), *E]),
        "vitna_hip_mfma_probe": (C.c_bool, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double), *E]),
        "vitna_hip_time_steps": (C.c_bool, [P, C.c_size_t, C.c_int32, C.c_size_t, C.c_int, C.POINTER(C.c_double), *E]),
        "vitna_hip_time_ffn": (C.c_bool, [P, C.c_int, C.POINTER(C.c_double), *E]),
        "vitna_hip_time_kernel": (C.c_bool, [P, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double),
                                             C.POINTER(C.c_double), *E]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_hip_lib = None


def hip():
    global _hip_lib
    if _hip_lib is None:
        _hip_lib = _hip()
    return _hip_lib


def _i32(a):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


class Device:
    """A model uploaded to the GPU through vitna_cuda_create."""

    def __init__(self, model, expert_cache_bytes=0, fast=False):
        """expert_cache_bytes: 0 keeps every expert resident; fewer bytes than the experts take puts them behind a
        cache of slots (the reference's expert cache), served by moe_route / moe_experts. fast: the model's gpu_fast
        (the reference's --precision fast): passes of 64 rows or more run their experts as the grouped GEMM."""
        self.model = model
        model.m.gpu_fast = bool(fast)
        self.lib = hip()
        self.err = C.create_string_buffer(512)
        cfg = model.cfg
        if cfg.n_heads:
            self.cos, self.sin = model.rope_tables()
            c, s = fptr(self.cos), fptr(self.sin)
        else:
            c = s = None
        self.g = self.lib.vitna_cuda_create(model.ptr, c, s, expert_cache_bytes, self.err, 512)
        if not self.g:
            raise VitnaError(self.err.value.decode(errors="replace"))

    def _ok(self, ok):
        if not ok:
            raise VitnaError(self.err.value.decode(errors="replace"))

    def close(self):
        if self.g:
            self.lib.vitna_cuda_free(self.g)
            self.g = None

    # --- the reference's ABI ---
    def moe_route(self, seq, token, pos, layer, want_next=False):
        E = self.model.cfg.n_experts
        lg = np.empty(E, np.float32)
        nx = np.empty(E, np.float32) if want_next else None
        self._ok(self.lib.vitna_cuda_moe_route(self.g, seq, token, pos, layer, fptr(lg), fptr(nx) if want_next else None,
                                               self.err, 512))
        return (lg, nx) if want_next else lg

    def moe_experts(self, layer, ids, weights, guess=None):
        ids = np.ascontiguousarray(ids, np.int32)
        w = np.ascontiguousarray(weights, np.float32)
        gs = None if guess is None else np.ascontiguousarray(guess, np.int32)
        self._ok(self.lib.vitna_cuda_moe_experts(self.g, layer, _i32(ids), fptr(w), ids.size, None if gs is None else _i32(gs),
                                                 self.err, 512))

    def moe_report(self):
        buf = C.create_string_buffer(1024)
        return self.lib.vitna_cuda_moe_report(self.g, buf, 1024).decode()

    def expert_cache_state(self):
        """(where[n_layers * E], counters dict) of the expert cache."""
        cfg = self.model.cfg
        where = np.empty(cfg.n_layers * cfg.n_experts, np.int32)
        cnt = (C.c_uint64 * 10)()
        self._ok(self.lib.vitna_hip_expert_cache_state(self.g, _i32(where), where.size, cnt, self.err, 512))
        keys = ("slots", "slot_bytes", "acquired", "hits", "in_flight", "misses", "prefetched", "prefetch_used", "copies",
                "bytes_copied")
        return where, dict(zip(keys, [int(v) for v in cnt]))

    def moe_head(self):
        out = np.empty(self.model.cfg.vocab, np.float32)
        self._ok(self.lib.vitna_cuda_moe_head(self.g, fptr(out), self.err, 512))
        return out

    # --- extensions ---
    def step(self, seq, token, pos, logits=True):
        out = np.empty(self.model.cfg.vocab, np.float32) if logits else None
        self._ok(self.lib.vitna_hip_moe_step(self.g, seq, token, pos, fptr(out) if logits else None, self.err, 512))
        return out

    # --- several rows a layer at a time (the ABI's rows_*) ---
    @staticmethod
    def _rows(rows):
        arr = (RowT * len(rows))()
        for i, (tok, pos, seq) in enumerate(rows):
            arr[i].token, arr[i].pos, arr[i].seq = tok, pos, seq
        return arr

    def rows_route(self, rows, layer, want_next=False):
        E = self.model.cfg.n_experts
        n = len(rows)
        lg = np.empty((n, E), np.float32)
        nx = np.empty((n, E), np.float32) if want_next else None
        self._ok(self.lib.vitna_cuda_moe_rows_route(self.g, self._rows(rows), n, layer, fptr(lg),
                                                    fptr(nx) if want_next else None, self.err, 512))
        return (lg, nx) if want_next else lg

    def rows_experts(self, layer, ids, weights, guess=None):
        ids = np.ascontiguousarray(ids, np.int32)
        w = np.ascontiguousarray(weights, np.float32)
        n, k = ids.shape
        g = None
        if guess is not None:
            g = np.ascontiguousarray(guess, np.int32)
            if g.shape != ids.shape:
                raise ValueError("a guess of %d experts for each of %d rows" % (k, n))
        self._ok(self.lib.vitna_cuda_moe_rows_experts(self.g, layer, n, _i32(ids), fptr(w), k,
                                                      _i32(g) if g is not None else None, self.err, 512))

    def rows_head(self, n, only=None):
        """logits of every row, or (only) of the rows it lists: the others' pointers NULL, their rows unset."""
        V = self.model.cfg.vocab
        out = np.empty((n, V), np.float32)
        want = set(range(n)) if only is None else set(only)
        ptrs = (_FP * n)(*[out[i].ctypes.data_as(_FP) if i in want else None for i in range(n)])
        self._ok(self.lib.vitna_cuda_moe_rows_head(self.g, n, ptrs, self.err, 512))
        return out

    def rows_step(self, rows, logits=True, only=None):
        """logits of every row (or, with only, of the rows it lists, the others' pointers NULL: their rows of the
        result stay unset) or none."""
        n = len(rows)
        out = np.empty((n, self.model.cfg.vocab), np.float32) if logits else None
        want = set(range(n)) if only is None else set(only)
        ptrs = (_FP * n)(*[out[i].ctypes.data_as(_FP) if i in want else None for i in range(n)]) if logits else None
        self._ok(self.lib.vitna_hip_moe_rows_step(self.g, self._rows(rows), n, ptrs, self.err, 512))
        return out

    def step_async(self, seq, token, pos):
        self._ok(self.lib.vitna_hip_moe_step_async(self.g, seq, token, pos, self.err, 512))

    def ffn(self, layer):
        self._ok(self.lib.vitna_hip_moe_ffn(self.g, layer, self.err, 512))

    def set_residual(self, x, row=0):
        x = np.ascontiguousarray(x, np.float32)
        self._ok(self.lib.vitna_hip_residual(self.g, row, fptr(x), True, self.err, 512))

    def rows_project(self, layer, which, x):
        """y = W x for n rows x (n x cols), W = layer's q, k, v, o (which 0..3) or the head (4), on the multi-row
        kernels of a rows step."""
        cfg = self.model.cfg
        qd, kd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        rows = [qd, kd, kd, cfg.hidden, cfg.vocab][which]
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], rows), np.float32)
        self._ok(self.lib.vitna_hip_rows_project(self.g, layer, which, fptr(x), x.shape[0], fptr(y), self.err, 512))
        return y

    def residual(self, row=0):
        x = np.empty(self.model.cfg.hidden, np.float32)
        self._ok(self.lib.vitna_hip_residual(self.g, row, fptr(x), False, self.err, 512))
        return x

    def routing(self, row=0):
        cfg = self.model.cfg
        lg = np.empty(cfg.n_experts, np.float32)
        ch = np.empty(cfg.n_experts_used, np.int32)
        ids = np.empty(cfg.n_experts_used, np.int32)
        w = np.empty(cfg.n_experts_used, np.float32)
        self._ok(self.lib.vitna_hip_routing(self.g, row, fptr(lg), _i32(ch), _i32(ids), fptr(w), self.err, 512))
        return lg, ch, ids, w

    def step_routing(self, layer):
        """(chosen largest first, ids in order, weights) of layer in the last device-routed step."""
        K = self.model.cfg.n_experts_used
        ch = np.empty(K, np.int32)
        ids = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        self._ok(self.lib.vitna_hip_step_routing(self.g, layer, _i32(ch), _i32(ids), fptr(w), self.err, 512))
        return ch, ids, w

    def rows_routing(self, layer, row):
        """(chosen largest first, ids in order, weights) of row at layer in the last device-routed rows step."""
        K = self.model.cfg.n_experts_used
        ch = np.empty(K, np.int32)
        ids = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        self._ok(self.lib.vitna_hip_rows_routing(self.g, layer, row, _i32(ch), _i32(ids), fptr(w), self.err, 512))
        return ch, ids, w

    def rows_max(self):
        return int(self.lib.vitna_cuda_moe_rows_max(self.g))

    def test_fast_rows(self, n):
        """The reference's test hook: on a fast model, passes of n rows or more take the grouped GEMM."""
        self.lib.vitna_cuda_test_fast_rows(self.g, n)

    def attention_io(self, row=0):
        """(q before its norm and rotation, attention output) of row at the last layer of the last step or pass."""
        cfg = self.model.cfg
        qd = cfg.n_heads * cfg.head_dim
        q = np.empty(qd, np.float32)
        att = np.empty(qd, np.float32)
        self._ok(self.lib.vitna_hip_attention_io(self.g, row, fptr(q), fptr(att), self.err, 512))
        return q, att

    def set_exact_rows(self, n):
        """Passes of the rows ABI of at most n rows take the single-token kernels (vitna_hip_set_exact_rows)."""
        self._ok(self.lib.vitna_hip_set_exact_rows(self.g, n, self.err, 512))

    def set_step_kernel(self, on):
        """Decode steps on the persistent step kernel (on) or the per-layer graph (off, the default); returns
        whether the model's shape takes the persistent kernel (vitna_hip_set_step_kernel)."""
        taken = C.c_int(0)
        self._ok(self.lib.vitna_hip_set_step_kernel(self.g, 1 if on else 0, C.byref(taken), self.err, 512))
        return bool(taken.value)

    def step_trace(self, seq, token, pos, block=0):
        """[layers, 6 phases, 3 stamps] s_memrealtime readings (100 MHz) of one traced step (vitna_hip_step_trace)."""
        L = self.model.cfg.n_layers
        out = np.zeros(L * 32, np.uint64)
        self._ok(self.lib.vitna_hip_step_trace(self.g, seq, token, pos, block, out.ctypes.data_as(C.POINTER(C.c_uint64)),
                                               out.size, self.err, 512))
        return out.reshape(L, 32)[:, :18].reshape(L, 6, 3)

    def kv(self, seq, layer, pos0, n, k=None, v=None):
        cfg = self.model.cfg
        kd = cfg.n_kv_heads * cfg.head_dim
        if k is None:
            k = np.empty((n, kd), np.float32)
            v = np.empty((n, kd), np.float32)
            self._ok(self.lib.vitna_hip_kv(self.g, seq, layer, pos0, n, fptr(k), fptr(v), False, self.err, 512))
            return k, v
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self._ok(self.lib.vitna_hip_kv(self.g, seq, layer, pos0, n, fptr(k), fptr(v), True, self.err, 512))

    def kv_fill(self, seed, n_pos):
        arr = (C.c_size_t * len(n_pos))(*n_pos)
        self._ok(self.lib.vitna_hip_kv_fill(self.g, seed, arr, self.err, 512))

    def sync(self):
        self._ok(self.lib.vitna_hip_sync(self.g, self.err, 512))

    def prefill(self, layer, x):
        """x (n x hidden) through the MoE half of layer on the device: (x + moe(x), experts chosen n x K)."""
        x = np.array(x, np.float32, order="C", copy=True)
        ch = np.empty((x.shape[0], self.model.cfg.n_experts_used), np.int32)
        self._ok(self.lib.vitna_hip_moe_prefill(self.g, layer, fptr(x), x.shape[0], _i32(ch), self.err, 512))
        return x, ch

    def prefill_noalloc(self, layer, x_dev, n, chosen_dev=None):
        """vitna_hip_moe_prefill_noalloc on device addresses (x_dev: n x hidden fp32, in place; chosen_dev: n x K
        int32 or None); asynchronous on the model's stream."""
        self._ok(self.lib.vitna_hip_moe_prefill_noalloc(self.g, layer, x_dev, n, chosen_dev, self.err, 512))

    def time_prefill(self, layer, n, seed=1, reps=10):
        """(total us, [norm + router, routing + grouping, gate/up, down, ordered sum] us) of a prefill of n rows."""
        tot = C.c_double()
        ph = (C.c_double * 5)()
        self._ok(self.lib.vitna_hip_time_prefill(self.g, layer, n, seed, reps, C.byref(tot), ph, self.err, 512))
        return tot.value, list(ph)

    def prefill_rows(self, n):
        """(input rows, output rows, chosen) of the first n rows of the last prefill on the device."""
        H, K = self.model.cfg.hidden, self.model.cfg.n_experts_used
        xi = np.empty((n, H), np.float32)
        xo = np.empty((n, H), np.float32)
        ch = np.empty((n, K), np.int32)
        self._ok(self.lib.vitna_hip_prefill_rows(self.g, n, fptr(xi), fptr(xo), _i32(ch), self.err, 512))
        return xi, xo, ch

    def time_kernel(self, which, reps, warmup=3):
        us = C.c_double()
        b = C.c_double()
        self._ok(self.lib.vitna_hip_time_kernel(self.g, which, reps, warmup, C.byref(us), C.byref(b), self.err, 512))
        return us.value, b.value

    def time_ffn(self, reps):
        """Mean microseconds of one layer's mixture-of-experts half, every layer in turn in one graph."""
        us = C.c_double()
        self._ok(self.lib.vitna_hip_time_ffn(self.g, reps, C.byref(us), self.err, 512))
        return us.value

    def time_steps(self, seq, token, pos, steps):
        ms = C.c_double()
        self._ok(self.lib.vitna_hip_time_steps(self.g, seq, token, pos, steps, C.byref(ms), self.err, 512))
        return ms.value

    def time_rows(self, rows, steps):
        """Milliseconds a rows step (device routing and grouping, logits left in HBM) of these rows."""
        ms = C.c_double()
        self._ok(self.lib.vitna_hip_time_rows(self.g, self._rows(rows), len(rows), steps, C.byref(ms), self.err, 512))
        return ms.value

    def device_name(self):
        return self.lib.vitna_cuda_device_name(self.g).decode()


def widen(matrix):
    """vitna_cuda_widen: the matrix widened to float32 on the GPU (two independent reads, required to agree)."""
    lib = hip()
    out = np.empty(matrix.rows * matrix.cols, np.float32)
    err = C.create_string_buffer(512)
    if not lib.vitna_cuda_widen(C.byref(matrix), fptr(out), err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return out.reshape(matrix.rows, matrix.cols)


def expert_check(gate, up, down, norm_w, x, eps):
    lib = hip()
    H, I = gate.cols, gate.rows
    xs = np.empty(H, np.float32)
    act = np.empty(I, np.float32)
    y = np.empty(H, np.float32)
    err = C.create_string_buffer(512)
    nw = np.ascontiguousarray(norm_w, np.float32)
    xx = np.ascontiguousarray(x, np.float32)
    if not lib.vitna_cuda_expert_check(C.byref(gate), C.byref(up), C.byref(down), fptr(nw), fptr(xx), eps, fptr(xs),
                                       fptr(act), fptr(y), err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return xs, act, y


def copy_probe(nbytes, reps=10):
    """vitna_hip_copy_probe: average microseconds of a plain device copy of nbytes."""
    us = C.c_double()
    err = C.create_string_buffer(512)
    if not hip().vitna_hip_copy_probe(nbytes, reps, C.byref(us), err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return us.value


def mfma_probe(blocks=1024, iters=2000, reps=3):
    """vitna_hip_mfma_probe: dense bf16 TFLOP/s of back-to-back 32x32x16 MFMAs on this device."""
    tf = C.c_double()
    err = C.create_string_buffer(512)
    if not hip().vitna_hip_mfma_probe(blocks, iters, reps, C.byref(tf), err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return tf.value


def host_route(logits, k, renormalize):
    """vitna_hip_host_route: the reference's host routing of the given logits -> (chosen, order, weights)."""
    lg = np.ascontiguousarray(logits, np.float32)
    ch = np.empty(k, np.int32)
    order = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    err = C.create_string_buffer(512)
    if not hip().vitna_hip_host_route(fptr(lg), lg.size, k, renormalize, _i32(ch), _i32(order), fptr(w), err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return ch, order, w


def route_check(logits, k, renormalize):
    """vitna_hip_route_check: the device's routing of the given logits -> (chosen, ids, weights)."""
    lib = hip()
    lg = np.ascontiguousarray(logits, np.float32)
    ch = np.empty(k, np.int32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    err = C.create_string_buffer(512)
    if not lib.vitna_hip_route_check(fptr(lg), lg.size, k, renormalize, _i32(ch), _i32(ids), fptr(w), err, 512):
        raise VitnaError(err.value.decode(errors="replace"))
    return ch, ids, w


def matrix_from_bytes(buf, dtype, rows, cols):
    """A Matrix over a numpy byte buffer (kept alive by the caller)."""
    return Matrix(buf.ctypes.data_as(C.c_void_p), dtype, rows, cols)
