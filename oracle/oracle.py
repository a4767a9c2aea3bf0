"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU parity checker
(oracle/liboracle.so, built from vitna_oracle.c). Imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libvitna_ref.so")

_FP = C.POINTER(C.c_float)
_IP = C.POINTER(C.c_int32)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError("oracle/liboracle.so is not built: make -C oracle")
        L = C.CDLL(LIB)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_widen.argtypes = [C.c_void_p, C.c_int, _FP, C.c_size_t]
        L.orc_matvec.argtypes = [C.c_void_p, C.c_int, _FP, _FP, C.c_size_t, C.c_size_t]
        L.orc_matvec_mt.argtypes = [C.c_void_p, C.c_int, _FP, _FP, C.c_size_t, C.c_size_t, C.c_int]
        L.orc_rmsnorm.argtypes = [_FP, _FP, _FP, C.c_size_t, C.c_float]
        L.orc_silu_mul.argtypes = [_FP, _FP, _FP, C.c_size_t]
        L.orc_top_k.argtypes = [_FP, C.c_size_t, C.c_size_t, _IP]
        L.orc_route.argtypes = [_FP, C.c_size_t, C.c_size_t, C.c_bool, _IP, _IP, _FP]
        L.orc_moe.argtypes = [C.c_void_p, C.c_size_t, _FP, _FP, _IP, _IP, _FP, _FP, C.c_int]
        L.orc_step.argtypes = [C.c_void_p, C.c_size_t, C.c_int32, C.c_size_t, _FP, _FP, _IP, _FP, C.c_int]
        _lib = L
    return _lib


def _f(a):
    return a.ctypes.data_as(_FP)


def _i(a):
    return a.ctypes.data_as(_IP)


def widen(buf, dtype, n):
    out = np.empty(n, np.float32)
    if lib().orc_widen(buf.ctypes.data_as(C.c_void_p), dtype, _f(out), n):
        raise ValueError("dtype")
    return out


def matvec(buf, dtype, x, rows, cols, threads=1):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    ptr = buf if isinstance(buf, int) else buf.ctypes.data_as(C.c_void_p)
    if lib().orc_matvec_mt(ptr, dtype, _f(x), _f(y), rows, cols, threads):
        raise ValueError("dtype")
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_f(x), _f(w), _f(y), x.size, eps)
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    o = np.empty_like(g)
    lib().orc_silu_mul(_f(g), _f(u), _f(o), g.size)
    return o


def top_k(logits, k):
    logits = np.ascontiguousarray(logits, np.float32)
    out = np.empty(k, np.int32)
    lib().orc_top_k(_f(logits), logits.size, k, _i(out))
    return out


def route(logits, k, renormalize):
    logits = np.ascontiguousarray(logits, np.float32)
    ch = np.empty(k, np.int32)
    order = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().orc_route(_f(logits), logits.size, k, renormalize, _i(ch), _i(order), _f(w))
    return ch, order, w


def moe(model, layer, xn, threads=1):
    """One layer's mixture of experts on normalized xn: (router logits, chosen, order, weights, proj)."""
    cfg = model.cfg
    xn = np.ascontiguousarray(xn, np.float32)
    lg = np.empty(cfg.n_experts, np.float32)
    ch = np.empty(cfg.n_experts_used, np.int32)
    order = np.empty(cfg.n_experts_used, np.int32)
    w = np.empty(cfg.n_experts_used, np.float32)
    proj = np.empty(cfg.hidden, np.float32)
    if lib().orc_moe(C.cast(model.ptr, C.c_void_p), layer, _f(xn), _f(lg), _i(ch), _i(order), _f(w), _f(proj), threads):
        raise RuntimeError("oracle moe failed")
    return lg, ch, order, w, proj


def step(model, seq, token, pos, threads=1, trace=True):
    """One CPU decode step (writes the model's host key-value cache at pos):
    (logits, router logits [L, E], chosen [L, K], residual after each layer [L, H])."""
    cfg = model.cfg
    L, E, K, H = cfg.n_layers, cfg.n_experts, cfg.n_experts_used, cfg.hidden
    logits = np.empty(cfg.vocab, np.float32)
    tl = np.empty((L, E), np.float32)
    tc = np.empty((L, K), np.int32)
    res = np.empty((L, H), np.float32)
    if lib().orc_step(C.cast(model.ptr, C.c_void_p), seq, token, pos, _f(logits), _f(tl) if trace else None,
                      _i(tc) if trace else None, _f(res) if trace else None, threads):
        raise RuntimeError("oracle step failed")
    return logits, tl, tc, res
