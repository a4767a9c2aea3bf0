"""vitna_hip_moe_prefill_noalloc: the prefill on device buffers the caller
owns, with the library's static working region in place of allocations,
against vitna_hip_moe_prefill (same kernels, allocated buffers) on the same
rows. Bit-exact: the same kernels in the same order on the same inputs give
the same bits, and the chosen experts are identical.

On a fresh model, before any allocating entry point has made the experts'
tiled copy, the no-allocation prefill runs the shared-stage GEMM kernel
(widening from the planes); the allocating prefill afterwards runs the kernel
that widens each wave's own weights from the tiled copy. The two must give
the same bits.

Two calls in a row, the second with fewer rows (the region keeps the first
call's contents), then a call with more rows than the region holds, which
must fail with a message and leave the device usable. Config 4's shape
(hidden 2048, 128 experts, top 8, expert width 768) is the one the region is
sized against.
"""
import ctypes as C

import numpy as np
import pytest

import vitna_amd as va
from test_gpu_decode import say

pytestmark = pytest.mark.gpu


class DeviceBuffer:
    """Device memory from the HIP runtime the library itself links (libamdhip64), outside the library."""

    def __init__(self, nbytes):
        va.hip()  # loads the library and with it the runtime
        self.rt = C.CDLL("libamdhip64.so.7")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(self.p), nbytes) == 0
        self.n = nbytes

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.n
        assert self.rt.hipMemcpy(self.p, a.ctypes.data, a.nbytes, 1) == 0  # host to device

    def get(self, shape, dtype):
        a = np.empty(shape, dtype)
        assert a.nbytes <= self.n
        assert self.rt.hipMemcpy(a.ctypes.data, self.p, a.nbytes, 2) == 0  # device to host
        return a

    def free(self):
        if self.p:
            self.rt.hipFree(self.p)
            self.p = C.c_void_p()


def test_prefill_noalloc_matches_allocating_entry():
    model = va.Model(va.shape(**va.CONFIGS[4]), 20260105, threads=16)
    dev = va.Device(model)
    cfg = model.cfg
    H, K = cfg.hidden, cfg.n_experts_used
    big = 1024
    xb = DeviceBuffer(big * H * 4)
    cb = DeviceBuffer(big * K * 4)
    try:
        for call, n in enumerate((700, 129)):
            say("no-alloc prefill, call", call, "rows", n)
            x = va.normal(500 + call, 3, n * H).reshape(n, H)
            want_x, want_ch = dev.prefill(0, x)
            xb.put(x)
            cb.put(np.full((n, K), -1, np.int32))
            dev.prefill_noalloc(0, xb.p.value, n, cb.p.value)
            dev.sync()
            got_x = xb.get((n, H), np.float32)
            got_ch = cb.get((n, K), np.int32)
            assert np.array_equal(got_ch, want_ch)
            assert np.array_equal(got_x.view(np.uint32), want_x.view(np.uint32))
        # without the chosen experts
        n = 64
        x = va.normal(777, 3, n * H).reshape(n, H)
        want_x, _ = dev.prefill(0, x)
        xb.put(x)
        dev.prefill_noalloc(0, xb.p.value, n, None)
        dev.sync()
        assert np.array_equal(xb.get((n, H), np.float32).view(np.uint32), want_x.view(np.uint32))
        # more rows than the region holds: refused before any launch, the device still serves
        with pytest.raises(va.VitnaError, match="static region holds"):
            dev.prefill_noalloc(0, xb.p.value, 65536, None)
        dev.prefill_noalloc(0, xb.p.value, n, None)
        dev.sync()
    finally:
        xb.free()
        cb.free()
        dev.close()
        model.free()


def test_prefill_noalloc_first_call_shared_stage_kernel():
    """The first call on a fresh model (no tiled copy yet: the shared-stage kernel) against the allocating prefill
    (the per-wave kernel) on the same rows, bit for bit; a second, smaller no-allocation call after that (now the
    per-wave kernel) too."""
    model = va.Model(va.shape(**va.CONFIGS[4]), 20260106, threads=16)
    dev = va.Device(model)
    cfg = model.cfg
    H, K = cfg.hidden, cfg.n_experts_used
    n = 600
    xb = DeviceBuffer(n * H * 4)
    cb = DeviceBuffer(n * K * 4)
    try:
        x = va.normal(900, 3, n * H).reshape(n, H)
        say("no-alloc prefill on a fresh model, rows", n)
        xb.put(x)
        cb.put(np.full((n, K), -1, np.int32))
        dev.prefill_noalloc(0, xb.p.value, n, cb.p.value)
        dev.sync()
        got_x = xb.get((n, H), np.float32)
        got_ch = cb.get((n, K), np.int32)
        want_x, want_ch = dev.prefill(0, x)
        assert np.array_equal(got_ch, want_ch)
        assert np.array_equal(got_x.view(np.uint32), want_x.view(np.uint32))
        m = 200
        xb.put(x[:m])
        dev.prefill_noalloc(0, xb.p.value, m, None)
        dev.sync()
        assert np.array_equal(xb.get((m, H), np.float32).view(np.uint32), want_x[:m].view(np.uint32))
    finally:
        xb.free()
        cb.free()
        dev.close()
        model.free()
