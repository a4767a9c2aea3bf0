"""Models whose matrices change dtype from layer to layer, as llama.cpp's
Q4_K_M writes them (llama.cpp's llama_tensor_get_type: attn_v and ffn_down,
the stacked experts' too, are Q6_K on the use_more_bits layers, the first and
last eighth and every third layer between, and Q4_K elsewhere), and the q / k
mix of the GGUF reader's mixed_dtypes variant (q Q6_K, k Q8_0 in one layer).
The reference dispatches every projection over any served dtype
(model_cuda.cu:2976-3024, attn_in_kernel<DT,DTV> :864-870); here the decode
GEMV fuses the dtype triples it is instantiated for and runs any other mix one
matrix a launch.

Each device path steps such a model against the CPU checker: the per-layer
graph step and the persistent step kernel (where it takes the model), the
ABI's layer-by-layer step with host routing, the device-routed rows step, the
prefill GEMM, all with the decode tests' bars (identical choice every layer,
logits within 1e-3 of max |cpu|; the prefill within its bf16 bound).
"""
import ctypes

import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import rel, say
from test_gpu_prefill import check_many

pytestmark = pytest.mark.gpu

REL = 1e-3
SPEC = dict(n_layers=8, hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
            n_experts=16, n_experts_used=4, renormalize=1, norm_std=0.1, ctx=96, seqs=4, kv_host=1)


def use_more_bits(i, n):
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


class MixedModel:
    """The Q4_K_M model of SPEC (v and down Q6_K) with v and every expert's down taken from a Q4_K twin of the same
    seed on the layers llama.cpp gives Q4_K, and layer 1's q and k from a third model (Q6_K, Q8_0). The twins own
    the bytes and live as long as this model; the base model's own matrices are put back before it is freed (each
    model frees the matrices it holds)."""

    def __init__(self, seed):
        self.base = va.Model(va.shape(**SPEC), seed)
        self.q4 = va.Model(va.shape(**dict(SPEC, dt_v=va.Q4_K, dt_down=va.Q4_K)), seed)
        self.qk = va.Model(va.shape(**dict(SPEC, dt_q=va.Q6_K, dt_k=va.Q8_0)), seed)
        m, n = self.base.m, SPEC["n_layers"]
        self.v_dtypes = []
        self.own = []  # (layer, expert or None, field, the base model's own matrix)
        for l in range(n):
            if not use_more_bits(l, n):
                self._take(l, None, "v", self.q4)
                for e in range(SPEC["n_experts"]):
                    self._take(l, e, "down", self.q4)
            self.v_dtypes.append(m.layers[l].v.dtype)
        self._take(1, None, "q", self.qk)
        self._take(1, None, "k", self.qk)

    def _take(self, l, e, field, twin):
        dst = self.base.m.layers[l] if e is None else self.base.m.layers[l].experts[e]
        src = twin.m.layers[l] if e is None else twin.m.layers[l].experts[e]
        keep = va.Matrix()
        ctypes.pointer(keep)[0] = getattr(dst, field)
        self.own.append((l, e, field, keep))
        setattr(dst, field, getattr(src, field))

    def free(self):
        for l, e, field, keep in self.own:
            dst = self.base.m.layers[l] if e is None else self.base.m.layers[l].experts[e]
            setattr(dst, field, keep)
        for x in (self.base, self.q4, self.qk):
            x.free()


def fill(model, dev, pos, seed):
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L, ctx = cfg.n_layers, model.m.ctx
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(model.m.seqs, L, ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(model.m.seqs, L, ctx, kd))
    kc[:] = va.normal(seed, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(seed, 102, vc.size).reshape(vc.shape)
    for s in range(model.m.seqs):
        for l in range(L):
            dev.kv(s, l, 0, pos, kc[s, l, :pos], vc[s, l, :pos])


def test_mix_is_the_q4km_rule():
    mm = MixedModel(5)
    try:
        assert mm.v_dtypes == [va.Q6_K if use_more_bits(l, 8) else va.Q4_K for l in range(8)]
        assert va.Q4_K in mm.v_dtypes and va.Q6_K in mm.v_dtypes
    finally:
        mm.free()


@pytest.mark.parametrize("persistent", [False, True], ids=["graph", "persistent"])
def test_mixed_device_step(persistent):
    say("dtype mix: device step", "persistent" if persistent else "graph")
    mm = MixedModel(808)
    model = mm.base
    dev = va.Device(model)
    try:
        pos = 70
        fill(model, dev, pos + 1, 808)
        taken = dev.set_step_kernel(persistent)
        say("  persistent kernel taken:", taken)
        for p in (pos - 1, pos):
            ref, _, tc, _ = oracle.step(model, 0, 17, p)
            logits = dev.step(0, 17, p)
            for l in range(model.cfg.n_layers):
                assert np.array_equal(dev.step_routing(l)[0], tc[l]), ("layer", l)
            r = rel(logits, ref)
            say("  pos", p, "logits rel err", r)
            assert r <= REL and float(np.max(np.abs(logits - ref))) <= 1e-2
    finally:
        dev.close()
        mm.free()


def test_mixed_abi_step():
    say("dtype mix: ABI step with host routing")
    mm = MixedModel(809)
    model = mm.base
    dev = va.Device(model)
    try:
        cfg = model.cfg
        pos, seq, tok = 40, 2, 123
        fill(model, dev, pos, 809)
        ref, _, tc, res = oracle.step(model, seq, tok, pos)
        for l in range(cfg.n_layers):
            lg = dev.moe_route(seq, tok, pos, l)
            ch, order, w = oracle.route(lg, cfg.n_experts_used, bool(cfg.renormalize))
            assert np.array_equal(ch, tc[l]), ("layer", l)
            dev.moe_experts(l, order, w)
            assert rel(dev.residual(), res[l]) <= REL, ("layer", l)
        r = rel(dev.moe_head(), ref)
        say("  logits rel err", r)
        assert r <= REL
    finally:
        dev.close()
        mm.free()


def test_mixed_rows_step():
    say("dtype mix: rows step")
    mm = MixedModel(810)
    model = mm.base
    dev = va.Device(model)
    try:
        cfg = model.cfg
        lens = [5, 60, 33, 90]
        fill(model, dev, max(lens), 810)
        rows = [(7 * s + 1, lens[s], s) for s in range(4)]
        logits = dev.rows_step(rows)
        for s, (tok, pos, seq) in enumerate(rows):
            ref, _, tc, _ = oracle.step(model, seq, tok, pos)
            for l in range(cfg.n_layers):
                assert np.array_equal(dev.rows_routing(l, s)[0], tc[l]), ("row", s, "layer", l)
            r = rel(logits[s], ref)
            say("  row", s, "logits rel err", r)
            assert r <= REL
    finally:
        dev.close()
        mm.free()


def test_mixed_prefill():
    """The prefill GEMM on a Q4_K-down layer and a Q6_K-down layer of the same model."""
    say("dtype mix: prefill")
    mm = MixedModel(811)
    model = mm.base
    dev = va.Device(model)
    try:
        n = 200
        for l in (0, 1):  # layer 0 uses more bits (Q6_K down), layer 1 not (Q4_K down)
            x = va.normal(811, l, n * model.cfg.hidden).reshape(n, model.cfg.hidden)
            out, chosen = dev.prefill(l, x)
            worst = check_many(model, l, x, out, chosen, range(n))
            say("  layer", l, "down", model.m.layers[l].experts[0].down.dtype, "largest error / bound", worst)
    finally:
        dev.close()
        mm.free()
