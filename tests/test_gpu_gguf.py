"""A GGUF checkpoint read by the library's GGUF reader (include/vitna_gguf.h)
and served on the GPU: the decode step of the model read back from the file
gives the same logits, bit for bit, as the same model uploaded from memory
(the device sees the same bytes), and agrees with the CPU checker's step on
the file-backed model within 1e-3 of max |cpu|."""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import rel, say

pytestmark = pytest.mark.gpu

SPEC = dict(n_layers=3, hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
            n_experts=32, n_experts_used=8, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1,
            ctx=96, seqs=1, kv_host=1)


def prefill(m, dev, pos):
    """Positions 0 .. pos - 1 of sequence 0's cache: the same seeded values on the host model and the device."""
    cfg = m.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    kc = np.ctypeslib.as_array(m.m.k_cache, shape=(cfg.n_layers, m.m.ctx, kd))
    vc = np.ctypeslib.as_array(m.m.v_cache, shape=(cfg.n_layers, m.m.ctx, kd))
    for l in range(cfg.n_layers):
        kc[l, :pos] = va.normal(3, 2 * l, pos * kd).reshape(pos, kd)
        vc[l, :pos] = va.normal(3, 2 * l + 1, pos * kd).reshape(pos, kd)
        dev.kv(0, l, 0, pos, kc[l, :pos], vc[l, :pos])


@pytest.mark.parametrize("norm_dtype", [va.F32, va.F16])
def test_gguf_model_on_device(tmp_path, norm_dtype):
    say("gguf model on device, norms", norm_dtype)
    model = va.Model(va.shape(**SPEC), 99)
    path = va.write_gguf(model, str(tmp_path), norm_dtype, 32)
    g = va.GgufModel(path, ctx=96, seqs=1)
    try:
        dev_g = va.Device(g)
        try:
            pos, token = 5, 123
            prefill(g, dev_g, pos)
            lg_g = dev_g.step(0, token, pos)
            ref, _, tc, _ = oracle.step(g, 0, token, pos)
            r = rel(lg_g, ref)
            say("  logits rel err vs the checker", r)
            assert r <= 1e-3
            assert np.array_equal(dev_g.step_routing(SPEC["n_layers"] - 1)[0], tc[-1])
        finally:
            dev_g.close()
        if norm_dtype == va.F32:
            dev_m = va.Device(model)
            try:
                prefill(model, dev_m, pos)
                lg_m = dev_m.step(0, token, pos)
            finally:
                dev_m.close()
            assert np.array_equal(lg_m.view(np.uint32), lg_g.view(np.uint32))
    finally:
        g.free()
        model.free()


def test_gguf_model_through_expert_cache(tmp_path):
    """The GGUF model's experts through a cache of 2K slots (the experts are views into the file's stacked
    tensors): the layer-at-a-time ABI gives the same bits as the same file with every expert resident."""
    from test_gpu_expert_cache import slot_bytes
    say("gguf model through the expert cache")
    model = va.Model(va.shape(**SPEC), 98)
    path = va.write_gguf(model, str(tmp_path), va.F32, 32)
    g = va.GgufModel(path, ctx=96, seqs=1)
    cfg = g.cfg
    K, L = cfg.n_experts_used, cfg.n_layers
    try:
        res = va.Device(g)
        cac = va.Device(g, expert_cache_bytes=2 * K * slot_bytes(cfg, SPEC))
        try:
            pos = 5
            prefill(g, res, pos)
            prefill(g, cac, pos)
            for t, token in enumerate([123, 7, 999]):
                outs = []
                for dev in (res, cac):
                    for l in range(L):
                        lg, nx = dev.moe_route(0, token, pos + t, l, want_next=True)
                        _, order, w = oracle.route(lg, K, bool(cfg.renormalize))
                        guess = oracle.route(nx, K, bool(cfg.renormalize))[0] if l + 1 < L else None
                        dev.moe_experts(l, order, w, guess)
                    outs.append(dev.moe_head())
                assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "token %d" % t
            _, cnt = cac.expert_cache_state()
            say("  cache counts", cnt)
            assert cnt["acquired"] == 3 * L * K and cnt["misses"] > 0
        finally:
            cac.close()
            res.close()
    finally:
        g.free()
        model.free()
