"""The reference's --precision fast behind its own ABI: a model created with
gpu_fast runs the experts of every pass of at least 64 rows
(vitna_cuda_moe_rows_experts, and the device-routed rows step) as the bf16
matrix-core grouped GEMM of the prefill (engine/src/model_cuda.cu:197-204,
3807, 5002-5022, 5275-5304). Passes go up to vitna_cuda_moe_rows_max = 1024
rows, the reference's MOE_ROWS, so model.c prompts in chunks of 1024.

Bars:
  * a fast pass of 64, 256 and 1024 rows, routed by the host as model.c
    routes: each row's mixture (its residual after the experts minus before)
    within the per-element bf16 GEMM bound of the checker's mixture of the same
    residual (test_gpu_prefill's bound), every layer; Q4_K gate/up with Q6_K
    down (the Q4_K_M convention) and Q8_0;
  * the exact mode unchanged: below 64 rows a fast model gives the bits of a
    model without gpu_fast, and a model without gpu_fast keeps the exact
    kernels at any row count (within 1e-3 of max |cpu|, as the rows tests);
  * the device-routed rows step of a fast pass gives the bits of the same pass
    played through the ABI layer by layer.
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import rel, say
from test_gpu_prefill import bounds_many

pytestmark = pytest.mark.gpu

SPECS = {
    "q4km": dict(n_layers=2, hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
                 n_experts=32, n_experts_used=8, renormalize=1, norm_std=0.1, ctx=48, kv_host=1),
    "q8": dict(n_layers=2, hidden=256, intermediate=256, n_heads=4, n_kv_heads=2, head_dim=64, vocab=300, n_experts=16,
               n_experts_used=4, renormalize=0, rms_eps=1e-5, dt_gate_up=va.Q8_0, dt_down=va.Q8_0, dt_q=va.Q8_0,
               dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0, dt_head=va.Q8_0, dt_embed=va.Q8_0, norm_std=0.1, ctx=48,
               kv_host=1),
}
SEQS = 64


def make(name, seed, fast):
    model = va.Model(va.shape(**dict(SPECS[name], seqs=SEQS)), seed)
    return model, va.Device(model, fast=fast)


def pass_rows(n, cfg, salt=0):
    """n rows over SEQS sequences, rows of one sequence at consecutive positions (they see each other's keys)."""
    return [(int((37 * i + salt) % cfg.vocab), int(i // SEQS), int(i % SEQS)) for i in range(n)]


def host_route(dev, rows, layer, cfg):
    lg = dev.rows_route(rows, layer)
    ids, ws = [], []
    for i in range(len(rows)):
        _, order, w = oracle.route(lg[i], cfg.n_experts_used, bool(cfg.renormalize))
        ids.append(order)
        ws.append(w)
    return np.array(ids), np.array(ws)


def residuals(dev, n):
    return np.stack([dev.residual(i) for i in range(n)])


@pytest.mark.parametrize("name,n", [("q4km", 64), ("q4km", 256), ("q4km", 1024), ("q8", 256)])
def test_fast_pass_within_bf16_bound(name, n):
    say("fast pass", name, n)
    model, dev = make(name, 31337, True)
    try:
        cfg = model.cfg
        assert dev.rows_max() == 1024
        rows = pass_rows(n, cfg)
        worst = 0.0
        for l in range(cfg.n_layers):
            ids, ws = host_route(dev, rows, l, cfg)
            x0 = residuals(dev, n)
            dev.rows_experts(l, ids, ws)
            x1 = residuals(dev, n)
            ch, proj, bound = bounds_many(model, l, x0)
            # the host's routing of the device's exact router logits is the checker's routing of the same residual
            assert np.array_equal(np.sort(ch, axis=1), np.sort(ids, axis=1))
            ratio = np.abs((x1.astype(np.float64) - x0) - proj) / bound
            worst = max(worst, float(ratio.max()))
            bad = np.argwhere(ratio > 1.0)
            assert bad.size == 0, ("layer", l, "(row, element) over the bound", bad[:8])
        say("  largest error / bound", worst)
    finally:
        dev.close()
        model.free()


@pytest.mark.parametrize("name", ["q4km", "q8"])
def test_exact_mode_unchanged(name):
    """Below the fast threshold a fast model runs the exact kernels (the same bits as a model without gpu_fast);
    a model without gpu_fast runs them at 64 rows and more, within the rows tests' tolerance of the checker."""
    say("exact mode", name)
    fm, fd = make(name, 4711, True)
    em, ed = make(name, 4711, False)
    try:
        cfg = fm.cfg
        for n in (63, 64):
            rows = pass_rows(n, cfg, salt=n)
            for l in range(cfg.n_layers):
                fi, fw = host_route(fd, rows, l, cfg)
                ei, ew = host_route(ed, rows, l, cfg)
                if n == 63:
                    assert np.array_equal(fi, ei)
                x0 = residuals(ed, n)
                fd.rows_experts(l, fi, fw)
                ed.rows_experts(l, ei, ew)
                xf, xe = residuals(fd, n), residuals(ed, n)
                if n == 63:
                    assert np.array_equal(xf.view(np.uint32), xe.view(np.uint32)), ("layer", l)
                    continue
                # the exact kernels at 64 rows: the checker's mixture within 1e-3 of its largest element
                H = cfg.hidden
                norm = np.ctypeslib.as_array(em.m.layers[l].mlp_norm, shape=(H,)).copy()
                for i in range(0, n, 7):
                    _, _, _, _, proj = oracle.moe(em, l, oracle.rmsnorm(x0[i], norm, cfg.rms_eps))
                    got = xe[i].astype(np.float64) - x0[i]
                    assert float(np.max(np.abs(got - proj)) / np.max(np.abs(proj))) <= 1e-3, ("row", i, "layer", l)
                # and the fast model's mixture is not the exact one's bits (it did take the GEMM)
                assert not np.array_equal(xf.view(np.uint32), xe.view(np.uint32))
    finally:
        fd.close()
        ed.close()
        fm.free()
        em.free()


def test_fast_rows_step_matches_abi():
    """vitna_hip_moe_rows_step on a fast model at 96 rows: device routing and the grouped GEMM in one graph, replayed
    twice; the logits' bits equal those of the same pass through the ABI layer by layer with the device's routing
    (the host's rule gives the same experts), and stay near the checker's step (bf16 experts: within 3e-2 of
    max |cpu|)."""
    say("fast rows step")
    model, dev = make("q4km", 2718, True)
    try:
        cfg = model.cfg
        n = 96
        rows = pass_rows(n, cfg, salt=5)
        a = np.stack(dev.rows_step(rows))
        b = np.stack(dev.rows_step(rows))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # the device's routing of every row and layer: the same experts as the host's rule on the same logits, and
        # weights within 2e-6 (libm's expf against the device's); the ABI pass is given the device's weights, so
        # that the same kernels see the same inputs
        dev_rt = [[dev.rows_routing(l, i) for i in range(n)] for l in range(cfg.n_layers)]
        for l in range(cfg.n_layers):
            ids, ws = host_route(dev, rows, l, cfg)
            d_ids = np.array([dev_rt[l][i][1] for i in range(n)])
            d_ws = np.array([dev_rt[l][i][2] for i in range(n)])
            assert np.array_equal(d_ids, ids), ("layer", l)
            assert float(np.max(np.abs(d_ws - ws) / np.abs(ws))) <= 2e-6
            dev.rows_experts(l, d_ids, d_ws)
        c = np.stack(dev.rows_head(n))
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        # the checker's step of a few rows, over the device's cache of the positions before each
        L, kd = cfg.n_layers, cfg.n_kv_heads * cfg.head_dim
        kc = np.ctypeslib.as_array(model.m.k_cache, shape=(SEQS, L, model.m.ctx, kd))
        vc = np.ctypeslib.as_array(model.m.v_cache, shape=(SEQS, L, model.m.ctx, kd))
        worst = 0.0
        for i in (0, 1, SEQS, n - 1):
            tok, pos, seq = rows[i]
            for l in range(L):
                if pos:
                    k, v = dev.kv(seq, l, 0, pos)
                    kc[seq, l, :pos] = k
                    vc[seq, l, :pos] = v
            ref, _, _, _ = oracle.step(model, seq, tok, pos)
            worst = max(worst, rel(a[i], ref))
        say("  rows step = ABI bits; logits rel err against the exact checker", worst)
        assert worst <= 3e-2
    finally:
        dev.close()
        model.free()


def test_exact_pass_at_rows_max():
    """A model without gpu_fast at the most rows a pass takes (vitna_cuda_moe_rows_max = 1024, 16 rows of each of
    64 sequences at consecutive positions): the device-routed rows step (one graph) and the same pass through the
    ABI layer by layer with the device's routing give the same logits bits, and sampled rows' logits are within
    1e-3 of max |cpu| of the checker's step over the device's cache."""
    say("exact pass at rows_max")
    model, dev = make("q4km", 1618, False)
    try:
        cfg = model.cfg
        n = dev.rows_max()
        assert n == 1024
        rows = pass_rows(n, cfg, salt=11)
        a = np.stack(dev.rows_step(rows))
        dev_rt = [[dev.rows_routing(l, i) for i in range(n)] for l in range(cfg.n_layers)]
        for l in range(cfg.n_layers):
            ids, ws = host_route(dev, rows, l, cfg)
            d_ids = np.array([dev_rt[l][i][1] for i in range(n)])
            d_ws = np.array([dev_rt[l][i][2] for i in range(n)])
            assert np.array_equal(d_ids, ids), ("layer", l)
            dev.rows_experts(l, d_ids, d_ws)
        c = np.stack(dev.rows_head(n))
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        L, kd = cfg.n_layers, cfg.n_kv_heads * cfg.head_dim
        kc = np.ctypeslib.as_array(model.m.k_cache, shape=(SEQS, L, model.m.ctx, kd))
        vc = np.ctypeslib.as_array(model.m.v_cache, shape=(SEQS, L, model.m.ctx, kd))
        worst = 0.0
        for i in (0, SEQS + 3, n - 1):
            tok, pos, seq = rows[i]
            for l in range(L):
                if pos:
                    k, v = dev.kv(seq, l, 0, pos)
                    kc[seq, l, :pos] = k
                    vc[seq, l, :pos] = v
            ref, _, tc, _ = oracle.step(model, seq, tok, pos)
            for l in range(L):
                assert np.array_equal(np.sort(dev_rt[l][i][1]), np.sort(tc[l])), ("row", i, "layer", l)
            worst = max(worst, rel(a[i], ref))
        say("  rows step = ABI bits at 1024 rows; logits rel err against the checker", worst)
        assert worst <= 1e-3
    finally:
        dev.close()
        model.free()
