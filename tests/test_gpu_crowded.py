"""Crowded passes: a pass of many rows puts tens of pairs on every expert (a prompt's chunk of 1024 rows of top-8
over 128 experts: 64 an expert). From 512 rows on, a model whose experts are resident runs them on tiles of 32
pairs of one expert (launch_gsx in kernels_skinny.hip) instead of the four-pair tiles of kernels_gmma.hip.

The bar is the grouped kernels': each layer, the device's residual rows before and after
vitna_cuda_moe_rows_experts (routed by the host from the device's router logits, as model.c routes a prompt's
chunk, engine/src/model.c:1006-1030) against the CPU checker's mixture of the same rows, every row, layer by layer,
for Q8_0, Q4_K / Q6_K and Q6_K / Q4_K experts. Experts hold several 32-pair tiles with a part-filled last one.
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import SMALL, say

pytestmark = pytest.mark.gpu

REL = 1e-4


@pytest.mark.parametrize("name,n", [("q8", 600), ("q4km", 520), ("q6gu", 1024)])
def test_crowded_pass_experts(name, n):
    say("crowded pass", name, n, "rows")
    model = va.Model(va.shape(**dict(SMALL[name], ctx=n + 8, seqs=1)), 31337)
    dev = va.Device(model)
    try:
        cfg = model.cfg
        H, K = cfg.hidden, cfg.n_experts_used
        rows = [((11 * i + 7) % cfg.vocab, i, 0) for i in range(n)]
        worst, most, least = 0.0, 0, n
        for l in range(cfg.n_layers):
            norm = np.ctypeslib.as_array(model.m.layers[l].mlp_norm, shape=(H,)).copy()
            lg = dev.rows_route(rows, l)
            x0 = np.stack([dev.residual(i) for i in range(n)])
            ids, ws, projs = [], [], []
            for i in range(n):
                ch, order, w = oracle.route(lg[i], K, bool(cfg.renormalize))
                _, cch, _, _, proj = oracle.moe(model, l, oracle.rmsnorm(x0[i], norm, cfg.rms_eps))
                assert np.array_equal(ch, cch), ("row", i, "layer", l)
                ids.append(order)
                ws.append(w)
                projs.append(proj)
            per = np.bincount(np.concatenate(ids), minlength=cfg.n_experts)
            most, least = max(most, int(per.max())), min(least, int(per[per > 0].min()))
            dev.rows_experts(l, np.array(ids), np.array(ws))
            x1 = np.stack([dev.residual(i) for i in range(n)])
            for i in range(n):
                got = x1[i].astype(np.float64) - x0[i]
                r = float(np.max(np.abs(got - projs[i])) / np.max(np.abs(projs[i])))
                worst = max(worst, r)
                assert r <= REL, ("row", i, "layer", l, r)
        say("  pairs an expert", least, "to", most, "; worst rel err of the mixture", worst)
        assert most > 64, "no expert took more than two tiles"
    finally:
        dev.close()
        model.free()
