"""Prefill through one mixture-of-experts layer: every row
normalized and routed exactly as the CPU routes it, the experts run as a
grouped bf16 MFMA GEMM (vitna_hip_moe_prefill, vitna_hip_time_prefill).

The bar, per row:
  - the chosen experts, largest first, identical to the CPU checker's (the
    router's logits are bit-exact, the routing rule is the reference's);
  - the weighted expert sum within PREFILL_REL of the row's max |CPU sum|.

PREFILL_REL, the bf16 bound: the GEMM rounds three things to bf16 (relative
error at most 2^-9 each): each weight q * d, the normalized row, and the
SwiGLU output; products are summed in fp32. The roundings of a sum's terms
are independent, so its error is about 2^-9/sqrt(3) times the root-sum-square
of its terms. A bf16 emulation in numpy on 24 config-4 rows gives a worst
4.6e-3 of max |sum| (fp16 everywhere would give 6.9e-4); the 16-expert model
below, with fewer terms per sum, runs higher. PREFILL_REL = 1e-2. A wrong
scale, a dropped block, a transposed tile or a row given another row's
experts gives errors of order 1.
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import rel, say

pytestmark = pytest.mark.gpu

PREFILL_REL = 1e-2

SMALL_Q8 = dict(n_layers=2, hidden=256, intermediate=256, n_experts=16, n_experts_used=4, renormalize=0,
                attention=0, rms_eps=1e-5, dt_gate_up=va.Q8_0, dt_down=va.Q8_0, norm_std=0.1)


def cpu_routing(model, layer, x):
    """Each row's experts (largest first) as the CPU checker chooses them."""
    cfg = model.cfg
    H, E, K = cfg.hidden, cfg.n_experts, cfg.n_experts_used
    lay = model.m.layers[layer]
    norm = np.ctypeslib.as_array(lay.mlp_norm, shape=(H,)).copy()
    out = np.empty((x.shape[0], K), np.int32)
    for i in range(x.shape[0]):
        xn = oracle.rmsnorm(x[i], norm, cfg.rms_eps)
        lg = oracle.matvec(lay.router.data, lay.router.dtype, xn, E, H)
        out[i] = oracle.route(lg, K, bool(cfg.renormalize))[0]
    return out


def cpu_moe(model, layer, x, threads=16):
    """Each row's (chosen, weighted expert sum) from the CPU checker."""
    cfg = model.cfg
    H = cfg.hidden
    norm = np.ctypeslib.as_array(model.m.layers[layer].mlp_norm, shape=(H,)).copy()
    xn = oracle.rmsnorm(x, norm, cfg.rms_eps)
    _, ch, _, _, proj = oracle.moe(model, layer, xn, threads=threads)
    return ch, proj


def check_rows(model, layer, x_in, x_out, chosen, rows):
    worst = 0.0
    for i in rows:
        ch, proj = cpu_moe(model, layer, x_in[i])
        assert np.array_equal(chosen[i], ch), ("row", i, chosen[i], ch)
        got = x_out[i].astype(np.float64) - x_in[i]
        r = float(np.max(np.abs(got - proj)) / np.max(np.abs(proj)))
        worst = max(worst, r)
        assert r <= PREFILL_REL, ("row", i, r)
    return worst


@pytest.mark.parametrize("n", [1, 37, 300])
def test_prefill_small(n):
    """Q8_0 experts, 16 of them, top-4: ragged groups, tiles cut short, a single row; both layers."""
    say("prefill small", n)
    model = va.Model(va.shape(**SMALL_Q8), 4242)
    dev = va.Device(model)
    try:
        for layer in range(model.cfg.n_layers):
            x = va.normal(90 + n, layer, n * model.cfg.hidden).reshape(n, model.cfg.hidden)
            out, chosen = dev.prefill(layer, x)
            worst = check_rows(model, layer, x, out, chosen, range(n))
            say("  layer", layer, "rows", n, "worst rel err", worst)
    finally:
        dev.close()
        model.free()


def test_prefill_config4_full():
    """BASELINE config 4 at full size: 4096 rows N(0,1) drawn on the device, 128 Q8_0 experts, top-8.
    Every row's choice is checked; the sums of 96 rows spread over the batch."""
    say("prefill config 4")
    model = va.Model(va.shape(**va.CONFIGS[4]), 20260104, threads=16)
    dev = va.Device(model)
    try:
        n = 4096
        tot, ph = dev.time_prefill(0, n, seed=11, reps=2)
        say("  prefill of %d rows: %.1f us (phases %s)" % (n, tot, ["%.1f" % p for p in ph]))
        x_in, x_out, chosen = dev.prefill_rows(n)
        assert np.all(np.isfinite(x_in)) and abs(float(np.std(x_in)) - 1.0) < 0.01
        ref = cpu_routing(model, 0, x_in)
        bad = np.nonzero(np.any(ref != chosen, axis=1))[0]
        assert bad.size == 0, ("rows with other experts", bad[:10])
        rows = np.linspace(0, n - 1, 96).astype(int)
        worst = check_rows(model, 0, x_in, x_out, chosen, rows)
        say("  worst rel err of 96 rows", worst)
    finally:
        dev.close()
        model.free()
