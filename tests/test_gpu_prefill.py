"""Prefill through one mixture-of-experts layer: every row
normalized and routed exactly as the CPU routes it, the experts run as a
grouped bf16 MFMA GEMM (vitna_hip_moe_prefill, vitna_hip_time_prefill).

The bar, per row:
  - the chosen experts, largest first, identical to the CPU checker's (the
    router's logits are bit-exact, the routing rule is the reference's);
  - every element of the weighted expert sum within its own bound, the bf16
    GEMM bound |gpu - cpu| <= 2^-8 * sum_k |x_k w_k| + 1e-6 of the output
    GEMM: for element r, 2^-8 * sum_e |w_e| sum_j |a_ej D_e[r, j]| + 1e-6, with
    the checker's SwiGLU outputs a_e and its own widened down weights D_e
    (oracle.widen). The bound takes a bf16 rounding of each factor of each
    product (2^-9 each); the error the gate/up GEMM leaves in a_e and the bf16
    rounding of each pair's part are of the same kind and size, and a bf16
    emulation of the device's arithmetic stays
    under a fifth of the bound at config 4's shape and under a third at the
    small one (tests/test_prefill_bound.py). The bound is 6-14% of the mean
    |sum|, so a wrong scale, a dropped block, a transposed tile or a row given
    another row's experts breaks it in every element it touches, however few.
"""
import ctypes

import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import say

pytestmark = pytest.mark.gpu


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


def expert_weights(mat):
    """An expert matrix widened to fp32 by the checker (the reference CPU's Q8_0 widening)."""
    n = va.row_bytes(mat.dtype, mat.cols) * mat.rows
    raw = np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(ctypes.cast(mat.data, ctypes.c_void_p).value))
    return oracle.widen(raw, mat.dtype, mat.rows * mat.cols).reshape(mat.rows, mat.cols)


def moe_bound(model, layer, x):
    """For one row: (chosen, the checker's weighted expert sum, each element's bound)."""
    cfg = model.cfg
    H = cfg.hidden
    lay = model.m.layers[layer]
    norm = np.ctypeslib.as_array(lay.mlp_norm, shape=(H,)).copy()
    xn = oracle.rmsnorm(x, norm, cfg.rms_eps)
    _, ch, order, wts, proj = oracle.moe(model, layer, xn)
    bound = np.full(H, 1e-6)
    for e, w in zip(order, wts):
        ex = lay.experts[int(e)]
        G, U, D = (expert_weights(m).astype(np.float64) for m in (ex.gate, ex.up, ex.down))
        g, u = G @ xn, U @ xn
        act = g / (1.0 + np.exp(-g)) * u
        bound += abs(float(w)) * 2.0 ** -8 * (np.abs(D) @ np.abs(act))
    return ch, proj, bound


def check_rows(model, layer, x_in, x_out, chosen, rows):
    """Every listed row against its bound; returns the largest |gpu - cpu| / bound seen."""
    worst = 0.0
    for i in rows:
        ch, proj, bound = moe_bound(model, layer, x_in[i])
        assert np.array_equal(chosen[i], ch), ("row", i, chosen[i], ch)
        got = x_out[i].astype(np.float64) - x_in[i]
        ratio = np.abs(got - proj) / bound
        worst = max(worst, float(ratio.max()))
        bad = np.nonzero(ratio > 1.0)[0]
        assert bad.size == 0, ("row", i, "elements over their bound", bad[:8], ratio[bad[:8]])
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
            say("  layer", layer, "rows", n, "largest error / bound", worst)
    finally:
        dev.close()
        model.free()


def test_prefill_wide_hidden():
    """A hidden size past the fused norm-and-router kernel's 2048 (4096): the separate norm and router kernels."""
    say("prefill hidden 4096")
    model = va.Model(va.shape(**dict(SMALL_Q8, n_layers=1, hidden=4096)), 4243)
    dev = va.Device(model)
    try:
        n = 37
        x = va.normal(77, 0, n * model.cfg.hidden).reshape(n, model.cfg.hidden)
        out, chosen = dev.prefill(0, x)
        worst = check_rows(model, 0, x, out, chosen, range(n))
        say("  rows", n, "largest error / bound", worst)
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
        say("  largest error / bound over 96 rows", worst)
    finally:
        dev.close()
        model.free()
