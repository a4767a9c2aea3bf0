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


def bounds_many(model, layer, xs, propagate=None):
    """moe_bound for many rows at once: each expert widened once, its rows' SwiGLU outputs and bound terms as matrix
    products. Returns (chosen [n][K], the checker's sums [n][H], bounds [n][H]).

    propagate (by default: when the layer's experts are K-quants) adds the first-order error the gate/up GEMM
    leaves in each SwiGLU output and the bf16 roundings after it, so that the bound is a bound whatever the
    weights' sign pattern. K-quant weights are d1 q - m1 with q in 0..15 (or ds (q - 32)), so a row's products
    cancel far more than Q8_0's symmetric ones: |g| is a small part of sum |x G|, and the gate's bf16 error, not
    the down GEMM's, sets the output's. For a pair (expert e, weight w) and output element r:
        dg = 2^-8 |G| |xn|, du = 2^-8 |U| |xn|                (bf16 operands of the gate/up GEMM)
        da = |silu'(g) u| dg + |silu(g)| du + 2^-9 |a|         (and the bf16 rounding of a = silu(g) u)
        |w| (2^-8 (|D| |a|)_r + (|D| da)_r + 2^-9 |(D a)_r|)   (bf16 operands of down, the bf16 part)
    summed over the row's pairs, plus 1e-6."""
    cfg = model.cfg
    H, K = cfg.hidden, cfg.n_experts_used
    lay = model.m.layers[layer]
    if propagate is None:
        propagate = lay.experts[0].gate.dtype != va.Q8_0 or lay.experts[0].down.dtype != va.Q8_0
    norm = np.ctypeslib.as_array(lay.mlp_norm, shape=(H,)).copy()
    n = xs.shape[0]
    xn = np.stack([oracle.rmsnorm(xs[i], norm, cfg.rms_eps) for i in range(n)])
    chosen = np.empty((n, K), np.int32)
    proj = np.empty((n, H), np.float32)
    users = {}
    for i in range(n):
        _, ch, order, wts, pr = oracle.moe(model, layer, xn[i])
        chosen[i], proj[i] = ch, pr
        for e, w in zip(order, wts):
            users.setdefault(int(e), []).append((i, abs(float(w))))
    bound = np.full((n, H), 1e-6)
    for e, lst in users.items():
        ex = lay.experts[e]
        G, U, D = (expert_weights(m).astype(np.float64) for m in (ex.gate, ex.up, ex.down))
        idx = np.array([i for i, _ in lst])
        wv = np.array([w for _, w in lst])
        X = xn[idx].astype(np.float64).T
        g, u = G @ X, U @ X
        with np.errstate(over="ignore"):
            sig = 1.0 / (1.0 + np.exp(-g))
        act = g * sig * u
        term = 2.0 ** -8 * (np.abs(D) @ np.abs(act))
        if propagate:
            dg, du = 2.0 ** -8 * (np.abs(G) @ np.abs(X)), 2.0 ** -8 * (np.abs(U) @ np.abs(X))
            dsilu = sig * (1.0 + g * (1.0 - sig))
            da = np.abs(dsilu * u) * dg + np.abs(g * sig) * du + 2.0 ** -9 * np.abs(act)
            term += np.abs(D) @ da + 2.0 ** -9 * np.abs(D @ act)
        bound[idx] += (term * wv[None, :]).T
    return chosen, proj, bound


def check_many(model, layer, x_in, x_out, chosen, rows):
    """check_rows over many rows with bounds_many; returns the largest |gpu - cpu| / bound seen."""
    rows = np.asarray(rows)
    ch, proj, bound = bounds_many(model, layer, x_in[rows])
    assert np.array_equal(chosen[rows], ch), ("rows with other experts", rows[np.any(chosen[rows] != ch, axis=1)][:8])
    got = x_out[rows].astype(np.float64) - x_in[rows]
    ratio = np.abs(got - proj) / bound
    bad = np.argwhere(ratio > 1.0)
    assert bad.size == 0, ("(row, element) over their bound", [(int(rows[r]), int(c)) for r, c in bad[:8]])
    return float(ratio.max())


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


KQ = {"q4k_q6k": dict(n_layers=2, hidden=512, intermediate=256, n_experts=16, n_experts_used=4, renormalize=1,
                     attention=0, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1),
      "q6k_q4k": dict(n_layers=1, hidden=1024, intermediate=512, n_experts=8, n_experts_used=2, renormalize=0,
                      attention=0, dt_gate_up=va.Q6_K, dt_down=va.Q4_K, norm_std=0.1)}


@pytest.mark.parametrize("name,n", [("q4k_q6k", 37), ("q4k_q6k", 300), ("q6k_q4k", 129)])
def test_prefill_kquant(name, n):
    """K-quant experts (Q4_K gate/up with Q6_K down, the Q4_K_M convention, and the other way round): the GEMM
    widens each 32-column group from the planes with the reference's arithmetic, then rounds it to bf16. Every
    row against the checker's choice and the per-element bound, every layer."""
    say("prefill k-quant", name, n)
    model = va.Model(va.shape(**KQ[name]), 4244)
    dev = va.Device(model)
    try:
        for layer in range(model.cfg.n_layers):
            x = va.normal(190 + n, layer, n * model.cfg.hidden).reshape(n, model.cfg.hidden)
            out, chosen = dev.prefill(layer, x)
            worst = check_many(model, layer, x, out, chosen, range(n))
            say("  layer", layer, "rows", n, "largest error / bound", worst)
    finally:
        dev.close()
        model.free()


def overflow_rows(chosen, E, tile=256):
    """Rows that cover every expert's first and last tile of pairs: for each expert (its pairs in row order, as the
    grouping lists them), the rows of its first pair, its 256th, its 257th (the overflow tile's first) and its
    last."""
    rows = set()
    for e in range(E):
        r = np.nonzero(np.any(chosen == e, axis=1))[0]
        if r.size == 0:
            continue
        for j in (0, min(tile - 1, r.size - 1), min(tile, r.size - 1), r.size - 1):
            rows.add(int(r[j]))
    return rows


def test_prefill_config4_full():
    """BASELINE config 4 at full size: 4096 rows N(0,1) drawn on the device, 128 Q8_0 experts, top-8.
    Every row's choice is checked; the sums of at least 512 rows, among them rows in every expert's first tile and
    in every expert's overflow tile (its pairs past 256)."""
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
        E = model.cfg.n_experts
        rows = overflow_rows(chosen, E)
        over = sum(1 for e in range(E) if np.count_nonzero(np.any(chosen == e, axis=1)) > 256)
        for r in np.random.RandomState(5).permutation(n):
            if len(rows) >= 512:
                break
            rows.add(int(r))
        rows = sorted(rows)
        assert len(rows) >= 512
        worst = check_many(model, 0, x_in, x_out, chosen, rows)
        say("  %d rows checked (%d experts with an overflow tile, each covered); largest error / bound %.3f"
            % (len(rows), over, worst))
    finally:
        dev.close()
        model.free()
