"""The prefill test's per-element bound (test_gpu_prefill.moe_bound) on the CPU:
it holds for a bf16 emulation of the device's arithmetic and fails for an
error confined to one element, so a tile or index mistake that touches few
columns cannot pass it."""
import numpy as np

import oracle
import vitna_amd as va
from test_gpu_prefill import KQ, SMALL_Q8, bounds_many, expert_weights, moe_bound


def bf16(a):
    """Round to bf16 (nearest even) and back to float32."""
    b = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32)


def test_bound_holds_for_bf16_and_catches_one_element():
    model = va.Model(va.shape(**SMALL_Q8), 31)
    try:
        cfg = model.cfg
        H = cfg.hidden
        lay = model.m.layers[0]
        norm = np.ctypeslib.as_array(lay.mlp_norm, shape=(H,)).copy()
        worst = 0.0
        for seed in range(6):
            x = va.normal(7, seed, H)
            ch, proj, bound = moe_bound(model, 0, x)
            assert np.all(bound > 0)
            # the device's arithmetic: bf16 inputs to each GEMM, fp32 sums, bf16 SwiGLU output, bf16 parts
            xn = oracle.rmsnorm(x, norm, cfg.rms_eps)
            _, _, order, wts, _ = oracle.moe(model, 0, xn)
            y = np.zeros(H, np.float64)
            for e, w in zip(order, wts):
                ex = lay.experts[int(e)]
                G, U, D = (bf16(expert_weights(m)) for m in (ex.gate, ex.up, ex.down))
                g = G.astype(np.float32) @ bf16(xn)
                u = U.astype(np.float32) @ bf16(xn)
                act = bf16(g / (1.0 + np.exp(-g)) * u)
                y += bf16(np.float32(w) * (D.astype(np.float32) @ act))  # each pair's part is kept in bf16
            ratio = np.abs(y - proj) / bound
            worst = max(worst, float(ratio.max()))
            assert ratio.max() <= 1.0
            # one element off by its bound's own size, or a column taken from the wrong expert: caught
            z = y.copy()
            z[H // 3] += 3 * bound[H // 3]
            assert (np.abs(z - proj) / bound).max() > 1.0
        print("largest emulated error / bound", worst)
        assert worst < 0.5  # margin: the device's error is well inside the bound
        assert worst > 1e-2  # the bound is not vacuous: the emulation's error is a visible part of it
    finally:
        model.free()


def test_kquant_bound_holds_for_bf16_and_catches_one_element():
    """The same for K-quant experts (Q4_K gate/up, Q6_K down) with bounds_many's propagated form: an emulation of
    the device (each weight widened as the reference widens it, then rounded to bf16) stays inside it, with a margin,
    and an error of three bounds in one element is caught."""
    model = va.Model(va.shape(**KQ["q4k_q6k"]), 4244)
    try:
        cfg = model.cfg
        H = cfg.hidden
        lay = model.m.layers[0]
        norm = np.ctypeslib.as_array(lay.mlp_norm, shape=(H,)).copy()
        xs = np.stack([va.normal(9, seed, H) for seed in range(8)])
        ch, proj, bound = bounds_many(model, 0, xs)
        worst = 0.0
        for i in range(xs.shape[0]):
            xn = oracle.rmsnorm(xs[i], norm, cfg.rms_eps)
            _, _, order, wts, _ = oracle.moe(model, 0, xn)
            y = np.zeros(H, np.float64)
            for e, w in zip(order, wts):
                ex = lay.experts[int(e)]
                G, U, D = (bf16(expert_weights(m)) for m in (ex.gate, ex.up, ex.down))
                g = G.astype(np.float32) @ bf16(xn)
                u = U.astype(np.float32) @ bf16(xn)
                act = bf16(g / (1.0 + np.exp(-g)) * u)
                y += bf16(np.float32(w) * (D.astype(np.float32) @ act))
            ratio = np.abs(y - proj[i]) / bound[i]
            worst = max(worst, float(ratio.max()))
            z = y.copy()
            z[H // 5] += 3 * bound[i][H // 5]
            assert (np.abs(z - proj[i]) / bound[i]).max() > 1.0
        print("largest emulated error / bound (K-quants)", worst)
        assert worst < 0.5
        assert worst > 1e-2
    finally:
        model.free()
