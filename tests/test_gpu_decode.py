"""Parity of the HIP decode path with the CPU checker (oracle/), on the GPU.

Bars:
  * widening: bit-exact (every weight of every format, two device reads);
  * the RMSNorm before the router and the router's logits: bit-exact, given
    the same residual (the device sums in the reference CPU's order);
  * top-k expert choice: identical, every layer;
  * expert outputs, residuals and vocab logits: max |gpu - cpu| <= 1e-3 of
    max |cpu| (fp32 accumulation in another order), with the reference's own
    LOGIT_ATOL of 1e-2 (reference/compare.mjs:84) also held.
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va

pytestmark = pytest.mark.gpu

REL = 1e-3


def same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("dtype,rows,cols,special", [(va.Q8_0, 64, 2048, False), (va.Q4_K, 48, 2048, False),
                                                      (va.Q6_K, 40, 768, False), (va.Q6_K, 8, 2048, True),
                                                      (va.Q4_K, 8, 4096, True), (va.Q8_0, 8, 1024, True)])
def test_widen_bit_exact(dtype, rows, cols, special):
    say("widen", dtype, rows, cols)
    buf = va.synth_matrix(dtype, 99, dtype, rows, cols, 0.02 / 127 if dtype == va.Q8_0 else 0.01)
    if special:
        # float16 scales that are subnormal, the largest, negative, zero, infinite, not a number
        be, bb = va.BLOCK[dtype]
        off = {va.Q8_0: 0, va.Q4_K: 0, va.Q6_K: 208}[dtype]
        for i, h in enumerate([0x0001, 0x03ff, 0x7bff, 0x8001, 0xbc00, 0x0000, 0x7c00, 0x7e00]):
            buf[i * bb + off:i * bb + off + 2] = np.frombuffer(np.uint16(h).tobytes(), np.uint8)
    m = va.matrix_from_bytes(buf, dtype, rows, cols)
    got = va.widen(m)
    want = oracle.widen(buf, dtype, rows * cols).reshape(rows, cols)
    if not special:
        assert same_bits(got, want)
        return
    # bit-exact wherever the checker's weight is a number or an infinity; where it is not a number (a NaN scale, or
    # an infinite scale times a zero quant) the device's weight is not a number either (the payload is not part of
    # the reference's contract: quant.c passes it through libm's float arithmetic)
    nan = np.isnan(want)
    assert nan.any() and np.array_equal(np.isnan(got), nan)
    assert same_bits(got[~nan], want[~nan])


def ffn_case(cfg_id, seed, x_tag):
    shp = va.shape(**va.CONFIGS[cfg_id])
    model = va.Model(shp, seed)
    dev = va.Device(model)
    return model, dev


@pytest.mark.parametrize("persistent", [False, True], ids=["graph", "persistent"])
@pytest.mark.parametrize("cfg_id", [0, 1])
def test_moe_layer_full_size(cfg_id, persistent):
    """BASELINE configs 0 and 1: one MoE layer, batch 1, full size, device routing; on the per-layer kernels and on
    the persistent step kernel."""
    say("moe layer config", cfg_id, "persistent" if persistent else "graph")
    model, dev = ffn_case(cfg_id, 1000 + cfg_id, 7)
    try:
        if persistent:
            assert dev.set_step_kernel(True)
        cfg = model.cfg
        H = cfg.hidden
        for trial in range(3):
            x = va.normal(77 + trial, 7, H)
            dev.set_residual(x)
            dev.ffn(0)
            out = dev.residual()
            lg_g, ch_g, ids_g, w_g = dev.routing()
            mlp_norm = np.ctypeslib.as_array(model.m.layers[0].mlp_norm, shape=(H,))
            xn = oracle.rmsnorm(x, mlp_norm, cfg.rms_eps)
            lg, ch, order, w, proj = oracle.moe(model, 0, xn, threads=16)
            assert same_bits(lg_g, lg), "router logits differ in bits"
            assert np.array_equal(ch_g, ch), (ch_g, ch)
            assert np.array_equal(ids_g, order)
            assert np.allclose(w_g, w, rtol=2e-6, atol=0)
            ref = (x + proj).astype(np.float32)
            r = float(np.max(np.abs(out.astype(np.float64) - ref)) / np.max(np.abs(proj)))
            say("  trial", trial, "chosen", list(ch), "rel err of the weighted sum", r)
            assert r <= REL
    finally:
        dev.close()
        model.free()


def test_expert_check_against_oracle():
    """vitna_cuda_expert_check: the norm bit-exact, the activation and output within tolerance."""
    say("expert check")
    model = va.Model(va.shape(**va.CONFIGS[1]), 31)
    try:
        cfg = model.cfg
        H, I = cfg.hidden, cfg.intermediate
        ex = model.m.layers[0].experts[5]
        mlp_norm = np.ctypeslib.as_array(model.m.layers[0].mlp_norm, shape=(H,)).copy()
        x = va.normal(5, 5, H)
        xs, act, y = va.expert_check(ex.gate, ex.up, ex.down, mlp_norm, x, cfg.rms_eps)
        xn = oracle.rmsnorm(x, mlp_norm, cfg.rms_eps)
        assert same_bits(xs, xn)
        g = oracle.matvec(ex.gate.data, ex.gate.dtype, xn, I, H)
        u = oracle.matvec(ex.up.data, ex.up.dtype, xn, I, H)
        a = oracle.silu_mul(g, u)
        assert rel(act, a) <= REL
        yy = oracle.matvec(ex.down.data, ex.down.dtype, a, H, I)
        assert rel(y, yy) <= REL
    finally:
        model.free()


SMALL = {
    "q8": dict(n_layers=2, hidden=256, intermediate=256, n_heads=4, n_kv_heads=2, head_dim=64, vocab=300,
               n_experts=16, n_experts_used=4, renormalize=0, rms_eps=1e-5, rope_theta=10000.0,
               dt_gate_up=va.Q8_0, dt_down=va.Q8_0, dt_q=va.Q8_0, dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0,
               dt_head=va.Q8_0, dt_embed=va.Q8_0, norm_std=0.1, ctx=80, seqs=2, kv_host=1),
    "q4km": dict(n_layers=3, hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
                 n_experts=32, n_experts_used=8, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1,
                 ctx=200, seqs=2, kv_host=1),
    # expert width 2048 with 8 experts a token: 512 (expert, slice) items a down row, 8 a lane (the down kernel's
    # one-row-at-a-time form), Q6_K and Q4_K down
    "wide_i": dict(n_layers=2, hidden=512, intermediate=2048, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
                   n_experts=16, n_experts_used=8, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1,
                   ctx=200, seqs=2, kv_host=1),
    "wide_i_q4": dict(n_layers=2, hidden=512, intermediate=2048, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
                      n_experts=16, n_experts_used=8, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q4_K, norm_std=0.1,
                      ctx=200, seqs=2, kv_host=1),
    # the merged attention and o-projection with a Q6_K o-projection, four head groups (parts) of four heads
    "q6o": dict(n_layers=2, hidden=512, intermediate=256, n_heads=16, n_kv_heads=4, head_dim=128, vocab=1000,
                n_experts=16, n_experts_used=4, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, dt_o=va.Q6_K,
                norm_std=0.1, ctx=200, seqs=2, kv_host=1),
    # Q6_K gate/up with Q4_K down (the grouped experts' one-wave-a-SIMD form for Q6_K)
    "q6gu": dict(n_layers=2, hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
                 n_experts=16, n_experts_used=4, renormalize=1, dt_gate_up=va.Q6_K, dt_down=va.Q4_K, norm_std=0.1,
                 ctx=200, seqs=2, kv_host=1),
    # two query heads: not a whole group of four, so the separate merge and o-projection GEMV
    "h2": dict(n_layers=2, hidden=256, intermediate=256, n_heads=2, n_kv_heads=1, head_dim=128, vocab=500,
               n_experts=16, n_experts_used=4, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1,
               ctx=200, seqs=2, kv_host=1),
}


def prefilled(name, seed, pos, seq=0):
    shp = va.shape(**SMALL[name])
    model = va.Model(shp, seed)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L, ctx = cfg.n_layers, model.m.ctx
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(model.m.seqs, L, ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(model.m.seqs, L, ctx, kd))
    kc[:] = va.normal(seed, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(seed, 102, vc.size).reshape(vc.shape)
    dev = va.Device(model)
    for s in range(model.m.seqs):
        for l in range(L):
            dev.kv(s, l, 0, pos, kc[s, l, :pos], vc[s, l, :pos])
    return model, dev, kc, vc


@pytest.mark.parametrize("name,pos,token", [("q8", 0, 3), ("q8", 65, 17), ("q4km", 130, 999), ("q4km", 63, 4),
                                            ("wide_i", 90, 12), ("wide_i_q4", 40, 77), ("q6o", 150, 21), ("h2", 130, 8)])
def test_abi_step_layer_by_layer(name, pos, token):
    """model.c's moe_step_on_gpu, played by the test: the device runs each layer up to its router, the host routes
    (the reference's rule), the device runs the experts. Router logits bit-exact given the device's residual; the
    choice identical to the CPU step's; logits within tolerance."""
    say("abi step", name, pos, token)
    model, dev, kc, vc = prefilled(name, 321, pos)
    try:
        cfg = model.cfg
        H, E, K = cfg.hidden, cfg.n_experts, cfg.n_experts_used
        seq = 1
        # the CPU step runs on the same cache (the host copy is the device's)
        ref_logits, ref_tl, ref_tc, ref_res = oracle.step(model, seq, token, pos)
        for l in range(cfg.n_layers):
            lg, nx = dev.moe_route(seq, token, pos, l, want_next=True)
            x = dev.residual()
            mlp_norm = np.ctypeslib.as_array(model.m.layers[l].mlp_norm, shape=(H,))
            xn = oracle.rmsnorm(x, mlp_norm, cfg.rms_eps)
            router = np.ctypeslib.as_array(C_f32(model.m.layers[l].router.data), shape=(E * H,))
            assert same_bits(lg, oracle.matvec(router, va.F32, xn, E, H)), "layer %d router" % l
            if l + 1 < cfg.n_layers:
                n_norm = np.ctypeslib.as_array(model.m.layers[l + 1].mlp_norm, shape=(H,))
                n_router = np.ctypeslib.as_array(C_f32(model.m.layers[l + 1].router.data), shape=(E * H,))
                assert same_bits(nx, oracle.matvec(n_router, va.F32, oracle.rmsnorm(x, n_norm, cfg.rms_eps), E, H))
            ch, order, w = oracle.route(lg, K, bool(cfg.renormalize))
            assert np.array_equal(ch, ref_tc[l]), "layer %d choice" % l
            dev.moe_experts(l, order, w)
            res = dev.residual()
            assert rel(res, ref_res[l]) <= REL, "layer %d residual" % l
        logits = dev.moe_head()
        r = rel(logits, ref_logits)
        say("  logits rel err", r, "max abs", float(np.max(np.abs(logits - ref_logits))))
        assert r <= REL
        assert np.max(np.abs(logits - ref_logits)) <= 1e-2
        # the keys and values the step wrote
        k, v = dev.kv(seq, cfg.n_layers - 1, pos, 1)
        assert rel(k[0], kc[seq, -1, pos]) <= REL and rel(v[0], vc[seq, -1, pos]) <= REL
    finally:
        dev.close()
        model.free()


def C_f32(addr):
    import ctypes
    return ctypes.cast(addr, ctypes.POINTER(ctypes.c_float))


@pytest.mark.parametrize("persistent", [False, True], ids=["graph", "persistent"])
@pytest.mark.parametrize("name,pos,token", [("q4km", 150, 7), ("q8", 79, 250), ("q4km", 192, 11), ("q4km", 199, 5),
                                            ("wide_i", 120, 3), ("q6o", 191, 40), ("h2", 64, 9)])
def test_device_step_matches_cpu(name, pos, token, persistent):
    """vitna_hip_moe_step (device routing, one graph): logits within tolerance of the CPU step, replayed at two
    positions through the same graph. Cases: mid-chunk; the last position of the context (q8: 79 of 80, q4km:
    199 of 200); 191 then 192, the last position of a full 64-position attention chunk then the first of the
    next."""
    say("device step", name, pos, token, "persistent" if persistent else "graph")
    model, dev, kc, vc = prefilled(name, 654, pos + 1)
    try:
        if persistent:
            dev.set_step_kernel(True)
        for p in (pos - 1, pos):
            ref_logits, _, ref_tc, _ = oracle.step(model, 0, token, p)
            logits = dev.step(0, token, p)
            lg, ch, ids, w = dev.routing()
            assert np.array_equal(ch, ref_tc[-1])
            r = rel(logits, ref_logits)
            say("  pos", p, "logits rel err", r)
            assert r <= REL
    finally:
        dev.close()
        model.free()


def routing_cases():
    rng = np.random.default_rng(11)
    cases = []
    for E, K in ((128, 8), (64, 8), (16, 4), (512, 16), (8, 8)):
        cases.append(("random E%d K%d" % (E, K), rng.normal(0, 1, E).astype(np.float32), K))
    ties = np.zeros(128, np.float32)
    ties[[3, 9, 17, 40, 41, 100]] = 2.0
    ties[[5, 6]] = 1.5
    cases.append(("ties", ties, 8))
    cases.append(("all equal", np.full(64, 0.25, np.float32), 8))
    q = np.round(rng.normal(0, 1, 128) * 4).astype(np.float32) / 4  # many exact duplicates
    cases.append(("quantized", q, 8))
    inf = rng.normal(0, 1, 128).astype(np.float32)
    inf[[7, 70]] = np.inf
    inf[[1, 2]] = -np.inf
    cases.append(("infinities", inf, 8))
    nan0 = rng.normal(0, 1, 128).astype(np.float32)
    nan0[0] = np.nan
    cases.append(("NaN first", nan0, 8))
    nanl = rng.normal(0, 1, 128).astype(np.float32)
    nanl[[5, 77]] = np.nan
    cases.append(("NaN later", nanl, 8))
    big = (rng.normal(0, 1, 128) * 40).astype(np.float32)
    cases.append(("wide range", big, 8))
    return cases


@pytest.mark.parametrize("renorm", [False, True])
def test_device_routing_rule(renorm):
    """The device's top-k / softmax / renormalization against the reference's rule (oracle.route), on crafted
    logits: ties (lower index first), duplicates, infinities, NaN where a pass starts and later. Choice and order
    identical; weights within 2 ulp-ish (the device's expf and sum order)."""
    for name, lg, K in routing_cases():
        say("routing", name, renorm)
        ch, ids, w = va.route_check(lg, K, renorm)
        rch, rorder, rw = oracle.route(lg, K, renorm)
        assert np.array_equal(ch, rch), (name, ch, rch)
        assert np.array_equal(ids, rorder), (name, ids, rorder)
        fin = np.isfinite(rw)
        assert np.array_equal(fin, np.isfinite(w)), name
        assert np.allclose(w[fin], rw[fin], rtol=3e-6, atol=0), (name, w, rw)
