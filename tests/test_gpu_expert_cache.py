"""The expert cache on the GPU (vitna_cuda_create's expert_cache_bytes; the reference's expert_cache_t,
engine/src/model_cuda.cu:249-290 and vitna_cuda_moe_experts :4757-4913).

A model whose cache holds fewer slots than it has experts runs the reference's layer-at-a-time step
(vitna_cuda_moe_route, the host's routing, vitna_cuda_moe_experts with the next layer's guess) and must give the
same bits as the same model with every expert resident, since the same kernels read the same bytes from a slot.
Which expert each slot holds, and the counts of the report, must be what the reference's rule gives for the same
requests (oracle/expert_cache.py); hits and copies still running at the request are one count there, as timing
decides between them."""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from expert_cache import ExpertCache

pytestmark = pytest.mark.gpu

SHAPE = dict(n_layers=3, hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000, n_experts=32,
             n_experts_used=8, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1, ctx=200, seqs=2,
             kv_host=1)


def say(*a):
    print(*a, flush=True)


def same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


def slot_bytes(cfg, spec=SHAPE):
    """A slot: gate, up and down, each matrix's planes 256-byte aligned (Q4_K: 128 + 16 bytes a 256-column block,
    Q6_K: 128 + 64 + 16 + 2, Q8_0: 32 + 2 a 32-column block)."""
    a = lambda x: (x + 255) // 256 * 256
    planes = {va.Q4_K: (256, (128, 16)), va.Q6_K: (256, (128, 64, 16, 2)), va.Q8_0: (32, (32, 2))}

    def mat(dt, rows, cols):
        width, fields = planes[dt]
        return sum(a(rows * (cols // width) * b) for b in fields)
    gu = mat(spec["dt_gate_up"], cfg.intermediate, cfg.hidden)
    return 2 * gu + mat(spec["dt_down"], cfg.hidden, cfg.intermediate)


def fill_kv(model, dev, pos):
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(model.m.seqs, cfg.n_layers, model.m.ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(model.m.seqs, cfg.n_layers, model.m.ctx, kd))
    for s in range(model.m.seqs):
        for l in range(cfg.n_layers):
            dev.kv(s, l, 0, pos, kc[s, l, :pos], vc[s, l, :pos])


@pytest.mark.parametrize("extra_slots", [0, 5])
def test_cached_experts_match_resident(extra_slots):
    say("expert cache, slots 2K +", extra_slots)
    model = va.Model(va.shape(**SHAPE), 777)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(model.m.seqs, cfg.n_layers, model.m.ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(model.m.seqs, cfg.n_layers, model.m.ctx, kd))
    kc[:] = va.normal(777, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(777, 102, vc.size).reshape(vc.shape)
    K, E, L = cfg.n_experts_used, cfg.n_experts, cfg.n_layers
    sb = slot_bytes(cfg)
    n_slots = 2 * K + extra_slots
    res = va.Device(model)
    cac = va.Device(model, expert_cache_bytes=n_slots * sb + sb // 2)
    try:
        where, cnt = cac.expert_cache_state()
        assert cnt["slots"] == n_slots and cnt["slot_bytes"] == sb
        assert (where == -1).all()
        sim = ExpertCache(L, E, n_slots, [sb] * L)
        pos0 = 40
        fill_kv(model, res, pos0)
        fill_kv(model, cac, pos0)
        seq = 1
        for t, token in enumerate([5, 17, 999, 5, 300, 17]):
            pos = pos0 + t
            for l in range(L):
                outs = []
                for dev in (res, cac):
                    lg, nx = dev.moe_route(seq, token, pos, l, want_next=True)
                    ch, order, w = oracle.route(lg, K, bool(cfg.renormalize))
                    guess = oracle.route(nx, K, bool(cfg.renormalize))[0] if l + 1 < L else None
                    dev.moe_experts(l, order, w, guess)
                    outs.append((ch, dev.residual()))
                    if dev is cac:
                        sim.experts(l, order, guess)
                assert np.array_equal(outs[0][0], outs[1][0]), "token %d layer %d choice" % (t, l)
                assert same_bits(outs[0][1], outs[1][1]), "token %d layer %d residual" % (t, l)
            assert same_bits(res.moe_head(), cac.moe_head()), "token %d logits" % t
        where, cnt = cac.expert_cache_state()
        ref = sim.counters()
        say("  device", cnt)
        say("  rule  ", ref)
        assert where.tolist() == sim.where
        assert cnt["acquired"] == ref["acquired"] and cnt["hits"] + cnt["in_flight"] == ref["present"]
        for k in ("misses", "prefetched", "prefetch_used", "copies", "bytes_copied"):
            assert cnt[k] == ref[k], k
        assert ref["misses"] > 0 and ref["present"] > 0 and ref["prefetched"] > 0
        rep = cac.moe_report()
        say("  report:", rep)
        assert ("%d slots" % n_slots) in rep and ("%d acquired" % ref["acquired"]) in rep
    finally:
        cac.close()
        res.close()
        model.free()


def test_cache_limits():
    say("expert cache limits")
    model = va.Model(va.shape(**SHAPE), 778)
    cfg = model.cfg
    sb = slot_bytes(cfg)
    try:
        # fewer slots than twice the experts a token goes through: refused, as the reference refuses it
        with pytest.raises(va.VitnaError, match="twice the experts"):
            va.Device(model, expert_cache_bytes=(2 * cfg.n_experts_used - 1) * sb)
        # room for every expert: all resident, no cache
        dev = va.Device(model, expert_cache_bytes=cfg.n_layers * cfg.n_experts * sb)
        try:
            with pytest.raises(va.VitnaError, match="resident"):
                dev.expert_cache_state()
        finally:
            dev.close()
        # the paths that read every expert in place refuse a cached model
        dev = va.Device(model, expert_cache_bytes=2 * cfg.n_experts_used * sb)
        try:
            with pytest.raises(va.VitnaError, match="cache of 16 slots"):
                dev.step(0, 3, 0)
            rows = [(3, 0, 0), (4, 0, 1)]
            with pytest.raises(va.VitnaError, match="cache of 16 slots"):
                dev.rows_step(rows)
            # a pass of rows through the cache checks its requests before it touches the cache
            dev.rows_route(rows, 0)
            K = cfg.n_experts_used
            ok = np.tile(np.arange(K, dtype=np.int32), (2, 1))
            w = np.full((2, K), 1.0 / K, np.float32)
            twice = ok.copy()
            twice[1, 1] = twice[1, 0]
            with pytest.raises(va.VitnaError, match="named twice"):
                dev.rows_experts(0, twice, w)
            outside = ok.copy()
            outside[0, 3] = cfg.n_experts
            with pytest.raises(va.VitnaError, match="outside"):
                dev.rows_experts(0, outside, w)
            with pytest.raises(va.VitnaError, match="outside"):
                dev.rows_experts(0, ok, w, guess=outside)
            with pytest.raises(va.VitnaError, match="routes to"):
                dev.rows_experts(0, ok[:, :K - 1], w[:, :K - 1])
            # one token's experts: the same checks before any slot is taken
            with pytest.raises(va.VitnaError, match="named twice"):
                dev.moe_experts(0, twice[1], w[1])
            with pytest.raises(va.VitnaError, match="outside"):
                dev.moe_experts(0, outside[0], w[0])
            _, cnt = dev.expert_cache_state()
            assert cnt["acquired"] == 0 and cnt["copies"] == 0
            dev.rows_experts(0, ok, w, guess=ok)
            _, cnt = dev.expert_cache_state()
            assert cnt["acquired"] == 2 * K and cnt["misses"] == K and cnt["prefetched"] == (K + 1) // 2
        finally:
            dev.close()
    finally:
        model.free()


@pytest.mark.parametrize("extra_slots,q8", [(0, False), (20, False), (0, True)])
def test_cached_rows_match_resident(extra_slots, q8):
    """Passes of rows through the cache (vitna_cuda_moe_rows_experts, model_cuda.cu:5134-5386): at 2K slots the
    rows' experts go in several waves, at 2K + 20 in one. Interleaved with single-token steps, which move experts
    between slots under the rows' tiled copies. Bits as with every expert resident; slots and counts as the rule."""
    say("expert cache rows, slots 2K +", extra_slots, "Q8_0 experts" if q8 else "")
    spec = dict(SHAPE, dt_gate_up=va.Q8_0, dt_down=va.Q8_0) if q8 else SHAPE
    model = va.Model(va.shape(**spec), 779)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(model.m.seqs, cfg.n_layers, model.m.ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(model.m.seqs, cfg.n_layers, model.m.ctx, kd))
    kc[:] = va.normal(779, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(779, 102, vc.size).reshape(vc.shape)
    K, E, L = cfg.n_experts_used, cfg.n_experts, cfg.n_layers
    sb = slot_bytes(cfg, spec)
    n_slots = 2 * K + extra_slots
    res = va.Device(model)
    cac = va.Device(model, expert_cache_bytes=n_slots * sb)
    # the grouped experts on both (a pass of several waves takes them on the cached model whatever the limit)
    res.set_exact_rows(0)
    cac.set_exact_rows(0)
    try:
        sim = ExpertCache(L, E, n_slots, [sb] * L)
        pos0 = 50
        fill_kv(model, res, pos0)
        fill_kv(model, cac, pos0)
        passes = [[(5, pos0, 0), (17, pos0, 1), (999, pos0 + 1, 1), (300, pos0 + 1, 0), (42, pos0 + 2, 0), (7, pos0 + 2, 1)],
                  "step",
                  [(11, pos0 + 3, 1), (12, pos0 + 4, 0), (13, pos0 + 4, 1)]]
        for pi, rows in enumerate(passes):
            if rows == "step":
                # one token through the single-token path: it moves experts between slots
                for l in range(L):
                    outs = []
                    for dev in (res, cac):
                        lg, nx = dev.moe_route(0, 77, pos0 + 3, l, want_next=True)
                        ch, order, w = oracle.route(lg, K, bool(cfg.renormalize))
                        guess = oracle.route(nx, K, bool(cfg.renormalize))[0] if l + 1 < L else None
                        dev.moe_experts(l, order, w, guess)
                        outs.append(dev.residual())
                        if dev is cac:
                            sim.experts(l, order, guess)
                    assert same_bits(outs[0], outs[1]), "step layer %d" % l
                continue
            n = len(rows)
            for l in range(L):
                outs = []
                for dev in (res, cac):
                    lg, nx = dev.rows_route(rows, l, want_next=True)
                    ids, ws, gs = [], [], []
                    for i in range(n):
                        ch, order, w = oracle.route(lg[i], K, bool(cfg.renormalize))
                        ids.append(order)
                        ws.append(w)
                        if l + 1 < L:
                            gs.append(oracle.route(nx[i], K, bool(cfg.renormalize))[0])
                    dev.rows_experts(l, np.array(ids), np.array(ws), np.array(gs) if gs else None)
                    outs.append((np.array(ids), [dev.residual(i) for i in range(n)]))
                    if dev is cac:
                        sim.rows_experts(l, ids, gs if gs else None)
                assert np.array_equal(outs[0][0], outs[1][0]), "pass %d layer %d choice" % (pi, l)
                for i in range(n):
                    assert same_bits(outs[0][1][i], outs[1][1][i]), "pass %d layer %d row %d residual" % (pi, l, i)
            assert same_bits(res.rows_head(n), cac.rows_head(n)), "pass %d logits" % pi
            where, cnt = cac.expert_cache_state()
            ref = sim.counters()
            say("  pass", pi, "device", cnt)
            say("  pass", pi, "rule  ", ref)
            assert where.tolist() == sim.where, "pass %d slots" % pi
            assert cnt["acquired"] == ref["acquired"] and cnt["hits"] + cnt["in_flight"] == ref["present"]
            for k in ("misses", "prefetched", "prefetch_used", "copies", "bytes_copied"):
                assert cnt[k] == ref[k], (pi, k)
    finally:
        cac.close()
        res.close()
        model.free()
