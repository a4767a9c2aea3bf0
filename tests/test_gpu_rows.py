"""Several rows a layer at a time (BASELINE config 3's ragged decode, and the
ABI's vitna_cuda_moe_rows_*), against the CPU checker run a step at a time.

Each row must give what its own step would: identical expert choice every
layer, logits within 1e-3 of max |cpu| (fp32 accumulation in another order).
Rows of one sequence at consecutive positions see each other's keys, as
consecutive steps would.
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import SMALL, rel, say

pytestmark = pytest.mark.gpu

REL = 1e-3


def model_with_cache(name, seed, prefill, seqs):
    return model_with_cache_spec(dict(SMALL[name]), seed, prefill, seqs)


def model_with_cache_spec(spec, seed, prefill, seqs):
    spec = dict(spec, seqs=seqs)
    model = va.Model(va.shape(**spec), seed)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L, ctx = cfg.n_layers, model.m.ctx
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(seqs, L, ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(seqs, L, ctx, kd))
    kc[:] = va.normal(seed, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(seed, 102, vc.size).reshape(vc.shape)
    dev = va.Device(model)
    for s in range(seqs):
        for l in range(L):
            dev.kv(s, l, 0, prefill[s], kc[s, l, :prefill[s]], vc[s, l, :prefill[s]])
    return model, dev


def cpu_rows(model, rows):
    """The CPU checker a step at a time, in the rows' order: (logits, chosen per layer) per row."""
    out = []
    for tok, pos, seq in rows:
        lg, _, tc, _ = oracle.step(model, seq, tok, pos)
        out.append((lg, tc))
    return out


@pytest.mark.parametrize("name", ["q8", "q4km"])
@pytest.mark.parametrize("exact", [True, False])
def test_rows_abi_layer_by_layer(name, exact):
    """model.c's moe_rows_on_gpu played by the test: rows up to the router on the device, the host routes each
    row, the device runs the experts: a single token's kernels a row (the pass is within vitna_hip_set_exact_rows'
    limit), or with the limit at 0 the multi-row projections and grouped experts. Two rows share sequence 1 at
    consecutive positions."""
    say("rows abi", name, "exact" if exact else "multi-row")
    prefill = [40, 17, 60]
    model, dev = model_with_cache(name, 777, prefill, 3)
    if not exact:
        dev.set_exact_rows(0)
    try:
        cfg = model.cfg
        K = cfg.n_experts_used
        rows = [(5, prefill[0], 0), (9, prefill[1], 1), (13, prefill[2], 2), (21, prefill[1] + 1, 1)]
        ref = cpu_rows(model, rows)
        for l in range(cfg.n_layers):
            lg = dev.rows_route(rows, l)
            ids, ws = [], []
            for i in range(len(rows)):
                ch, order, w = oracle.route(lg[i], K, bool(cfg.renormalize))
                assert np.array_equal(ch, ref[i][1][l]), ("row", i, "layer", l)
                ids.append(order)
                ws.append(w)
            dev.rows_experts(l, np.array(ids), np.array(ws))
        logits = dev.rows_head(len(rows))
        for i in range(len(rows)):
            r = rel(logits[i], ref[i][0])
            say("  row", i, "logits rel err", r)
            assert r <= REL
    finally:
        dev.close()
        model.free()


@pytest.mark.parametrize("name", ["q8", "q4km"])
def test_rows_step_device_routed(name):
    """vitna_hip_moe_rows_step: ragged rows of distinct sequences (config 3's shape, scaled down), routed and
    grouped on the device, replayed twice through one graph (the second pass one position on)."""
    say("rows step", name)
    seqs = 6
    prefill = [3, 70, 12, 45, 1, 66]
    model, dev = model_with_cache(name, 888, [p + 1 for p in prefill], seqs)
    try:
        for shift in (0, 1):
            rows = [(11 * s + 3, prefill[s] - 1 + shift, s) for s in range(seqs)]
            ref = cpu_rows(model, rows)
            logits = dev.rows_step(rows)
            for i in range(seqs):
                r = rel(logits[i], ref[i][0])
                assert r <= REL, ("row", i, r)
            say("  pass", shift, "max rel err", max(rel(logits[i], ref[i][0]) for i in range(seqs)))
    finally:
        dev.close()
        model.free()


@pytest.mark.parametrize("name", ["q8", "q4km", "q6gu"])
def test_rows_crowded_experts(name):
    """The grouped experts alone (the rows ABI with vitna_hip_set_exact_rows at 0), 24 rows on 16 (32) experts: about six tokens an expert, so experts take
    several four-token tiles, and the small models' short rows give the kernels' column split empty and
    odd-started ranges. Each layer: the device's residual rows before and after vitna_cuda_moe_rows_experts
    (routed by the host from the device's router logits, as model.c routes), against the CPU checker's
    mixture of the same rows. Layer by layer, so no error is carried into the next layer's input."""
    say("rows crowded experts", name)
    seqs = 24
    prefill = [1 + (7 * s) % 60 for s in range(seqs)]
    model, dev = model_with_cache(name, 999, prefill, seqs)
    dev.set_exact_rows(0)  # the grouped kernels, not a single token's a row
    try:
        cfg = model.cfg
        H, K = cfg.hidden, cfg.n_experts_used
        rows = [(5 * s + 1, prefill[s], s) for s in range(seqs)]
        most, worst = 0, 0.0
        for l in range(cfg.n_layers):
            norm = np.ctypeslib.as_array(model.m.layers[l].mlp_norm, shape=(H,)).copy()
            lg = dev.rows_route(rows, l)
            x0 = np.stack([dev.residual(i) for i in range(seqs)])
            ids, ws, projs = [], [], []
            for i in range(seqs):
                ch, order, w = oracle.route(lg[i], K, bool(cfg.renormalize))
                _, cch, _, _, proj = oracle.moe(model, l, oracle.rmsnorm(x0[i], norm, cfg.rms_eps))
                assert np.array_equal(ch, cch), ("row", i, "layer", l)
                ids.append(order)
                ws.append(w)
                projs.append(proj)
            most = max(most, int(np.bincount(np.concatenate(ids)).max()))
            dev.rows_experts(l, np.array(ids), np.array(ws))
            x1 = np.stack([dev.residual(i) for i in range(seqs)])
            for i in range(seqs):
                got = x1[i].astype(np.float64) - x0[i]
                r = float(np.max(np.abs(got - projs[i])) / np.max(np.abs(projs[i])))
                worst = max(worst, r)
                assert r <= REL, ("row", i, "layer", l, r)
        assert most > 4, "no expert took more than one tile"
        say("  most rows on one expert", most, "worst rel err of the mixture", worst)
    finally:
        dev.close()
        model.free()


WIDE = dict(n_layers=1, hidden=256, intermediate=256, n_heads=32, n_kv_heads=4, head_dim=128, vocab=40000,
            n_experts=8, n_experts_used=2, norm_std=0.1, ctx=40, kv_host=1)


@pytest.mark.parametrize("dt", ["k", "q8"])
def test_rows_wide_projections(dt):
    """Projections wider than 2048 columns (the o-projection's 4096 = 16 superblocks, two splits) are split across
    blocks, the last block of a tile adding the splits' sums in order; a head of 40000 rows (1250 tiles) takes the
    wide kernel, whose activations go through LDS; 36 rows take two token tiles. A rows step of 36 sequences
    against the CPU checker, twice through one graph, so the split counters must come back to zero."""
    say("rows wide projections", dt)
    spec = dict(WIDE)
    if dt == "q8":
        spec.update(dt_q=va.Q8_0, dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0, dt_head=va.Q8_0)
    seqs = 36
    prefill = [1 + (5 * s) % 30 for s in range(seqs)]
    spec["seqs"] = seqs
    model = va.Model(va.shape(**spec), 4242)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L, ctx = cfg.n_layers, model.m.ctx
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(seqs, L, ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(seqs, L, ctx, kd))
    kc[:] = va.normal(4242, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(4242, 102, vc.size).reshape(vc.shape)
    dev = va.Device(model)
    try:
        for s in range(seqs):
            dev.kv(s, 0, 0, prefill[s] + 1, kc[s, 0, :prefill[s] + 1], vc[s, 0, :prefill[s] + 1])
        for shift in (0, 1):
            rows = [(7 * s + 2, prefill[s] - 1 + shift, s) for s in range(seqs)]
            ref = cpu_rows(model, rows)
            logits = dev.rows_step(rows)
            worst = max(rel(logits[i], ref[i][0]) for i in range(seqs))
            say("  pass", shift, "max rel err", worst)
            assert worst <= REL
    finally:
        dev.close()
        model.free()


def _matrix(model, layer, which):
    m = model.m
    return [m.layers[layer].q, m.layers[layer].k, m.layers[layer].v, m.layers[layer].o, m.lm_head][which]


@pytest.mark.parametrize("name", ["q8", "q4km", "wide_k", "wide_q8"])
def test_rows_projections_isolated(name):
    """Each projection of a rows step alone (vitna_hip_rows_project) against the checker's widening of the same
    matrix times the same rows in float64: q, k, v, o of layer 0 and the head, for 5, 32 and 40 rows (one token
    tile, a full one, two). Independent of how well-conditioned a model's logits are, so the bound is tight:
    within 2e-5 of max |ref| (the activations' bf16 hi + lo split leaves about 2^-17 a product)."""
    say("rows projections", name)
    if name.startswith("wide"):
        spec = dict(WIDE, seqs=1)
        if name == "wide_q8":
            spec.update(dt_q=va.Q8_0, dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0, dt_head=va.Q8_0)
    else:
        spec = dict(SMALL[name])
    model = va.Model(va.shape(**spec), 5150)
    dev = va.Device(model)
    try:
        rng = np.random.RandomState(7)
        worst = 0.0
        for which in range(5):
            mat = _matrix(model, 0, which)
            W = oracle.widen(mat.bytes(), mat.dtype, mat.rows * mat.cols).reshape(mat.rows, mat.cols).astype(np.float64)
            for n in (5, 32, 40):
                x = rng.standard_normal((n, mat.cols)).astype(np.float32)
                y = dev.rows_project(0, which, x)
                ref = x.astype(np.float64) @ W.T
                r = float(np.max(np.abs(y - ref)) / np.max(np.abs(ref)))
                worst = max(worst, r)
                assert r <= 2e-5, (which, n, r)
        say("  worst rel err", worst)
    finally:
        dev.close()
        model.free()


@pytest.mark.parametrize("name", ["q4km", "q8", "wide_k"])
def test_rows_projections_token_tiles(name):
    """A pass of 200 rows (seven token tiles: the exact kernel takes two a block, the weights loaded once for both)
    against the same rows projected 32 at a time (one token tile a block): the same bits, q, k, v, o and the head."""
    say("rows projections, token tiles", name)
    spec = dict(WIDE, seqs=1) if name == "wide_k" else dict(SMALL[name])
    model = va.Model(va.shape(**spec), 6161)
    dev = va.Device(model)
    try:
        rng = np.random.RandomState(3)
        for which in range(5):
            mat = _matrix(model, 0, which)
            x = rng.standard_normal((200, mat.cols)).astype(np.float32)
            y = dev.rows_project(0, which, x)
            y32 = np.concatenate([dev.rows_project(0, which, x[i:i + 32]) for i in range(0, 200, 32)])
            assert np.array_equal(y.view(np.uint32), y32.view(np.uint32)), ("matrix", which)
    finally:
        dev.close()
        model.free()


NARROW = dict(n_layers=2, hidden=256, intermediate=256, n_heads=2, n_kv_heads=1, head_dim=64, vocab=300, n_experts=8,
              n_experts_used=2, renormalize=0, rms_eps=1e-5, rope_theta=10000.0, dt_gate_up=va.Q8_0, dt_down=va.Q8_0,
              dt_q=va.Q8_0, dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0, dt_head=va.Q8_0, dt_embed=va.Q8_0, norm_std=0.1,
              ctx=40, kv_host=1)


def test_rows_narrow_fallbacks():
    """An o-projection width that is not a multiple of 256 (2 heads x 64 = 128) takes the kernel that widens and
    splits each weight; head dimension 64 takes the fp32 vector attention. A rows step of 6 sequences against the
    CPU checker, and each projection alone (q, k, v and the head on the exact-integer kernel, o on the fallback)
    against the oracle in float64."""
    say("rows narrow fallbacks")
    seqs = 6
    prefill = [3, 17, 9, 30, 1, 22]
    model, dev = model_with_cache_spec(dict(NARROW), 3131, [p + 1 for p in prefill], seqs)
    try:
        rows = [(13 * s + 5, prefill[s] - 1, s) for s in range(seqs)]
        ref = cpu_rows(model, rows)
        logits = dev.rows_step(rows)
        worst = max(rel(logits[i], ref[i][0]) for i in range(seqs))
        say("  rows step max rel err", worst)
        assert worst <= REL
        rng = np.random.RandomState(11)
        for which in range(5):
            mat = _matrix(model, 0, which)
            W = oracle.widen(mat.bytes(), mat.dtype, mat.rows * mat.cols).reshape(mat.rows, mat.cols).astype(np.float64)
            x = rng.standard_normal((7, mat.cols)).astype(np.float32)
            y = dev.rows_project(0, which, x)
            ref_y = x.astype(np.float64) @ W.T
            r = float(np.max(np.abs(y - ref_y)) / np.max(np.abs(ref_y)))
            assert r <= 2e-5, (which, r)
    finally:
        dev.close()
        model.free()


@pytest.mark.parametrize("n", [1, 2, 3])
def test_rows_step_few_rows(n):
    """Passes of fewer than four rows take the multi-row GEMV for the projections (the matrix-core kernels start at
    four): a rows step of n sequences against the CPU checker."""
    say("rows step few rows", n)
    prefill = [12, 40, 5][:n]
    model, dev = model_with_cache("q4km", 600 + n, [p + 1 for p in prefill], n)
    try:
        rows = [(3 * s + 7, prefill[s] - 1, s) for s in range(n)]
        ref = cpu_rows(model, rows)
        logits = dev.rows_step(rows)
        worst = max(rel(logits[i], ref[i][0]) for i in range(n))
        say("  max rel err", worst)
        assert worst <= REL
    finally:
        dev.close()
        model.free()
