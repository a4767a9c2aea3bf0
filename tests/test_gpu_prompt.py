"""A prompt through the rows path: passes of many rows of ONE sequence at consecutive positions, as model.c feeds
a prompt in chunks of vitna_cuda_moe_rows_max (engine/src/model.c:1006-1030). Such a pass (more rows than
vitna_hip_set_exact_rows' limit) takes the attention kernel that reads each chunk of keys and values once for a tile
of rows (attention_flash_kernel), where passes of rows of several sequences read them once a row.

Bars:
  * a 1024-row pass and a 90-row pass after it, as the device-routed rows step and through the ABI layer by layer
    with the routing the step chose (the host's rule picks the same experts): the same logits bits (the same
    kernels); sampled rows' router logits bit-exact against the checker's norm and router on the device's residual
    (a pass of 128 rows or more takes the prefill's norm and router kernels); every layer's experts identical to the checker's step of sampled rows over the device's cache,
    their logits within 1e-3 of max |cpu|;
  * query groups of 4 (tiles of 16 rows) and of 8 query heads a key-value head (tiles of 8 rows), and a pass whose
    row count leaves the last tile part-filled;
  * the same pass with every row of another sequence added to it takes the per-row kernel: the one-sequence rows
    within 1e-3 of that pass's (sums in another order).
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import C_f32, SMALL, rel, same_bits, say

pytestmark = pytest.mark.gpu

SPECS = {
    "g4": dict(SMALL["q4km"], seqs=2, ctx=1200),
    "g8": dict(n_layers=2, hidden=512, intermediate=256, n_heads=16, n_kv_heads=2, head_dim=128, vocab=1000,
               n_experts=16, n_experts_used=4, renormalize=1, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, norm_std=0.1,
               ctx=1200, seqs=2, kv_host=1),
}


def abi_pass(model, dev, rows, dev_rt):
    """The rows through the ABI layer by layer, each row given the routing the device-routed step chose (the host's
    rule picks the same experts from the same logits; the device's weights are used so that the same kernels see
    the same inputs)."""
    cfg = model.cfg
    K, ren = cfg.n_experts_used, bool(cfg.renormalize)
    E, H = cfg.n_experts, cfg.hidden
    chosen = []
    for l in range(cfg.n_layers):
        lg = dev.rows_route(rows, l)
        # router logits bit-exact against the checker's norm and router on the device's residual rows
        norm = np.ctypeslib.as_array(model.m.layers[l].mlp_norm, shape=(H,))
        router = np.ctypeslib.as_array(C_f32(model.m.layers[l].router.data), shape=(E * H,))
        for i in (0, len(rows) // 3, len(rows) - 1):
            xn = oracle.rmsnorm(dev.residual(i), norm, cfg.rms_eps)
            assert same_bits(lg[i], oracle.matvec(router, va.F32, xn, E, H)), ("router logits", "layer", l, "row", i)
        ids = np.array([dev_rt[l][i][1] for i in range(len(rows))])
        ws = np.array([dev_rt[l][i][2] for i in range(len(rows))])
        ch = []
        for i in range(len(rows)):
            c, order, w = oracle.route(lg[i], K, ren)
            assert np.array_equal(order, ids[i]), ("layer", l, "row", i)
            ch.append(c)
        dev.rows_experts(l, ids, ws)
        chosen.append(ch)
    return dev.rows_head(len(rows)), chosen


def check_rows(model, dev, rows, logits, chosen, sample):
    cfg = model.cfg
    L, kd = cfg.n_layers, cfg.n_kv_heads * cfg.head_dim
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(model.m.seqs, L, model.m.ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(model.m.seqs, L, model.m.ctx, kd))
    worst = 0.0
    for i in sample:
        tok, pos, seq = rows[i]
        for l in range(L):
            if pos:
                k, v = dev.kv(seq, l, 0, pos)
                kc[seq, l, :pos] = k
                vc[seq, l, :pos] = v
        ref, _, tc, _ = oracle.step(model, seq, tok, pos)
        for l in range(L):
            assert np.array_equal(np.sort(chosen[l][i]), np.sort(tc[l])), ("row", i, "layer", l)
        worst = max(worst, rel(logits[i], ref))
    return worst


@pytest.mark.parametrize("name", ["g4", "g8"])
def test_prompt_passes(name):
    say("prompt passes", name)
    model = va.Model(va.shape(**SPECS[name]), 777)
    a, b = va.Device(model), va.Device(model)
    try:
        cfg = model.cfg
        worst = 0.0
        for start, n in ((0, 1024), (1024, 90)):
            rows = [((13 * (start + i) + 5) % cfg.vocab, start + i, 0) for i in range(n)]
            lb = np.stack(b.rows_step(rows))
            dev_rt = [[b.rows_routing(l, i) for i in range(n)] for l in range(cfg.n_layers)]
            la, chosen = abi_pass(model, a, rows, dev_rt)
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), ("pass at", start)
            worst = max(worst, check_rows(model, a, rows, la, chosen, (0, 1, 63, 64, n // 2, n - 2, n - 1)))
        say("  logits rel err against the checker (sampled rows)", worst)
        assert worst <= 1e-3
    finally:
        a.close()
        b.close()
        model.free()


def test_prompt_against_per_row_kernel():
    """A 300-row pass of sequence 0 (tiles) against the same rows with one row of sequence 1 appended (the per-row
    kernel for every row): the sequence-0 rows within 1e-3 of max |logits| of each other."""
    say("prompt tiles against the per-row kernel")
    model = va.Model(va.shape(**SPECS["g8"]), 4321)
    a, b = va.Device(model), va.Device(model)
    try:
        cfg = model.cfg
        rows = [((11 * i + 3) % cfg.vocab, i, 0) for i in range(300)]
        la = np.stack(a.rows_step(rows))
        lb = np.stack(b.rows_step(rows + [(7, 0, 1)]))[:300]
        worst = max(rel(la[i], lb[i]) for i in range(300))
        say("  tiles against per-row: max rel diff", worst)
        assert worst <= 1e-3
    finally:
        a.close()
        b.close()
        model.free()


def test_prompt_head_rows():
    """A pass of more rows than the exact limit that asks one row's logits (a prompt's last chunk, model.c:1011)
    runs the head on that row alone, and one that asks none runs no head: the asked row's logits within 1e-5 of
    max |logits| of the all-rows head (another kernel), and after a pass with no logits and one with one row, the
    all-rows pass gives its first bits again (each head form its own captured graph)."""
    say("prompt head rows")
    model = va.Model(va.shape(**SPECS["g8"]), 2468)
    dev = va.Device(model)
    try:
        cfg = model.cfg
        n = 200
        rows = [((17 * i + 1) % cfg.vocab, i, 0) for i in range(n)]
        full = np.stack(dev.rows_step(rows))
        dev.rows_step(rows, logits=False)
        one = dev.rows_step(rows, only=[n - 1])[n - 1]
        r = float(np.max(np.abs(one - full[n - 1])) / np.max(np.abs(full[n - 1])))
        say("  one row's head against the all-rows head: rel diff", r)
        assert r <= 1e-5
        again = np.stack(dev.rows_step(rows))
        assert np.array_equal(again.view(np.uint32), full.view(np.uint32))
    finally:
        dev.close()
        model.free()
