"""Passes of rows through the reference's rows ABI give each row the bits of its own step.

model.c checks drafted tokens (generate --speculate) and runs a server's batched steps as passes of rows
(vitna_llama_steps_exact / vitna_llama_step_rows -> moe_rows_on_gpu, engine/src/model.c:810-833, 1052-1190), and
takes every row as "the one a step would give" (main.c:1003-1007): the same tokens and logits with drafts or
without (main.c:96-99). Passes of at most 64 rows (PASS_MAX) therefore run each row through the kernels of a
single token's step here (several rows a launch); the bar is bit-equality with the same rows run one at a time
through vitna_cuda_moe_route / _experts / _head, for:
  * rows of one sequence at consecutive positions (a drafted pass: each row's key stored before the others read
    it), across an attention chunk boundary;
  * rows of different sequences, and a mix of both;
  * 64 rows of 64 sequences;
  * the merged attention + o-projection (Q4_K, Q6_K and Q8_0 o-projections) and the separate merge + GEMV (two
    query heads);
  * a model whose experts pass through the expert cache: a pass whose experts fit one wave of its rule, and one
    taken in groups of rows.
Each row's router logits at every layer, its final logits and the keys and values it stored are compared.
"""
import numpy as np
import pytest

import oracle
import vitna_amd as va
from test_gpu_decode import SMALL, say

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


def make(spec, seed, prefill, expert_cache_bytes=0):
    """A model and a device whose sequences hold prefill[s] positions of seeded keys and values."""
    model = va.Model(va.shape(**spec), seed)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L, ctx, S = cfg.n_layers, model.m.ctx, model.m.seqs
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(S, L, ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(S, L, ctx, kd))
    kc[:] = va.normal(seed, 101, kc.size).reshape(kc.shape)
    vc[:] = va.normal(seed, 102, vc.size).reshape(vc.shape)
    devs = []
    for ecb in (0, expert_cache_bytes):
        dev = va.Device(model, expert_cache_bytes=ecb)
        for s in range(S):
            for l in range(L):
                if prefill[s]:
                    dev.kv(s, l, 0, prefill[s], kc[s, l, :prefill[s]], vc[s, l, :prefill[s]])
        devs.append(dev)
    return model, devs[0], devs[1]


def one_at_a_time(dev, cfg, rows):
    """Each row as its own step through the single-token ABI, in order: (router logits per layer, logits)."""
    K, ren = cfg.n_experts_used, bool(cfg.renormalize)
    out = []
    for tok, pos, seq in rows:
        lgs = []
        for l in range(cfg.n_layers):
            lg = dev.moe_route(seq, tok, pos, l)
            _, order, w = oracle.route(lg, K, ren)
            dev.moe_experts(l, order, w)
            lgs.append(lg)
        out.append((lgs, dev.moe_head()))
    return out


def as_pass(dev, cfg, rows):
    """The rows as one pass of the rows ABI, layer by layer with the host's routing (moe_rows_on_gpu)."""
    K, ren = cfg.n_experts_used, bool(cfg.renormalize)
    lgs = []
    for l in range(cfg.n_layers):
        lg = dev.rows_route(rows, l)
        ids, ws = [], []
        for i in range(len(rows)):
            _, order, w = oracle.route(lg[i], K, ren)
            ids.append(order)
            ws.append(w)
        dev.rows_experts(l, np.array(ids), np.array(ws))
        lgs.append(lg)
    return lgs, dev.rows_head(len(rows))


def check(cfg, rows, single, pas, dev_a, dev_b):
    lgs, logits = pas
    for i, (tok, pos, seq) in enumerate(rows):
        for l in range(cfg.n_layers):
            assert same_bits(single[i][0][l], lgs[l][i]), ("router logits", "row", i, "layer", l)
        assert same_bits(single[i][1], logits[i]), ("logits", "row", i)
        for l in range(cfg.n_layers):
            ka, va_ = dev_a.kv(seq, l, pos, 1)
            kb, vb = dev_b.kv(seq, l, pos, 1)
            assert same_bits(ka, kb) and same_bits(va_, vb), ("cache", "row", i, "layer", l)


CASES = {
    # a drafted pass: one sequence, consecutive positions across the 64-position chunk boundary
    "drafted": lambda p: [(5, p[0], 0), (9, p[0] + 1, 0), (13, p[0] + 2, 0), (21, p[0] + 3, 0)],
    # a server's batched step: two sequences, one row each
    "batched": lambda p: [(7, p[0], 0), (11, p[1], 1)],
    # both: two rows of sequence 1, one of sequence 0
    "mixed": lambda p: [(3, p[1], 1), (8, p[0], 0), (17, p[1] + 1, 1)],
}


@pytest.mark.parametrize("name", ["q8", "q4km", "q6o", "h2"])
@pytest.mark.parametrize("case", ["drafted", "batched", "mixed"])
def test_pass_rows_are_step_bits(name, case):
    say("exact rows", name, case)
    prefill = [62, 40]
    model, single_dev, pass_dev = make(dict(SMALL[name]), 1357, prefill)
    try:
        cfg = model.cfg
        rows = CASES[case](prefill)
        single = one_at_a_time(single_dev, cfg, rows)
        pas = as_pass(pass_dev, cfg, rows)
        check(cfg, rows, single, pas, single_dev, pass_dev)
        # after the pass, a single token's step on each device: the same bits (the pass left nothing behind)
        tok, pos, seq = max(rows, key=lambda r: (r[2] == rows[0][2], r[1]))
        nxt = [(tok + 1, pos + 1, seq)]
        a, b = one_at_a_time(single_dev, cfg, nxt), one_at_a_time(pass_dev, cfg, nxt)
        assert same_bits(a[0][1], b[0][1]), "the step after the pass"
        with pytest.raises(va.VitnaError, match="twice"):
            pass_dev.rows_route(rows, 0)
            ids = np.tile(np.arange(cfg.n_experts_used), (len(rows), 1))
            ids[-1, 1] = ids[-1, 0]
            pass_dev.rows_experts(0, ids, np.full(ids.shape, 0.125))
    finally:
        single_dev.close()
        pass_dev.close()
        model.free()


def test_sixty_four_rows():
    """The most rows a pass of model.c checks (PASS_MAX): 64 sequences at ragged positions, one row each, and the
    same 64 rows again one position on."""
    say("exact rows, 64 sequences")
    spec = dict(SMALL["q4km"], seqs=64, ctx=96)
    prefill = [(13 * s) % 90 for s in range(64)]
    model, single_dev, pass_dev = make(spec, 2468, prefill)
    try:
        cfg = model.cfg
        for shift in (0, 1):
            rows = [((29 * s + 5) % cfg.vocab, prefill[s] + shift, s) for s in range(64)]
            single = one_at_a_time(single_dev, cfg, rows)
            pas = as_pass(pass_dev, cfg, rows)
            check(cfg, rows, single, pas, single_dev, pass_dev)
    finally:
        single_dev.close()
        pass_dev.close()
        model.free()


def test_longer_pass_takes_multi_row_kernels():
    """65 rows (past PASS_MAX) and a pass after vitna_hip_set_exact_rows(0) take the multi-row kernels: their
    logits within 1e-3 of max |step|, and not all of the step's bits (the sums run in another order)."""
    say("exact rows: the multi-row kernels past the limit")
    spec = dict(SMALL["q4km"], seqs=65, ctx=96)
    prefill = [(7 * s) % 80 for s in range(65)]
    model, single_dev, pass_dev = make(spec, 97531, prefill)
    try:
        cfg = model.cfg
        rows = [((31 * s + 2) % cfg.vocab, prefill[s], s) for s in range(65)]
        single = one_at_a_time(single_dev, cfg, rows)
        _, logits = as_pass(pass_dev, cfg, rows)
        worst = max(float(np.max(np.abs(logits[i] - single[i][1])) / np.max(np.abs(single[i][1]))) for i in range(65))
        say("  65 rows: logits rel err against the steps", worst)
        assert worst <= 1e-3
        assert not all(same_bits(single[i][1], logits[i]) for i in range(65))
        with pytest.raises(va.VitnaError):
            pass_dev.set_exact_rows(65)
        pass_dev.set_exact_rows(0)
        rows2 = [(tok, pos + 1, seq) for tok, pos, seq in rows[:4]]
        single2 = one_at_a_time(single_dev, cfg, rows2)
        _, logits2 = as_pass(pass_dev, cfg, rows2)
        worst2 = max(float(np.max(np.abs(logits2[i] - single2[i][1])) / np.max(np.abs(single2[i][1]))) for i in range(4))
        say("  4 rows with the limit at 0: logits rel err", worst2)
        assert worst2 <= 1e-3
    finally:
        single_dev.close()
        pass_dev.close()
        model.free()


@pytest.mark.parametrize("extra", [20, 0])
def test_cached_experts_pass_is_step_bits(extra):
    """A model with an expert cache of 2K + extra slots, the steps' bits of the same model with every expert
    resident. With 20 extra (the rule's waves take 28 experts) a drafted pass of three rows names at most 24: one
    wave. With none (waves of K experts) every row is a group of its own, a pass of the cache each."""
    say("exact rows through the expert cache, 2K +", extra, "slots")
    spec = dict(SMALL["q4km"])
    from test_gpu_expert_cache import slot_bytes
    model0 = va.Model(va.shape(**spec), 8642)
    sb = slot_bytes(model0.cfg, spec)
    model0.free()
    K = spec["n_experts_used"]
    prefill = [50, 30]
    model, single_dev, pass_dev = make(spec, 8642, prefill, expert_cache_bytes=(2 * K + extra) * sb)
    try:
        cfg = model.cfg
        for p in (50, 53):
            rows = [(5, p, 0), (6, p + 1, 0), (7, p + 2, 0)]
            single = one_at_a_time(single_dev, cfg, rows)
            pas = as_pass(pass_dev, cfg, rows)
            check(cfg, rows, single, pas, single_dev, pass_dev)
        _, cnt = pass_dev.expert_cache_state()
        say("  cache", cnt)
        assert cnt["slots"] == 2 * K + extra
    finally:
        single_dev.close()
        pass_dev.close()
        model.free()
