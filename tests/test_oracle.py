"""The CPU checker (oracle/) pinned before anything is compared with it.

Checks, in order of independence from the oracle's own code:
  * golden vectors written by the reference engine's own compiled C code
    (tests/golden/make_golden.py -> ref_vectors.npz): widening of every block
    format, including float16 scales that are subnormal, infinite or NaN;
    vitna_matvec for each dtype and shape; vitna_rmsnorm; vitna_silu_mul; and
    whole vitna_llama_step calls on three synthetic models, router traced;
  * known answers built by an encoder (values chosen, packed into blocks the
    way the formats define, then decoded), brute force over every 6-bit scale
    and min of Q4_K and every 6-bit quant of Q6_K;
  * a double-precision bound on the matvec, and the routing rule's special
    cases (ties, NaN, renormalization).
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle
import vitna_amd as va

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


@pytest.mark.parametrize("name,dtype,be", [("q8_0", va.Q8_0, 32), ("q4_k", va.Q4_K, 256), ("q6_k", va.Q6_K, 256)])
def test_dequant_golden(gold, name, dtype, be):
    blocks = gold["dequant.%s.blocks" % name]
    out = gold["dequant.%s.out" % name]
    assert same_bits(oracle.widen(blocks, dtype, out.size), out)


MATVEC = [("q8_0.16x2048", va.Q8_0, 16, 2048), ("q8_0.8x1024", va.Q8_0, 8, 1024), ("q4_k.16x2048", va.Q4_K, 16, 2048),
          ("q4_k.4x4096", va.Q4_K, 4, 4096), ("q6_k.16x768", va.Q6_K, 16, 768), ("q6_k.8x2048", va.Q6_K, 8, 2048),
          ("f32.16x2048", va.F32, 16, 2048), ("f32.5x100", va.F32, 5, 100)]


@pytest.mark.parametrize("name,dtype,rows,cols", MATVEC)
def test_matvec_golden(gold, name, dtype, rows, cols):
    w = gold["matvec.%s.w" % name]
    x = gold["matvec.%s.x" % name]
    y = gold["matvec.%s.y" % name]
    assert same_bits(oracle.matvec(w, dtype, x, rows, cols), y)
    assert same_bits(oracle.matvec(w, dtype, x, rows, cols, threads=3), y)
    # the bound of engine/tests/unit_tests.c:761-807: within 2e-5 of sum |w x| of the double-precision product
    wf = oracle.widen(w, dtype, rows * cols).reshape(rows, cols).astype(np.float64)
    exact = wf @ x.astype(np.float64)
    bound = 2e-5 * (np.abs(wf) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - exact) <= bound)


@pytest.mark.parametrize("n", [2048, 128, 24, 7, 40])
def test_rmsnorm_golden(gold, n):
    i = [2048, 128, 24, 7, 40].index(n)
    x, w, y = gold["rmsnorm.%d.x" % n], gold["rmsnorm.%d.w" % n], gold["rmsnorm.%d.y" % n]
    assert same_bits(oracle.rmsnorm(x, w, 1e-5 if i & 1 else 1e-6), y)
    # the double formula
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + (1e-5 if i & 1 else 1e-6)) * w
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_silu_golden(gold):
    g, u, o = gold["silu.g"], gold["silu.u"], gold["silu.out"]
    got = oracle.silu_mul(g, u)
    assert same_bits(got, o)


STEPS = {
    "q8": dict(n_layers=2, hidden=256, intermediate=128, n_heads=4, n_kv_heads=2, head_dim=64, vocab=300,
               n_experts=16, n_experts_used=4, renormalize=0, rms_eps=1e-5, rope_theta=10000.0,
               dt_gate_up=va.Q8_0, dt_down=va.Q8_0, dt_q=va.Q8_0, dt_k=va.Q8_0, dt_v=va.Q8_0, dt_o=va.Q8_0,
               dt_head=va.Q8_0, dt_embed=va.Q8_0, norm_std=0.1, ctx=16, seqs=1, kv_host=1),
}
STEPS["q4km"] = dict(STEPS["q8"], hidden=512, intermediate=256, n_heads=8, n_kv_heads=2, renormalize=1, rms_eps=1e-6,
                     rope_theta=1e6, dt_gate_up=va.Q4_K, dt_down=va.Q6_K, dt_q=va.Q4_K, dt_k=va.Q4_K, dt_v=va.Q6_K,
                     dt_o=va.Q4_K, dt_head=va.Q6_K, dt_embed=va.Q4_K)
STEPS["e64k8"] = dict(STEPS["q8"], n_layers=1, intermediate=256, n_experts=64, n_experts_used=8)
STEP_ARGS = {"q8": (4242, 9, 17), "q4km": (4343, 11, 250), "e64k8": (4444, 3, 5)}


def make_step_model(name):
    seed, pos, token = STEP_ARGS[name]
    m = va.Model(va.shape(**STEPS[name]), seed)
    cfg = m.cfg
    n = m.m.seqs * cfg.n_layers * m.m.ctx * cfg.n_kv_heads * cfg.head_dim
    kc = np.ctypeslib.as_array(m.m.k_cache, shape=(n,))
    vc = np.ctypeslib.as_array(m.m.v_cache, shape=(n,))
    kc[:] = va.normal(seed, 101, n)
    vc[:] = va.normal(seed, 102, n)
    return m, pos, token


@pytest.mark.parametrize("name", list(STEPS))
def test_step_golden(gold, name):
    m, pos, token = make_step_model(name)
    try:
        logits, tl, tc, res = oracle.step(m, 0, token, pos)
        assert same_bits(tl.ravel(), gold["step.%s.router" % name])
        assert np.array_equal(tc.ravel(), gold["step.%s.chosen" % name])
        assert same_bits(res[-1], gold["step.%s.resid" % name])
        assert same_bits(logits, gold["step.%s.logits" % name])
        cfg = m.cfg
        kd = cfg.n_kv_heads * cfg.head_dim
        kc = np.ctypeslib.as_array(m.m.k_cache, shape=(cfg.n_layers, m.m.ctx, kd))
        vc = np.ctypeslib.as_array(m.m.v_cache, shape=(cfg.n_layers, m.m.ctx, kd))
        kv = np.concatenate([kc[:, pos].ravel(), vc[:, pos].ravel()])
        assert same_bits(kv, gold["step.%s.kv" % name])
    finally:
        m.free()


def test_generator_reproduces_golden_inputs(gold):
    """The synthetic inputs the golden vectors were made from come back bit for bit."""
    w = va.synth_matrix(va.Q4_K, 555 + 2, 9, 16, 2048, 0.01)
    assert np.array_equal(w, gold["matvec.q4_k.16x2048.w"])
    x = va.normal(556 + 2, 10, 2048)
    assert same_bits(x, gold["matvec.q4_k.16x2048.x"])


# ---- known answers from an encoder ------------------------------------------

def f16(x):
    return int(np.float16(x).view(np.uint16))


def test_q8_0_known_answer():
    q = np.array([(i * 37) % 255 - 127 for i in range(32)], np.int8)
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(0xB000).tobytes(), np.uint8)  # -0.125
    blk[2:] = q.view(np.uint8)
    got = oracle.widen(blk, va.Q8_0, 32)
    assert same_bits(got, q.astype(np.float32) * np.float32(-0.125))


def pack_q4k(d, dmin, sc, mn, q):
    """Encode a Q4_K block: six-bit scales and mins as ggml packs them, nibbles group by group."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(f16(dmin)).tobytes(), np.uint8)
    s = b[4:16]
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    for i in range(256):
        g, l = divmod(i, 32)
        b[16 + 32 * (g // 2) + l] |= (int(q[i]) & 15) << (4 if g & 1 else 0)
    return b


def test_q4_k_brute_force_scales_and_mins():
    """Every (scale, min) pair of 0..63 in every group decodes to (d*sc)*q - (dmin*mn)."""
    rng = np.random.default_rng(7)
    d, dmin = 0.5, 0.25
    q = rng.integers(0, 16, 256)
    blocks, want = [], []
    for a in range(64):
        for g0 in range(8):
            sc = rng.integers(0, 64, 8)
            mn = rng.integers(0, 64, 8)
            sc[g0] = a
            mn[(g0 + 3) % 8] = a
            mn[g0] = 63 - a
            blocks.append(pack_q4k(d, dmin, sc, mn, q))
            w = np.empty(256, np.float32)
            for i in range(256):
                g = i // 32
                p = np.float32(np.float32(d) * np.float32(sc[g])) * np.float32(q[i])
                w[i] = np.float32(p - np.float32(np.float32(dmin) * np.float32(mn[g])))
            want.append(w)
    got = oracle.widen(np.concatenate(blocks), va.Q4_K, 256 * len(blocks))
    assert same_bits(got, np.concatenate(want))


def pack_q6k(d, scales, q):
    b = np.zeros(210, np.uint8)
    for i in range(256):
        h, r, l = i // 128, (i % 128) // 32, i % 32
        b[64 * h + 32 * (r & 1) + l] |= (int(q[i]) & 15) << (4 * (r >> 1))
        b[128 + 32 * h + l] |= ((int(q[i]) >> 4) & 3) << (2 * r)
    b[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(f16(d)).tobytes(), np.uint8)
    return b


def test_q6_k_brute_force_quants():
    """Every six-bit quant in every position of the block decodes to (d*sc)*(q-32)."""
    rng = np.random.default_rng(8)
    blocks, want = [], []
    for shift in range(64):
        q = (np.arange(256) + shift) % 64
        scales = rng.integers(-32, 32, 16)
        blocks.append(pack_q6k(0.25, scales, q))
        w = np.array([np.float32(np.float32(0.25) * np.float32(scales[i // 16])) * np.float32(q[i] - 32)
                      for i in range(256)], np.float32)
        want.append(w)
    got = oracle.widen(np.concatenate(blocks), va.Q6_K, 256 * len(blocks))
    assert same_bits(got, np.concatenate(want))


def test_f16_every_value():
    """Every float16 bit pattern converts as numpy's float16 does (subnormals, infinities, NaN payload class)."""
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert same_bits(got[~nan], ref[~nan])


# ---- routing -------------------------------------------------------------------

def test_top_k_ties_lower_index_first():
    assert list(oracle.top_k(np.array([1, 3, 3, 2, 3], np.float32), 3)) == [1, 2, 4]
    assert list(oracle.top_k(np.zeros(8, np.float32), 4)) == [0, 1, 2, 3]


def test_top_k_nan_first_candidate_is_kept():
    # a NaN where the scan starts is never displaced; a later NaN never wins
    assert oracle.top_k(np.array([np.nan, 5, 1], np.float32), 1)[0] == 0
    assert oracle.top_k(np.array([1, np.nan, 5], np.float32), 1)[0] == 2


def test_route_weights():
    rng = np.random.default_rng(3)
    lg = rng.normal(0, 1, 128).astype(np.float32)
    ch, order, w = oracle.route(lg, 8, False)
    assert list(order) == sorted(ch)
    p = np.exp(lg.astype(np.float64) - lg.max())
    p /= p.sum()
    assert np.allclose(w, p[order], rtol=1e-6)
    ch2, order2, w2 = oracle.route(lg, 8, True)
    assert np.array_equal(order, order2)
    assert np.allclose(w2, p[order] / p[order].sum(), rtol=1e-6)
    assert abs(float(np.sum(w2, dtype=np.float64)) - 1.0) < 1e-6
