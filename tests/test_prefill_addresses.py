"""Host-side bounds of the prefill GEMM kernels' global memory accesses (no GPU).

The index arithmetic of prefill_wgemm_kernel (pw_body) and prefill_gemm_kernel
(vitna-anchor_amd/csrc/kernels_prefill.hip), restated over every work item a
plan makes and every lane, load slot and stage, and every byte range each load
touches checked against its buffer:
  - the activations: gate/up reads xb [n][H] bf16 at the row a pair names
    (pairs[e][p] / 16), down reads act [n K][I] bf16 at the expert's pair
    offset; stages 0 .. S - 1, each 16 bytes at chunk position c of a 128-byte
    stage row;
  - the weights: the per-wave kernel reads the experts' tiled copy
    ([E][rows / 64][cols / 128][8704] bytes), the shared-stage kernel the
    planes of each dtype (its pf_bgroup loads);
  - the outputs: act rows pbase + p for p < cnt, ypart rows row K + slot.
A plan is what group_kernel and prefill_plan_kernel build: each expert's pairs
in row order, tiles of 256 pairs. The check runs on random routings, on
routings that crowd every row onto a few experts (tiles of up to 65535 rows'
pairs), and at the row counts the entry points admit (1 .. 65536), so an
address a diagnostic build moves past its buffer shows up here before any GPU
run.
"""
import numpy as np
import pytest

Q8, Q4, Q6 = 14, 17, 19
KMAX = 16  # ROUTE_K_MAX: pairs hold row * 16 + slot
BM = 256


def plan(chosen, E):
    """counts, offsets, pairs (each expert's pair codes in row order) and the tile list."""
    n, K = chosen.shape
    pairs = [[] for _ in range(E)]
    for r in range(n):
        for s in range(K):
            pairs[chosen[r, s]].append(r * KMAX + s)
    count = np.array([len(p) for p in pairs])
    off = np.concatenate([[0], np.cumsum(count)[:-1]])
    tiles = [(e, i) for e in range(E) for i in range((count[e] + BM - 1) // BM)]
    return count, off, pairs, tiles


def act_rows_wgemm(pairs, count, off, e, m0, gate_up, ML):
    """Rows of xb (gate/up) or act (down) pw_body's activation loads read: slot (wv NA + i) 64 + lane, row slot / 8,
    clamped to the expert's last pair."""
    sl = np.arange(4 * ML * 64)
    pa = np.minimum(m0 + (sl >> 3), count[e] - 1)
    if gate_up:
        return np.array([pairs[e][p] // KMAX for p in pa])
    return off[e] + pa


def check_plan(chosen, E, H, I, dts=(Q8, Q8)):
    n, K = chosen.shape
    count, off, pairs, tiles = plan(chosen, E)
    xb_bytes, act_bytes, yp_bytes = n * H * 2, n * K * I * 2, n * K * H * 2
    for gate_up in (True, False):
        KD = H if gate_up else I
        S = KD // 64
        NT = I // 128 if gate_up else H // 256
        # the activations: the last stage's last 16-byte chunk of the farthest row (both kernels share the layout)
        for e, t in tiles:
            m0 = t * BM
            rows = count[e] - m0
            ML = 8 if rows > 128 else 4 if rows > 64 else 2
            r = act_rows_wgemm(pairs, count, off, e, m0, gate_up, ML)
            width = H if gate_up else I
            lo = int(r.min()) * width * 2
            hi = int(r.max()) * width * 2 + 16 * 7 + (S - 1) * 128 + 16
            assert lo >= 0 and hi <= (xb_bytes if gate_up else act_bytes), (gate_up, e, t, hi)
            # the outputs
            last = count[e] - 1
            if gate_up:
                assert (off[e] + last) * I * 2 + I * 2 <= act_bytes
            else:
                code = pairs[e][last]
                assert ((code // KMAX) * K + code % KMAX + 1) * H * 2 <= yp_bytes
                assert code % KMAX < K and code // KMAX < n
        # the per-wave kernel's weights (Q8_0 tiled copy): the farthest 8-byte quant load and 4-byte scale load of
        # the expert's last row group and column block
        rows_w, cols_w = (I, H) if gate_up else (H, I)
        units = cols_w // 128
        stride = (rows_w // 64) * units * 8704
        for nt in range(NT):
            for wv in range(4):
                for tt in range(2):
                    r0 = nt * 128 + wv * 32 if gate_up else nt * 256 + wv * 64 + tt * 32
                    assert r0 + 31 < rows_w
                    g0 = (E - 1) * stride + (r0 >> 6) * units * 8704
                    rin = (r0 & 32) + 31
                    x = S - 1
                    u = (x >> 1) * 8704
                    q_end = g0 + rin * 16 + 8 + u + (4 * (x & 1) + 3) * 1024 + 8
                    d_end = g0 + 8192 + rin * 8 + u + 4 * (x & 1) + 4
                    assert q_end <= E * stride and d_end <= E * stride
        # the shared-stage kernel's weights from the planes: thread (bn, bh) reads group g = 2 s + bh of row wrow
        dt = dts[0] if gate_up else dts[1]
        nb = cols_w // (32 if dt == Q8 else 256)
        last_row = rows_w - 1
        g = 2 * (S - 1) + 1
        if dt == Q8:
            assert ((E - 1) * rows_w * nb + last_row * nb + g) * 32 + 32 <= E * rows_w * nb * 32
            assert ((E - 1) * rows_w * nb + last_row * nb + g) * 2 + 2 <= E * rows_w * nb * 2
        else:
            blk = (E - 1) * rows_w * nb + last_row * nb + (g >> 3)
            gi = g & 7
            if dt == Q4:
                assert blk * 128 + 32 * (gi >> 1) + 32 <= E * rows_w * nb * 128
                assert blk * 16 + 16 <= E * rows_w * nb * 16
            else:
                h, rr = gi >> 2, gi & 3
                assert blk * 128 + 64 * h + 32 * (rr & 1) + 32 <= E * rows_w * nb * 128
                assert blk * 64 + 32 * h + 32 <= E * rows_w * nb * 64
                assert blk * 16 + 8 * h + 2 * rr + 2 <= E * rows_w * nb * 16
                assert blk * 2 + 2 <= E * rows_w * nb * 2
    return len(tiles)


def random_choice(rng, n, E, K):
    return np.stack([rng.choice(E, K, replace=False) for _ in range(n)]).astype(np.int32)


@pytest.mark.parametrize("n,E,K,H,I", [(1, 16, 4, 256, 256), (37, 16, 4, 512, 256), (300, 32, 8, 512, 256),
                                       (4096, 128, 8, 2048, 768), (1025, 64, 8, 2048, 1024)])
def test_random_plans_stay_in_bounds(n, E, K, H, I):
    rng = np.random.default_rng(n)
    for dts in ((Q8, Q8), (Q4, Q6), (Q6, Q4)):
        check_plan(random_choice(rng, n, E, K), E, H, I, dts)


@pytest.mark.parametrize("n", [255, 256, 257, 513, 4096, 65536])
def test_crowded_plans_stay_in_bounds(n):
    """Every row on the same K experts: one expert per slot holds n pairs, up to 256 tiles of one expert (the tile
    index's 16 bits), the longest tails and the last tile's clamp."""
    E, K, H, I = 16, 8, 256, 256
    chosen = np.tile(np.arange(K, dtype=np.int32), (n, 1))
    tiles = check_plan(chosen, E, H, I)
    assert tiles == K * ((n + BM - 1) // BM)
    assert (n + BM - 1) // BM - 1 < 1 << 16
