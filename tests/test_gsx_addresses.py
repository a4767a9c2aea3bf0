"""The index arithmetic of the crowded passes' grouped kernels (launch_gsx, vitna-anchor_amd/csrc/kernels_skinny.hip),
restated on the CPU: every load and store of the plan, the gathers, gate/up and down stays inside the buffer the
engine allocates for it (ensure_tiled: operand images 32 T x width x 4 bytes, sums T x (width / 256) x 1536 bytes
and twice that, the SwiGLU output 32 T x I floats, ypart ROWS_MAX x K x H floats, the tiled copies
E x rows / 32 x cols / 256 tiles), and every pair a tile names is one of its expert's, on random routings and on
routings that crowd every row onto the same K experts, at 64 to 1024 rows.
"""
import numpy as np
import pytest

ROUTE_K_MAX = 16
ROWS_MAX = 1024
TILE_BYTES = {"q4k": 4608, "q6k": 6720, "q8": 8704}


def max_tiles(n, K, E):
    return (n * K + 31) // 32 + E


def plan(count):
    tiles = (count + 31) // 32
    off = np.concatenate([[0], np.cumsum(tiles)])
    te = np.full(off[-1], -1)
    for e in range(len(count)):
        te[off[e]:off[e + 1]] = e
    return off, te


def img_piece(row, K, c8, order):
    """img_put's piece index (u32x4 units) of columns 8 c8 .. of row `row`, and the hi/lo offset."""
    tt, l, b, c = row >> 5, row & 31, c8 >> 5, 8 * (c8 & 31)
    base = (tt * (K // 256) + b) * 2048
    if order == "a":
        U, r = c >> 6, c & 63
        i, kq = ((r >> 5) << 1) | ((r >> 3) & 1), (r >> 4) & 1
    else:
        r = c & 127
        U, i, kq = 2 * (c >> 7) + ((r >> 5) & 1), ((r >> 4) & 1) + 2 * (r >> 6), (r >> 3) & 1
    return base + ((U * 4 + i) * 2) * 64 + l + 32 * kq + np.array([0, 64])


def sum_index(row, K, g, gran):
    """img_sum32 / img_sum16's uint16 indices of group g's three pieces."""
    tt, l, w, gi = row >> 5, row & 31, g >> 3, g & 7
    per = K // (256 if gran == 32 else 128)
    return (((tt * per + w) * 3 * 64 + l + 32 * (gi >> 2)) * 4 + (gi & 3)) + 256 * np.arange(3)


def check(n, K, E, H, I, ids, dt_gu="q4k", dt_dn="q6k"):
    T = max_tiles(n, K, E)
    W = max(H, I)
    count = np.bincount(ids.ravel(), minlength=E)
    pairs = [[r * ROUTE_K_MAX + s for r in range(n) for s in range(K) if ids[r, s] == e] for e in range(E)]
    off, te = plan(count)
    assert off[-1] <= T, "tiles past max_tiles"
    img_in_pieces, img_act_pieces = 32 * T * H * 4 // 16, 32 * T * I * 4 // 16
    s32_elems, s16_elems = T * (W // 256) * 1536 // 2, T * (W // 128) * 1536 // 2
    rows = np.arange(32)
    for t in range(off[-1]):
        e = te[t]
        j0 = 32 * (t - off[e])
        assert 0 <= j0 < count[e]
        idx = np.minimum(j0 + rows, count[e] - 1)
        src = np.array([pairs[e][j] // ROUTE_K_MAX for j in idx])
        assert src.max() < n
        vrow = 32 * t + rows
        # gathers: reads of xn (n x H) and of the SwiGLU output (32 T x I), writes of both images and the sums
        assert (src.max() + 1) * H <= n * H and (vrow.max() + 1) * I <= 32 * T * I
        for K_, pieces in ((H, img_in_pieces), (I, img_act_pieces)):
            for c8 in (0, K_ // 8 - 1):
                for order in "ab":
                    assert img_piece(int(vrow.max()), K_, c8, order).max() < pieces
            assert sum_index(int(vrow.max()), K_, K_ // 32 - 1, 32).max() < s32_elems
            assert sum_index(int(vrow.max()), K_, K_ // 16 - 1, 16).max() < s16_elems
        # gate/up: weight tile e I / 32 + x of the tiled copy; the SwiGLU output's rows of the tile
        for x in (0, I // 32 - 1):
            tile = e * (I // 32) + x
            assert ((tile * (H // 256) + H // 256 - 1) + 1) * TILE_BYTES[dt_gu] <= E * (I // 32) * (H // 256) * TILE_BYTES[dt_gu]
        assert ((32 * t + 31) * I + I - 1) < 32 * T * I
        # down: two weight tiles a block (K-quants) from 2 blockIdx.x; ypart of the tile's real pairs only
        nr = 2 if dt_dn != "q8" else 1
        for bx in (0, H // (32 * nr) - 1):
            for r in range(nr):
                tile = e * (H // 32) + nr * bx + r
                assert tile < E * (H // 32)
        for j in range(j0, min(j0 + 32, count[e])):
            p = pairs[e][j]
            row, slot = p // ROUTE_K_MAX, p % ROUTE_K_MAX
            assert ids[row, slot] == e
            assert ((row * K + slot) * H + H - 1) < ROWS_MAX * K * H
    # every pair of every expert lands in exactly one tile slot
    assert sum(min(32, count[te[t]] - 32 * (t - off[te[t]])) for t in range(off[-1])) == n * K


@pytest.mark.parametrize("n,K,E,H,I", [(64, 8, 128, 2048, 768), (1024, 8, 128, 2048, 768), (520, 8, 32, 512, 256),
                                       (600, 4, 16, 256, 256), (1024, 4, 16, 512, 256)])
def test_random_routing(n, K, E, H, I):
    rng = np.random.default_rng(n * 7 + E)
    ids = np.stack([np.sort(rng.choice(E, K, replace=False)) for _ in range(n)])
    check(n, K, E, H, I, ids)
    check(n, K, E, H, I, ids, dt_gu="q8", dt_dn="q8")


@pytest.mark.parametrize("n", [64, 333, 1024])
def test_crowded_routing(n):
    """Every row on the same K experts: each of them holds n pairs (n / 32 tiles, the last part-filled)."""
    K, E = 8, 128
    ids = np.tile(np.arange(3, 3 + K), (n, 1))
    check(n, K, E, 2048, 768, ids)
