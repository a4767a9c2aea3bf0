"""vitna_hip_host_route (the reference's host routing, engine/src/model.c:626-703, offered to callers of the
layer-at-a-time ABI) against the checker's route (oracle/vitna_oracle.c orc_route): bit-exact choice, order and
weights, on seeded logits and on ties, signed zeros, infinities and NaNs. Host code: runs without a GPU."""
import numpy as np
import pytest

import oracle
import vitna_amd as va


def cases():
    rng = np.random.RandomState(11)
    out = []
    for E, K in ((16, 4), (64, 8), (128, 8), (32, 8)):
        for _ in range(20):
            out.append((rng.standard_normal(E).astype(np.float32), K))
    lg = np.zeros(32, np.float32)
    out.append((lg, 8))                                    # all equal: the lowest ids
    lg = rng.standard_normal(32).astype(np.float32)
    lg[[3, 9, 20]] = 2.5                                   # a three-way tie at the top
    out.append((lg, 8))
    lg = np.array([-0.0, 0.0] * 8, np.float32)             # signed zeros compare equal
    out.append((lg, 4))
    lg = rng.standard_normal(16).astype(np.float32)
    lg[5], lg[7] = np.inf, -np.inf
    out.append((lg, 4))
    lg = rng.standard_normal(16).astype(np.float32)
    lg[0] = np.nan                                          # a NaN where every pass starts is kept
    out.append((lg, 4))
    lg = rng.standard_normal(16).astype(np.float32)
    lg[6] = np.nan                                          # a later NaN never wins
    out.append((lg, 4))
    return out


@pytest.mark.parametrize("renorm", [False, True])
def test_host_route_matches_checker(renorm):
    for lg, K in cases():
        ch, order, w = va.host_route(lg, K, renorm)
        rch, rorder, rw = oracle.route(lg, K, renorm)
        assert np.array_equal(ch, rch) and np.array_equal(order, rorder), (lg, ch, rch)
        assert np.array_equal(w.view(np.uint32), np.asarray(rw, np.float32).view(np.uint32)), (lg, w, rw)


def test_host_route_refuses_bad_shapes():
    with pytest.raises(va.VitnaError):
        va.host_route(np.zeros(4, np.float32), 5, False)
