"""The expert-cache rule the tests check the device against (oracle/expert_cache.py), pinned by sequences worked
out by hand from the reference's rule (engine/src/model_cuda.cu free_slot :4334, fill :4355,
vitna_cuda_moe_experts :4757-4913)."""
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
from expert_cache import ExpertCache  # noqa: E402


def test_worked_sequence():
    # 2 layers of 8 experts, k = 2, 4 slots; an expert copies 100 bytes in layer 0 and 150 in layer 1
    c = ExpertCache(2, 8, 4, [100, 150])
    # layer 0 wants 0 and 1: two misses into the empty slots 0 and 1 (clock 1, 2); the guess's upper half (one
    # place, expert 2 of layer 1) goes to slot 2 (clock 3)
    assert c.experts(0, [0, 1], guess=[2, 3]) == [0, 1]
    assert c.where[8 + 2] == 2 and c.prefetched == 1
    # layer 1 wants 2 (present, a used guess; clock 4) and 4 (a miss into empty slot 3, clock 5)
    assert c.experts(1, [2, 4]) == [2, 3]
    assert c.prefetch_used == 1
    # layer 0 wants 0 (present, clock 6) and 5: no slot is empty; of those not held (1, 2, 3) every place has been
    # used once, so the least recently used, slot 1 (expert 1 of layer 0, clock 2), is given up
    assert c.experts(0, [0, 5], guess=[4, 6]) == [0, 1]
    assert c.where[1] == -1 and c.where[5] == 1
    # the guess's upper half is expert 4 of layer 1, present: nothing copied
    assert c.counters() == dict(acquired=6, present=2, misses=4, prefetched=1, prefetch_used=1, copies=5,
                                bytes_copied=100 + 100 + 150 + 150 + 100)
    assert c.where == [0, -1, -1, -1, -1, 1, -1, -1] + [-1, -1, 2, -1, 3, -1, -1, -1]


def test_least_used_kept_over_recent():
    # 1 layer of 8 experts, k = 1, 2 slots: expert 0 used three times stays; the once-used ones take turns
    c = ExpertCache(1, 8, 2, [10])
    for e in (0, 0, 0, 1, 2, 3):
        c.experts(0, [e])
    assert c.where[0] >= 0 and c.where[3] >= 0 and c.where[1] == -1 and c.where[2] == -1
    assert c.misses == 4 and c.present == 2


def test_held_places_never_given_up():
    # k = 2, 4 slots full of layer 0's experts; a request naming two new experts gives up neither of its own
    c = ExpertCache(1, 8, 4, [1])
    c.experts(0, [0, 1])
    c.experts(0, [2, 3])
    slots = c.experts(0, [4, 5])
    assert sorted(slots) == [0, 1] and c.where[4] >= 0 and c.where[5] >= 0
    for e in (4, 5):
        assert c.place[c.where[e]] == e


def test_uses_halved_every_65536():
    c = ExpertCache(1, 4, 2, [1])
    for i in range(65535):
        c.experts(0, [i % 2])
    assert c.uses[0] == 32768 and c.uses[1] == 32767
    c.experts(0, [0])  # the 65,536th acquisition: every count halved after counting
    assert c.uses[0] == 32769 // 2 and c.uses[1] == 32767 // 2
    assert c.acquired == 65536


def test_counters_add_up():
    import random
    rnd = random.Random(5)
    c = ExpertCache(3, 16, 9, [7, 8, 9])
    for t in range(200):
        for l in range(3):
            ids = rnd.sample(range(16), 4)
            guess = rnd.sample(range(16), 4) if l < 2 else None
            slots = c.experts(l, ids, guess)
            assert len(set(slots)) == 4
            for e, s in zip(ids, slots):
                assert c.place[s] == l * 16 + e
    k = c.counters()
    assert k["acquired"] == 200 * 3 * 4 == k["present"] + k["misses"]
    assert k["copies"] == k["misses"] + k["prefetched"]
    assert k["prefetch_used"] <= k["prefetched"]
    # where and the slots' places agree
    for s, p in enumerate(c.place):
        if p >= 0:
            assert c.where[p] == s
    assert sum(1 for w in c.where if w >= 0) == sum(1 for p in c.place if p >= 0)


def test_rows_worked_sequence():
    # a pass of rows (model_cuda.cu:5134-5386): 2 layers of 8 experts, k = 2, 4 slots, so waves of 2 experts
    c = ExpertCache(2, 8, 4, [100, 150])
    # three rows want {0, 1}, {1, 3}, {5, 1}: experts 0, 1, 3, 5 in order; wave (0, 1) misses both, expert 1's other
    # two rows are hits; the pair fills slots 0 and 1 (clock 1, 2); wave (3, 5) fills slots 2 and 3 (clock 3, 4)
    slots = c.rows_experts(0, [[0, 1], [1, 3], [5, 1]], guess=[[2, 4], [2, 6], [7, 2]])
    assert slots == {0: 0, 1: 1, 3: 2, 5: 3}
    # the guess's upper half per row: 2 (then 2 again, once), 7. The last wave's slots 2, 3 are still held; of 0 and 1,
    # slot 0's expert was used once, slot 1's three times: 2 goes to slot 0 (clock 5), 7 to slot 1 (clock 6)
    assert c.where[:8] == [-1, -1, -1, 2, -1, 3, -1, -1]
    assert c.where[8:] == [-1, -1, 0, -1, -1, -1, -1, 1]
    assert c.counters() == dict(acquired=6, present=2, misses=4, prefetched=2, prefetch_used=0, copies=6,
                                bytes_copied=4 * 100 + 2 * 150)
    # layer 1, rows {2, 7}, {2, 4}: wave (2, 4): 2 present twice (a used guess, clock 7), 4 a miss; of the slots not
    # held, 1 (expert 7 of layer 1), 2 and 3 were each used once, slot 2 least recently (clock 3): 4 goes there
    # (clock 8). Wave (7): present in slot 1 (a used guess)
    slots = c.rows_experts(1, [[2, 7], [2, 4]])
    assert slots == {2: 0, 4: 2, 7: 1}
    assert c.where[3] == -1 and c.where[8 + 4] == 2
    assert c.counters() == dict(acquired=10, present=5, misses=5, prefetched=2, prefetch_used=2, copies=7,
                                bytes_copied=4 * 100 + 3 * 150)


def test_rows_halving_on_crossing():
    # the counts are halved when a pass's requests cross a multiple of 65,536, not only when they land on one
    c = ExpertCache(1, 4, 2, [1])
    c.rows_experts(0, [[0]] * 65534)
    assert c.uses[0] == 65534
    c.rows_experts(0, [[1]] * 3)
    assert c.acquired == 65537 and c.uses[0] == 32767 and c.uses[1] == 1


def test_rows_match_single_rows():
    # a pass of one row asks for what a step asks for: same slots, same counts as the step's rule
    import random
    rnd = random.Random(9)
    a = ExpertCache(3, 16, 9, [7, 8, 9])
    b = ExpertCache(3, 16, 9, [7, 8, 9])
    for t in range(300):
        for l in range(3):
            ids = sorted(rnd.sample(range(16), 4))
            guess = rnd.sample(range(16), 4) if l < 2 else None
            sa = a.experts(l, ids, guess)
            sb = b.rows_experts(l, [ids], [guess] if guess else None)
            assert [sb[e] for e in ids] == sa
    assert a.counters() == b.counters() and a.where == b.where
