"""The reference's GPU expert-cache rule, restated in Python for the tests.

Test infrastructure only: the tests compare the device library's cache state
(vitna_hip_expert_cache_state) with this simulation of the same requests. The
library never imports it.

Reference: engine/src/model_cuda.cu
  - expert_cache_t :249-290 (slots, where, uses halved every 65,536, clock);
  - free_slot :4334-4352 (an empty slot, else the least used of those not
    held, the least recently used between equals);
  - fill :4355-4391 (the slot takes the place, is held, last_use = ++clock);
  - vitna_cuda_moe_experts :4757-4913, the path without the expert stream or
    the CPU split: every requested place counts a use; held places are hits
    (or in flight, when their copy has not finished: timing, which this
    simulation cannot see, so it counts both as "present"); the places lacking
    are filled in request order; after the kernels, the first ceil(k / 2)
    places of the guess that the device lacks are filled while a slot is free;
    then every hold is released.
  - vitna_cuda_moe_rows_experts :5134-5386, the same without the expert
    stream: each wanted expert counts one use per row that wants it (the
    halving when the count crosses a multiple of 65,536); the wanted experts,
    in order of expert, go in waves of at most n_slots - k: a wave releases
    the previous wave's holds, holds the experts present (hits, or in flight,
    counted once per row) and fills those lacking k at a time, a miss for the
    first row and hits for the others; after the last wave, of each row's
    guess the first ceil(k / 2) experts, each once, are filled while a slot is
    free; then every hold is released.
"""


class ExpertCache:
    def __init__(self, n_layers, n_experts, n_slots, expert_bytes):
        self.E = n_experts
        self.n_places = n_layers * n_experts
        self.n_slots = n_slots
        self.expert_bytes = list(expert_bytes)  # bytes a fill copies, per layer
        self.place = [-1] * n_slots
        self.held = [False] * n_slots
        self.guessed = [False] * n_slots
        self.last_use = [0] * n_slots
        self.where = [-1] * self.n_places
        self.uses = [0] * self.n_places
        self.clock = 0
        self.acquired = 0
        self.present = 0  # hits + in flight
        self.misses = 0
        self.prefetched = 0
        self.prefetch_used = 0
        self.copies = 0
        self.bytes_copied = 0

    def free_slot(self):
        best = -1
        for i in range(self.n_slots):
            if self.held[i]:
                continue
            if self.place[i] < 0:
                return i
            if best < 0:
                best = i
                continue
            ux, ub = self.uses[self.place[i]], self.uses[self.place[best]]
            if ux < ub or (ux == ub and self.last_use[i] < self.last_use[best]):
                best = i
        return best

    def fill(self, s, place, guessed):
        if self.place[s] >= 0:
            self.where[self.place[s]] = -1
        self.place[s] = place
        self.where[place] = s
        self.held[s] = True
        self.guessed[s] = guessed
        self.clock += 1
        self.last_use[s] = self.clock
        self.copies += 1
        self.bytes_copied += self.expert_bytes[place // self.E]

    def experts(self, layer, ids, guess=None):
        """One vitna_cuda_moe_experts call; returns the slot of each requested expert."""
        k = len(ids)
        slot_of = [-1] * k
        missing = []
        for i, e in enumerate(ids):
            place = layer * self.E + int(e)
            self.uses[place] += 1
            self.acquired += 1
            if self.acquired % 65536 == 0:
                self.uses = [u // 2 for u in self.uses]
            s = self.where[place]
            slot_of[i] = s
            if s < 0:
                missing.append(i)
                self.misses += 1
                continue
            self.held[s] = True
            self.clock += 1
            self.last_use[s] = self.clock
            self.present += 1
            if self.guessed[s]:
                self.prefetch_used += 1
                self.guessed[s] = False
        for i in missing:
            s = self.free_slot()
            assert s >= 0, "no slot free: the cache must hold twice the experts a token goes through"
            self.fill(s, layer * self.E + int(ids[i]), False)
            slot_of[i] = s
        if guess is not None and (layer + 1) * self.E < self.n_places:
            for j in range((k + 1) // 2):
                place = (layer + 1) * self.E + int(guess[j])
                if self.where[place] >= 0:
                    continue
                s = self.free_slot()
                if s < 0:
                    break
                self.fill(s, place, True)
                self.prefetched += 1
        self.held = [False] * self.n_slots
        return slot_of

    def rows_experts(self, layer, ids, guess=None):
        """One vitna_cuda_moe_rows_experts call over n rows (ids, guess: n lists of k); returns {expert: slot}."""
        k = len(ids[0])
        cnt = {}
        for row in ids:
            for e in row:
                cnt[int(e)] = cnt.get(int(e), 0) + 1
        want = sorted(cnt)
        for x in want:
            self.uses[layer * self.E + x] += cnt[x]
            before = self.acquired
            self.acquired += cnt[x]
            if before // 65536 != self.acquired // 65536:
                self.uses = [u // 2 for u in self.uses]
        slot_of = {}
        W = self.n_slots - k
        for w0 in range(0, len(want), W):
            self.held = [False] * self.n_slots
            batch = []
            wave = want[w0:w0 + W]
            for i in range(len(wave) + 1):
                if i < len(wave):
                    x = wave[i]
                    s = self.where[layer * self.E + x]
                    if s >= 0:
                        self.held[s] = True
                        self.clock += 1
                        self.last_use[s] = self.clock
                        self.present += cnt[x]
                        if self.guessed[s]:
                            self.prefetch_used += 1
                            self.guessed[s] = False
                        slot_of[x] = s
                        continue
                    self.misses += 1
                    self.present += cnt[x] - 1
                    batch.append(x)
                    if len(batch) < k:
                        continue
                for x in batch:
                    s = self.free_slot()
                    assert s >= 0
                    self.fill(s, layer * self.E + x, False)
                    slot_of[x] = s
                batch = []
        if guess is not None and (layer + 1) * self.E < self.n_places:
            mark = set()
            room = True
            for row in guess:
                if not room:
                    break
                for j in range((k + 1) // 2):
                    x = int(row[j])
                    if x in mark:
                        continue
                    mark.add(x)
                    place = (layer + 1) * self.E + x
                    if self.where[place] >= 0:
                        continue
                    s = self.free_slot()
                    if s < 0:
                        room = False
                        break
                    self.fill(s, place, True)
                    self.prefetched += 1
        self.held = [False] * self.n_slots
        return slot_of

    def counters(self):
        return dict(acquired=self.acquired, present=self.present, misses=self.misses, prefetched=self.prefetched,
                    prefetch_used=self.prefetch_used, copies=self.copies, bytes_copied=self.bytes_copied)
