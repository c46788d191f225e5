"""A host model of the persistent launch's stamped spike ring (atlas_tick.h persistent_run):
the stamp of a tick, the words a publication writes and clears, and what a reader past the
tick's barrier can observe.  The model replays publication schedules, including bursts exactly
lcm(R, 4095) ticks apart, and checks that no word a reader may see validates for a tick unless
that tick wrote it.  The ring depths are the engine's own for delay-0 and delay-1 plans.

The reader model: a reader of tick e has passed the barrier of e, so every producer has issued
its stores of tick e, and it arrived at barrier e - R + 1 <= e only after waiting for its stores
of tick e - R to complete (the vmcnt(0) wait before each publication).  Each word then holds
either the value the publication of e - R left or the value e writes, and the reader may see
either of them, independently per word (the stores of e are issued, not completed)."""
import re
from pathlib import Path

import numpy as np
import pytest

from atlas_hip import engine, models, native

HEADER = Path(__file__).resolve().parents[1] / "brian2-atlas_amd" / "csrc" / "device" / "atlas_tick.h"
REC_IDS = 7          # ids a ring record carries after its count word
VALUE_BITS = 20


def stamp(tick: int) -> int:
    """ring_stamp: ((tick + 1) mod 4095) + 1, never 0."""
    return (tick + 1) % 4095 + 1


def word(st: int, value: int) -> int:
    return st << VALUE_BITS | value


class Ring:
    """One block's words in every slot of a ring of R ticks: the record (count, first 7 ids) and
    the id list, as the publications of `rule` leave them.  rule "clear" is the kernel's (the
    words past the count that the slot's previous tick wrote are cleared); "keep" leaves them."""

    def __init__(self, depth: int, width: int, rule: str):
        self.R = depth
        self.rule = rule
        self.ids = np.zeros((depth, width), np.int64)
        self.rec = np.zeros((depth, 1 + REC_IDS), np.int64)
        self.prev = np.zeros(depth, np.int64)   # the block's count in each slot (the kernel's ring_prev)

    def publish(self, tick: int, fired: list[int]) -> tuple[np.ndarray, np.ndarray]:
        """Stores of tick `tick`; returns the slot's words as they were before them."""
        slot = tick % self.R
        before = (self.ids[slot].copy(), self.rec[slot].copy())
        st = stamp(tick)
        for k, neuron in enumerate(fired):
            self.ids[slot, k] = word(st, neuron)
            if k < REC_IDS:
                self.rec[slot, 1 + k] = word(st, neuron)
        if self.rule == "clear":
            for i in range(len(fired), int(self.prev[slot])):
                self.ids[slot, i] = 0
                if i < REC_IDS:
                    self.rec[slot, 1 + i] = 0
        self.rec[slot, 0] = word(st, len(fired))
        self.prev[slot] = len(fired)
        return before


def stale_validations(rule: str, depth: int, counts: list[int], width: int = 64) -> list[tuple[int, int]]:
    """Replays one block's publications (tick t fires counts[t] neurons, ids drawn per tick) and
    returns every (tick, word index) where a word the reader may see carries the tick's stamp
    but is not the word that tick wrote."""
    ring = Ring(depth, width, rule)
    rng = np.random.default_rng(len(counts) * 31 + depth)
    bad = []
    for tick, c in enumerate(counts):
        fired = sorted(rng.integers(0, 1 << VALUE_BITS, c).tolist())
        old_ids, old_rec = ring.publish(tick, fired)
        slot = tick % depth
        new_ids, new_rec = ring.ids[slot], ring.rec[slot]
        st = stamp(tick)
        # the reader validates the count word, then the id words below the count, in the record
        # and in the list; either version of each word may be the one it sees
        for k in range(min(c, REC_IDS)):
            for seen in (old_rec[1 + k], new_rec[1 + k]):
                if seen >> VALUE_BITS == st and seen != new_rec[1 + k]:
                    bad.append((tick, k))
        for i in range(c):
            for seen in (old_ids[i], new_ids[i]):
                if seen >> VALUE_BITS == st and seen != new_ids[i]:
                    bad.append((tick, i))
        if old_rec[0] >> VALUE_BITS == st:
            bad.append((tick, -1))
    return bad


def bursts(period: int, ticks: int, size: int, seed: int) -> list[int]:
    """Counts of 0-2 per tick, with a burst of `size` at tick 5 and every `period` ticks after."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, 3, ticks).tolist()
    for t in range(5, ticks, period):
        counts[t] = size
    return counts


def ring_depth(delay: int) -> int:
    doc = models.cuba_network(4000, steps=20) if delay == 0 else \
        models.cuba_network(4000, indegree=80, delay_ticks=delay, steps=20)
    plan = engine.lower(doc)
    engine.allocate(plan)
    engine.generate(plan, native.device_header_text())
    assert plan.persistent is not None, "the plan runs persistent"
    return plan.populations[0].ring


def test_stamp_rule_is_the_kernels():
    text = HEADER.read_text()
    assert re.search(r"ring_stamp\(i64 tick\) \{ return \(u32\)\(\(u64\)\(tick \+ 1\) % 4095u\) \+ 1u; \}", text)
    assert "ring_store_u32(&ids[i], 0u)" in text and "s.ring_prev[slot] = before" in text
    assert f"#define ATLAS_REC_IDS {REC_IDS}u" in text


@pytest.mark.parametrize("delay,expected_depth", [(0, 3), (1, 4)])
def test_engine_ring_depths(delay, expected_depth):
    assert ring_depth(delay) == expected_depth


@pytest.mark.parametrize("delay", [0, 1])
def test_kept_words_alias_after_lcm_ticks(delay):
    """The rule without clearing: a burst's id words past the later counts stay in their slot, and
    lcm(R, 4095) ticks later (4095 for the delay-0 ring of 3, 16,380 for delay 1's ring of 4) they
    carry the stamp the reader of the next burst waits for."""
    depth = ring_depth(delay)
    period = int(np.lcm(depth, 4095))
    assert period == {0: 4095, 1: 16380}[delay]
    counts = bursts(period, 2 * period + 10, 40, seed=delay)
    bad = stale_validations("keep", depth, counts)
    assert bad and {t for t, _ in bad} <= {5 + period, 5 + 2 * period}


@pytest.mark.parametrize("delay", [0, 1])
@pytest.mark.parametrize("size", [8, 40, 64])
def test_cleared_words_never_validate_stale(delay, size):
    depth = ring_depth(delay)
    period = int(np.lcm(depth, 4095))
    counts = bursts(period, 2 * period + 10, size, seed=size)
    assert stale_validations("clear", depth, counts) == []


@pytest.mark.parametrize("depth", [2, 3, 4, 5, 6, 8, 42])
def test_cleared_words_never_validate_stale_random_schedules(depth):
    """Random counts with bursts at random ticks and at every multiple of lcm(R, 4095)."""
    rng = np.random.default_rng(depth)
    ticks = 3 * int(np.lcm(depth, 4095)) if depth <= 6 else 30_000
    counts = np.minimum(rng.poisson(1.5, ticks), 64)
    counts[rng.integers(0, ticks, 200)] = rng.integers(8, 65, 200)
    counts[5::int(np.lcm(depth, 4095))] = 64
    assert stale_validations("clear", depth, counts.tolist()) == []
