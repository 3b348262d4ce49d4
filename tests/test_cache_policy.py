"""The expert slot cache (qmoe_xcache_*, host only) against a restatement of
the reference C port's cache policy (oracle/cache_ref.py, c/src/cache.c:
cache_get 187-204, cache_put 216-259, pick_victim 99-163, pin/unpin/
mark_hot 261-299): on random operation sequences per policy the hits,
misses, evicted items, resident sets and counters agree step by step.  The
restatement itself is pinned by hand-built cases whose victims follow from
the policy text (LRU oldest, LFU least frequent, ADAPTIVE (freq+4*hot)/
nbytes, cold before hot, pinned never, ties to the older entry)."""
import random

import pytest

from conftest import load_pkg
from oracle import cache_ref as cr

POLICIES = [cr.LRU, cr.LFU, cr.ADAPTIVE]


def test_reference_restatement_known_victims():
    # LRU: the least recently used goes
    c = cr.PartitionCache(3, cr.LRU, 100)
    for i in (1, 2, 3):
        c.put(i)
    c.get(1)
    assert c.put(4) == (True, 2)
    # LFU: the least frequent goes, ties to the older
    c = cr.PartitionCache(3, cr.LFU, 100)
    for i in (1, 2, 3):
        c.put(i)
    c.get(1), c.get(1), c.get(3)
    assert c.put(4) == (True, 2)
    c.get(4)
    assert c.put(5) == (True, 3)  # 3 (freq 2, older) vs 4 (freq 2, newer)
    # ADAPTIVE: cold before hot whatever the frequency; pinned never
    c = cr.PartitionCache(3, cr.ADAPTIVE, 100)
    for i in (1, 2, 3):
        c.put(i)
    for _ in range(5):
        c.get(2)
    c.mark_hot(1, True)
    c.mark_hot(3, True)
    assert c.put(4) == (True, 2)  # the only cold one, though the most used
    c.pin(4, True)
    c.mark_hot(1, False)
    assert c.put(5) == (True, 1)
    # everything pinned: rejected
    c = cr.PartitionCache(1, cr.LRU, 100)
    c.put(1, pin=True)
    assert c.put(2) == (False, None) and c.rejected == 1


def test_reference_quirk_cold_reset():
    """after a cold entry replaces a hot best, the best score is 0, so later
    cold entries (ADAPTIVE scores > 0) cannot replace it: the first cold
    entry met after a hot one wins even if a later cold one scores lower"""
    c = cr.PartitionCache(3, cr.ADAPTIVE, 1)
    c.put(1, hot=True)  # oldest, hot
    c.put(2)            # cold, will get freq 3
    c.get(2), c.get(2)
    c.put(3)            # cold, freq 1 (lower score than 2)
    assert c.put(4) == (True, 2)


@pytest.mark.parametrize("policy", POLICIES)
def test_library_matches_reference(policy):
    pkg = load_pkg()
    rng = random.Random(policy * 7919 + 1)
    parts, items, slots, nbytes = 3, 24, 5, 1769472
    lib_c = pkg.ExpertCache(parts, items, slots, policy, nbytes)
    refs = [cr.PartitionCache(slots, policy, nbytes) for _ in range(parts)]
    for step in range(4000):
        p = rng.randrange(parts)
        it = rng.randrange(items) if rng.random() < 0.5 else rng.randrange(8)  # skewed
        op = rng.random()
        ref = refs[p]
        if op < 0.55:
            hit = lib_c.get(p, it) >= 0
            assert hit == ref.get(it), (step, "get", p, it)
            if not hit:
                pin = rng.random() < 0.1
                hot = rng.random() < 0.2
                slot, ev = lib_c.put(p, it, pin, hot)
                ok, rev = ref.put(it, pin, hot)
                assert (slot >= 0) == ok, (step, "put", p, it)
                assert ev == (-1 if rev is None else rev), (step, "evicted", ev, rev)
        elif op < 0.75:
            pinned = rng.random() < 0.5
            assert bool(lib_c.pin(p, it, pinned)) == ref.pin(it, pinned), (step, "pin")
        elif op < 0.9:
            hot = rng.random() < 0.5
            assert bool(lib_c.mark_hot(p, it, hot)) == ref.mark_hot(it, hot), (step, "hot")
        else:
            for j in range(items):
                assert (lib_c.peek(p, j) >= 0) == (j in ref.resident()), (step, "peek", j)
    got = lib_c.counts()
    want = dict(hits=sum(r.hits for r in refs), misses=sum(r.misses for r in refs),
                evictions=sum(r.evictions for r in refs), rejected=sum(r.rejected for r in refs))
    assert got == want
    lib_c.close()


def test_slots_stay_within_the_partition_and_are_reused():
    pkg = load_pkg()
    c = pkg.ExpertCache(2, 10, 3, cr.LRU, 64)
    slots = {c.put(0, i)[0] for i in range(3)}
    assert slots == {0, 1, 2}
    slot, ev = c.put(0, 7)
    assert ev == 0 and slot == c.peek(0, 7) and c.peek(0, 0) == -1
    assert c.put(1, 0)[0] == 0  # the other partition has its own slots
    c.clear(0)
    assert all(c.peek(0, i) == -1 for i in range(10)) and c.peek(1, 0) == 0
    with pytest.raises(pkg.QmoeError):
        pkg.ExpertCache(1, 4, 5, cr.LRU, 64)  # more slots than items


def _closed_form_victim(entries, policy):
    """the victim rule the device-resolved residency kernel evaluates with
    block-wide minima instead of a recency walk: no unpinned cold entry ->
    min (score, touched) over the hot; the oldest unpinned entry cold ->
    min (score, touched) over the cold; else the oldest cold entry.  Score
    0 (LRU), freq (LFU), freq + 4*hot (ADAPTIVE, one entry size)."""
    un = [e for e in entries if not e.pinned]
    if not un:
        return None
    oldest = min(un, key=lambda e: e.touched)
    cold = [e for e in un if not e.hot]
    if cold and oldest.hot:
        return min(cold, key=lambda e: e.touched)
    cand = cold if cold else un

    def score(e):
        return 0 if policy == cr.LRU else e.freq + (4 if policy == cr.ADAPTIVE and e.hot else 0)
    return min(cand, key=lambda e: (score(e), e.touched))


@pytest.mark.parametrize("policy", [cr.LRU, cr.LFU, cr.ADAPTIVE])
def test_closed_form_victim_equals_recency_walk(policy):
    """the closed form against pick_victim's walk (cache.c:99-163, restated
    in the oracle) on random states: frequencies with many ties, hot and
    pinned marks at random, distinct touch times"""
    rng = random.Random(1234 + policy)
    for trial in range(3000):
        slots = rng.randint(1, 12)
        c = cr.PartitionCache(slots, policy, 1769472)
        touched = rng.sample(range(1, 10 * slots + 1), slots)
        entries = []
        for s, t in enumerate(touched):
            e = cr.Entry(s, rng.random() < 0.3, rng.random() < 0.5, t)
            e.freq = rng.randint(1, 6)
            entries.append(e)
        c.recency = sorted(entries, key=lambda e: -e.touched)  # most recent first
        want = c.pick_victim()
        got = _closed_form_victim(entries, policy)
        assert (want is None) == (got is None), trial
        if want is not None:
            assert got.item == want.item, (trial, slots)
