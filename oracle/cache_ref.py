"""Pure-Python restatement of the reference C port's expert cache policy
(c/src/cache.c), as the checker of the library's slot cache -- TEST
INFRASTRUCTURE ONLY (imported by tests/).

Restated: cache_get (cache.c:187-204: a hit bumps freq, touched and
recency), cache_put (cache.c:216-259: insert with freq 1, evict by
pick_victim while full), pick_victim (cache.c:99-163: least recent first,
pinned skipped, cold before hot with the best score reset to 0, LRU oldest
/ LFU freq / ADAPTIVE (freq + 4*hot) / nbytes, ties to the older entry),
cache_pin/unpin and cache_mark_hot (cache.c:261-299).  Capacity is counted
in entries of one size per partition (a layer's slot pool), and "touched"
is a logical clock; the library states the same two departures.
"""
LRU, LFU, ADAPTIVE = 0, 1, 2


class Entry:
    __slots__ = ("item", "pinned", "hot", "freq", "touched")

    def __init__(self, item, pinned, hot, touched):
        self.item, self.pinned, self.hot, self.freq, self.touched = item, pinned, hot, 1, touched


class PartitionCache:
    def __init__(self, slots, policy, nbytes):
        self.slots, self.policy, self.nbytes = slots, policy, nbytes
        self.recency = []  # most recent first (cache.c head)
        self.by_item = {}
        self.clock = 0
        self.hits = self.misses = self.evictions = self.rejected = 0

    def _front(self, e):
        if e in self.recency:
            self.recency.remove(e)
        self.recency.insert(0, e)

    def get(self, item):
        e = self.by_item.get(item)
        if e is None:
            self.misses += 1
            return False
        e.freq += 1
        self.clock += 1
        e.touched = self.clock
        self._front(e)
        self.hits += 1
        return True

    def pick_victim(self):
        best, best_score, best_touched = None, 0.0, 0
        for e in reversed(self.recency):  # tail (least recent) to head
            if e.pinned:
                continue
            if best is not None and not e.hot and best.hot:
                best, best_score, best_touched = e, 0.0, e.touched
                continue
            if best is not None and e.hot and not best.hot:
                continue
            if self.policy == LRU:
                score = 0.0
            elif self.policy == LFU:
                score = float(e.freq)
            else:
                score = float(e.freq + (4 if e.hot else 0)) / float(self.nbytes)
            if best is None:
                better = True
            elif self.policy == LRU:
                better = e.touched < best_touched
            else:
                better = score < best_score or (score == best_score and e.touched < best_touched)
            if better:
                best, best_score, best_touched = e, score, e.touched
        return best

    def put(self, item, pin=False, hot=False):
        """returns (inserted, evicted item or None)"""
        old = self.by_item.get(item)
        if old is not None:
            pin, hot = pin or old.pinned, hot or old.hot
            self.recency.remove(old)
            del self.by_item[item]
        evicted = None
        if len(self.by_item) >= self.slots:
            v = self.pick_victim()
            if v is None:
                self.rejected += 1
                return False, None
            self.recency.remove(v)
            del self.by_item[v.item]
            self.evictions += 1
            evicted = v.item
        self.clock += 1
        e = Entry(item, pin, hot, self.clock)
        self.by_item[item] = e
        self.recency.insert(0, e)
        return True, evicted

    def pin(self, item, pinned):
        e = self.by_item.get(item)
        if e is None:
            return False
        changed = bool(e.pinned) != bool(pinned)
        e.pinned = bool(pinned)
        return changed

    def mark_hot(self, item, hot):
        e = self.by_item.get(item)
        if e is None:
            return False
        e.hot = bool(hot)
        return True

    def resident(self):
        return set(self.by_item)
