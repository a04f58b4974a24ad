"""Restatement of ``ExpertBank``'s device LRU (``offload.py:86-129``) - test oracle only.

A textbook ``OrderedDict`` LRU: a hit moves the key to the MRU end; a miss
inserts it and, while over capacity, pops the LRU end (counting evictions);
capacity 0 never caches. ``access`` returns ``(hit, evicted_key_or_None)``.
"""

import collections


class LRUOracle:
    def __init__(self, capacity):
        self.capacity = int(capacity)
        self.cache = collections.OrderedDict()
        self.hits = 0
        self.misses = 0
        self.evictions = 0

    def access(self, key):
        if key in self.cache:
            self.hits += 1
            self.cache.move_to_end(key)
            return True, None
        self.misses += 1
        evicted = None
        if self.capacity > 0:
            self.cache[key] = True
            while len(self.cache) > self.capacity:
                evicted, _ = self.cache.popitem(last=False)
                self.evictions += 1
        return False, evicted

    def stats(self):
        tot = self.hits + self.misses
        return {"hits": self.hits, "misses": self.misses, "evictions": self.evictions,
                "hit_rate": (self.hits / tot) if tot else 0.0, "cached": len(self.cache)}
