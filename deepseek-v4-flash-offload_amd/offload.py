"""Host-resident packed experts + device caches, MI355X edition of ``offload.ExpertBank``.

Same constructor, methods and ``stats()`` keys as the reference
(``offload.py:22-151``):

* ``register`` stores the six packed tensors of an expert in a pinned host
  record of the native slot cache (one contiguous record per expert; on a CPU
  device, or when pinning fails, it degrades exactly like the reference:
  one message, then pageable memory);
* ``get`` keeps the reference's bf16 LRU of dequantised experts
  (``capacity`` entries); a miss copies the packed record to the device and
  dequantises it with the HIP kernel (bit-exact with ``dequant_fp4_weight``);
* ``get_packed`` makes the expert resident in the native LRU slot cache
  (``packed_capacity`` slots, default 4 x ``capacity`` as in the reference)
  and returns device copies of its six tensors, which the caller owns;
* ``acquire_table`` is the batched fast path used by the MoE layer: one call
  per (layer, step) makes all routed experts resident and returns the device
  pointer table of the grouped GEMMs. Misses are copied on a side stream and
  counted once per routed expert (the reference counts ``get`` three times
  per expert).

There is no CPU compute path: ``get``/``get_packed`` on a CPU bank raise.
"""

import collections
import os

import numpy as np
import torch

from dsv4_hip import ops
from dsv4_hip.slots import FIELDS, SlotCache, SlotLayout


def _device(device):
    d = str(device)
    if d.startswith("npu"):
        d = "cuda" + d[3:]
    return torch.device(d)


class ExpertBank:
    """Host-resident packed expert weights + device LRU caches.

    Parameters follow ``offload.ExpertBank``: ``capacity`` bf16 experts kept
    dequantised on the device; ``packed_capacity`` (env ``DSV4_PACKED_SLOTS``,
    default ``4 * capacity``) packed slots; ``pin`` (env ``DSV4_PIN_HOST``,
    default on) page-locks the host records."""

    def __init__(self, capacity: int, device, dtype=torch.bfloat16, verbose=False, pin=None):
        self.capacity = int(capacity)
        self.device = _device(device)
        self.dtype = dtype
        self.verbose = verbose
        if pin is None:
            pin = os.environ.get("DSV4_PIN_HOST", "1") == "1"
        self.pin = pin
        self._host = {}            # CPU banks only: (layer, eid) -> six CPU tensors
        self._cache = collections.OrderedDict()
        self.hits = 0
        self.misses = 0
        self.evictions = 0
        self.packed_capacity = int(os.environ.get("DSV4_PACKED_SLOTS", str(4 * self.capacity)))
        self._slots = None
        self._layout = None
        self._resident = {}        # layer -> (registered count, full pointer table)

    # -- host bank --------------------------------------------------------
    def _ensure_slots(self, tensors):
        if self._slots is None:
            self._layout = SlotLayout(tensors)
            self._slots = SlotCache(self.device, max(1, self.packed_capacity), self._layout, pin=self.pin)

    def register(self, layer, eid, w1p, w1s, w2p, w2s, w3p, w3s):
        """Store the raw packed expert weights (CPU tensors, as loaded)."""
        tup = (w1p, w1s, w2p, w2s, w3p, w3s)
        key = (int(layer), int(eid))
        if self.device.type != "cuda":
            if self.pin:
                try:
                    tup = tuple(x if x.is_pinned() else x.pin_memory() for x in tup)
                except RuntimeError as exc:  # no page-locked memory: degrade once
                    print(f"[ExpertBank] pin_memory failed, using pageable memory: {exc}", flush=True)
                    self.pin = False
            self._host[key] = tup
            return
        tensors = dict(zip(FIELDS, tup))
        self._ensure_slots(tensors)
        pinned = self._slots.register(layer, eid, tensors)
        if self.pin and not pinned:
            print("[ExpertBank] page-locked host allocation failed, using pageable memory", flush=True)
            self.pin = False

    def has(self, layer, eid):
        key = (int(layer), int(eid))
        return key in self._host or (self._slots is not None and self._slots.has(*key))

    def num_experts(self):
        return len(self._host) + (len(self._slots.keys_registered) if self._slots is not None else 0)

    def _need_gpu(self, what):
        if self.device.type != "cuda" or self._slots is None:
            raise RuntimeError(f"ExpertBank.{what} needs a ROCm device bank with registered experts "
                               f"(device={self.device}); there is no CPU path")

    # -- device bf16 cache (reference get) ----------------------------------
    def _dequant_on_device(self, layer, eid):
        """One record copy and ONE dequant launch for the expert's three tensors (the
        reference dequantises them one call each, ``offload.py:77-84``)."""
        buf = torch.empty(self._layout.record_bytes, dtype=torch.uint8, device=self.device)
        self._slots.copy_record(layer, eid, buf)
        v = self._slots.record_bytes_views(buf)   # packed fields as stored (tiled or not)
        names = ("w1", "w2", "w3")
        ts = ops.dequant_mxfp4_multi([(v[w + "p"], v[w + "s"]) for w in names], tiled=self._layout.tiled)
        return {w: (t if self.dtype == torch.bfloat16 else t.to(self.dtype)) for w, t in zip(names, ts)}

    def get(self, layer, eid):
        self._need_gpu("get")
        key = (int(layer), int(eid))
        cached = self._cache.get(key)
        if cached is not None:
            self.hits += 1
            self._cache.move_to_end(key)
            return cached
        self.misses += 1
        if not self._slots.has(*key):
            raise KeyError(f"expert {key} is not registered")
        vals = self._dequant_on_device(*key)
        if self.capacity > 0:
            self._cache[key] = vals
            while len(self._cache) > self.capacity:
                self._cache.popitem(last=False)
                self.evictions += 1
        return vals

    # -- device packed slot cache -------------------------------------------
    def get_packed(self, layer, eid):
        """Packed device tensors ``{"w{1,2,3}p": [N, K/2], "w{1,2,3}s": [N, K/32]}``,
        owned by the caller like the reference's (``offload.py:122-124``): copies
        of the slot, so a later acquire that reuses the slot cannot change them."""
        self._need_gpu("get_packed")
        slots, _ = self._slots.acquire(int(layer), [int(eid)])
        return self._slots.slot_copy(int(slots[0]))

    def acquire_table(self, layer, expert_ids, n_experts):
        """Make every expert in ``expert_ids`` resident; returns (device pointer table [E, 6], n_miss)."""
        self._need_gpu("acquire_table")
        eids = np.unique(np.asarray(expert_ids, dtype=np.int64)).astype(np.int32)
        slots, n_miss = self._slots.acquire(int(layer), eids)
        return self._slots.table(eids, slots, n_experts), n_miss

    def resident_table(self, layer, n_experts):
        """Device pointer table [E, 6] of every registered expert of ``layer``, or
        None. Only when the packed slot cache can hold every registered expert of
        every layer at once: then no acquire can evict one, the table stays valid,
        and the routed ids never need to reach the host. The first call per layer
        copies its missing experts in; the table is rebuilt when more experts are
        registered. (Lookups through this table are not counted as hits.)"""
        if self.device.type != "cuda" or self._slots is None:
            return None
        n_reg = len(self._slots.keys_registered)
        if self.packed_capacity < n_reg:
            return None
        layer = int(layer)
        hit = self._resident.get(layer)
        if hit is not None and hit[0] == n_reg:
            return hit[1]
        eids = np.array(sorted(e for (lay, e) in self._slots.keys_registered if lay == layer and 0 <= e < n_experts),
                        dtype=np.int32)
        if eids.size == 0:
            return None
        slots, _ = self._slots.acquire(layer, eids)
        tab = self._slots.table(eids, slots, n_experts)
        self._resident[layer] = (n_reg, tab)
        return tab

    def prefetch(self, layer, expert_ids):
        """Start side-stream copies of the non-resident experts of a coming layer."""
        self._need_gpu("prefetch")
        return self._slots.prefetch(int(layer), np.unique(np.asarray(expert_ids, dtype=np.int64)))

    def invalidate(self):
        self._cache.clear()
        self._resident.clear()
        if self._slots is not None:
            self._slots.invalidate()

    def stats(self):
        tot = self.hits + self.misses
        rate = (self.hits / tot) if tot else 0.0
        ps = self._slots.stats() if self._slots is not None else {
            "hits": 0, "misses": 0, "evictions": 0, "prefetched": 0, "bytes_h2d": 0, "cached": 0}
        ptot = ps["hits"] + ps["misses"]
        return {"hits": self.hits, "misses": self.misses,
                "evictions": self.evictions, "hit_rate": rate,
                "cached": len(self._cache), "capacity": self.capacity,
                "packed_hits": ps["hits"], "packed_misses": ps["misses"],
                "packed_hit_rate": (ps["hits"] / ptot) if ptot else 0.0,
                "packed_cached": ps["cached"], "packed_capacity": self.packed_capacity,
                "pinned": self.pin,
                "packed_evictions": ps["evictions"], "prefetched": ps["prefetched"],
                "h2d_bytes": ps["bytes_h2d"]}

    def __repr__(self):
        s = self.stats()
        return (f"ExpertBank(experts={self.num_experts()}, cached={s['cached']}/"
                f"{s['capacity']}, hit_rate={s['hit_rate']:.3f})")
