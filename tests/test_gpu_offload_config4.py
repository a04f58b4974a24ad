"""GPU: the expert-offload workload at its full size.

8 layers x 256 experts registered in the pinned host pool at the real record
size (hidden 4096, inter 2048: 13,369,344 bytes of packed MXFP4 per expert,
27.4 GB in all), 512 device slots (6.8 GB), 512 decode steps of 8 tokens with
top-8 Zipf(1.1) routing per layer whose hot set drifts (every 8 steps, 4
adjacent-rank swaps among ranks 0..127 per layer). Each (step, layer) acquires
its routed experts through ``SlotCache.acquire``, the batched form of
``ExpertBank.get_packed`` (offload.py:103-129).

Checked:
* hit / miss / eviction counts equal a textbook LRU replay of the same
  acquisitions (``oracle.lru.LRUOracle``, the policy ``test_offload.py:67-86``
  pins), step by step;
* every acquired slot holds exactly its expert's record when the compute
  stream reads it (all 13.4 MB, compared on the device). Records are
  distinct per (layer, expert): each carries its key in its first w1 scale
  bytes, on top of one of eight random base records.
Mismatches are counted on the device and checked every 32 steps, so the test
stops soon after the first one.
"""

import numpy as np
import pytest
import torch

from dsv4_hip import synth
from dsv4_hip.slots import FIELDS, SlotCache, SlotLayout
from oracle.lru import LRUOracle

pytestmark = pytest.mark.gpu

L, E, K, T, N_SLOTS, STEPS = 8, 256, 8, 8, 512, 512
D, I = 4096, 2048


def _tagged(base, layer, eid):
    t = dict(base)
    w1s = base["w1s"].clone()
    w1s.view(-1)[:8] = torch.tensor([layer, eid], dtype=torch.int32).view(torch.uint8)
    t["w1s"] = w1s
    return t


@pytest.mark.timeout(600)
def test_offload_config4_full_size_matches_lru_replay(gpu):
    bases = [{k: torch.from_numpy(v) for k, v in synth.expert_weights(e, D, I).items()} for e in range(8)]
    layout = SlotLayout(bases[0])
    assert layout.record_bytes >= 13_369_344 and layout.tiled
    cache = SlotCache(gpu, N_SLOTS, layout, pin=True)
    pinned = True
    for l in range(L):
        for e in range(E):
            pinned &= cache.register(l, e, _tagged(bases[(l * 7 + e) % 8], l, e))
    print(f"registered {L * E} records of {layout.record_bytes} B, pinned={pinned}", flush=True)
    # the eight base records as the slots hold them (tiled packed fields), on the device
    rb = layout.record_bytes
    tmp = SlotCache(gpu, 1, layout, pin=False)
    base_dev = torch.empty((8, rb), dtype=torch.uint8, device=gpu)
    for b in range(8):
        tmp.register(0, b, bases[b])
        tmp.copy_record(0, b, base_dev[b])
    torch.cuda.synchronize()
    tmp.close()
    tag_off = layout.offsets["w1s"]
    pool2d = cache.pool.view(N_SLOTS, rb)
    route = synth.DriftingZipf(L, E, K)
    ora = LRUOracle(N_SLOTS)
    bad = torch.zeros((), dtype=torch.int64, device=gpu)
    n_miss_total = 0
    for s in range(STEPS):
        ids = route.step(T)
        for l in range(L):
            u = np.unique(ids[l]).astype(np.int32)
            slots, nm = cache.acquire(l, u)
            exp_miss = sum(0 if ora.access((l, int(e)))[0] else 1 for e in u)
            assert nm == exp_miss, (s, l, nm, exp_miss)
            n_miss_total += nm
            sl = torch.from_numpy(slots.astype(np.int64)).to(gpu, non_blocking=True)
            bidx = torch.from_numpy(((l * 7 + u) % 8).astype(np.int64)).to(gpu, non_blocking=True)
            want = base_dev.index_select(0, bidx)
            tags = np.stack([np.full(u.size, l, np.int32), u.astype(np.int32)], 1).view(np.uint8)
            want[:, tag_off:tag_off + 8] = torch.from_numpy(tags).to(gpu, non_blocking=True)
            bad += (pool2d.index_select(0, sl) != want).any(dim=1).sum()
        if (s + 1) % 32 == 0:
            nbad = int(bad.item())
            assert nbad == 0, f"{nbad} acquired slot(s) held the wrong bytes by step {s}"
            st = cache.stats()
            print(f"step {s + 1}: hits={st['hits']} misses={st['misses']} evictions={st['evictions']}", flush=True)
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
    st, so = cache.stats(), ora.stats()
    print(f"config 4: hit rate {so['hit_rate']:.4f}, misses {so['misses']}, evictions {so['evictions']}, "
          f"H2D {st['bytes_h2d'] / 1e9:.1f} GB", flush=True)
    assert (st["hits"], st["misses"], st["evictions"]) == (so["hits"], so["misses"], so["evictions"])
    assert st["misses"] == n_miss_total and st["bytes_h2d"] == st["misses"] * rb
    assert st["cached"] == N_SLOTS and so["evictions"] > 10_000
    assert 0.3 < so["hit_rate"] < 0.7
    cache.close()
    del cache, base_dev
    torch.cuda.empty_cache()
