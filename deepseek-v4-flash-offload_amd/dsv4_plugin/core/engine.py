"""Expert offload engine: checkpoint-key capture and (layer, expert) lookups.

Surface of ``dsv4_plugin/core/engine.py`` in the reference (``:23-116``):
``parse_expert_name``, ``is_expert_weight``, ``ExpertOffloadEngine`` with
``capture`` / ``get`` / ``get_packed`` / ``stats`` and the process-wide
``get_engine`` singleton (``DSV4_EXPERT_SLOTS``, default 512). Captured experts
go into an ``offload.ExpertBank`` whose packed slots feed the HIP grouped GEMMs;
``acquire_table`` is the batched fast path the MoE layer uses.
"""

import os
import re
import sys

import torch

_PKG = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from offload import ExpertBank  # noqa: E402

# Checkpoint keys of routed experts: [model.]layers.<L>.ffn.experts.<E>.w{1,2,3}.{weight,scale}
# and the speculative-decoding block [model.]mtp.<K>.ffn.experts.<E>.w{1,2,3}.{weight,scale}.
_KEY = re.compile(r"(?:^|\.)(?P<blk>layers|mtp)\.(?P<idx>\d+)\.ffn\.experts\.(?P<eid>\d+)"
                  r"\.(?P<w>w[123])\.(?P<kind>weight|scale)$")
_PART = {"weight": "p", "scale": "s"}
_PARTS = ("w1p", "w1s", "w2p", "w2s", "w3p", "w3s")


def parse_expert_name(name: str):
    """``(layer, eid, "w1"|"w2"|"w3", "weight"|"scale")`` or None; MTP block k -> layer -1-k."""
    m = _KEY.search(name)
    if m is None:
        return None
    idx = int(m.group("idx"))
    layer = idx if m.group("blk") == "layers" else -1 - idx
    return layer, int(m.group("eid")), m.group("w"), m.group("kind")


def is_expert_weight(name: str, include_mtp: bool = False) -> bool:
    """Main-model routed-expert key (``mtp.*`` only with ``include_mtp``)."""
    m = _KEY.search(name)
    return m is not None and (include_mtp or m.group("blk") == "layers")


class ExpertOffloadEngine:
    """Host packed-expert pool + device slot caches, addressed by (layer, eid)."""

    def __init__(self, slot_capacity: int, device="cuda:0", dtype=torch.bfloat16):
        self.bank = ExpertBank(capacity=slot_capacity, device=device, dtype=dtype)
        self._pending = {}   # (layer, eid) -> {part: tensor} until all six parts arrive
        self.captured = 0

    def capture(self, name: str, tensor: torch.Tensor) -> bool:
        """Take an expert tensor from the weight stream; True if consumed."""
        parsed = parse_expert_name(name)
        if parsed is None:
            return False
        layer, eid, w, kind = parsed
        parts = self._pending.setdefault((layer, eid), {})
        parts[w + _PART[kind]] = tensor.detach().to("cpu")
        if len(parts) == len(_PARTS):
            self.bank.register(layer, eid, *(parts[k] for k in _PARTS))
            del self._pending[(layer, eid)]
            self.captured += 1
        return True

    def get(self, layer: int, eid: int):
        """bf16 ``{"w1","w2","w3"}`` on the device (H2D + dequant on a miss)."""
        return self.bank.get(layer, eid)

    def get_packed(self, layer: int, eid: int):
        """Packed ``w{1,2,3}p`` ``[N, K/2]`` + ``w{1,2,3}s`` ``[N, K/32]`` device views."""
        return self.bank.get_packed(layer, eid)

    def acquire_table(self, layer: int, expert_ids, n_experts: int):
        return self.bank.acquire_table(layer, expert_ids, n_experts)

    def prefetch(self, layer: int, expert_ids):
        return self.bank.prefetch(layer, expert_ids)

    def stats(self):
        s = self.bank.stats()
        s["captured"] = self.captured
        s["parked"] = len(self._pending)
        return s

    def __repr__(self):
        return f"ExpertOffloadEngine({self.bank!r}, captured={self.captured})"


_ENGINE = None


def get_engine(slot_capacity=None, device="cuda:0") -> ExpertOffloadEngine:
    """The process-wide engine, created on first use (``slot_capacity`` only then)."""
    global _ENGINE
    if _ENGINE is None:
        if slot_capacity is None:
            slot_capacity = int(os.environ.get("DSV4_EXPERT_SLOTS", "512"))
        _ENGINE = ExpertOffloadEngine(slot_capacity=slot_capacity, device=device)
    return _ENGINE
