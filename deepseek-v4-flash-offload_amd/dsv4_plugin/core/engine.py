"""Expert offload engine: checkpoint-key capture and (layer, expert) lookups.

Surface of ``dsv4_plugin/core/engine.py`` in the reference (``:23-116``):
``parse_expert_name``, ``is_expert_weight``, ``ExpertOffloadEngine`` with
``capture`` / ``get`` / ``get_packed`` / ``stats`` and the process-wide
``get_engine`` singleton (``DSV4_EXPERT_SLOTS``, default 512). Captured experts
go into an ``offload.ExpertBank`` whose packed slots feed the HIP grouped GEMMs;
``acquire_table`` is the batched fast path the MoE layer uses. The shared
expert's FP8 tensors are copied on the side (``capture_shared``) so the layer
can run it inside the routed launches (``get_shared``).
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
# The shared expert of layer L in the checkpoint's FP8 form:
# [model.]layers.<L>.ffn.shared_experts.w{1,2,3}.{weight,scale}
_SHARED_KEY = re.compile(r"(?:^|\.)layers\.(?P<idx>\d+)\.ffn\.shared_experts\.(?P<w>w[123])"
                         r"\.(?P<kind>weight|scale)$")


def parse_expert_name(name: str):
    """``(layer, eid, "w1"|"w2"|"w3", "weight"|"scale")`` or None; MTP block k -> layer -1-k."""
    m = _KEY.search(name)
    if m is None:
        return None
    idx = int(m.group("idx"))
    layer = idx if m.group("blk") == "layers" else -1 - idx
    return layer, int(m.group("eid")), m.group("w"), m.group("kind")


def parse_shared_name(name: str):
    """``(layer, "w1"|"w2"|"w3", "weight"|"scale")`` of a shared-expert key, or None."""
    m = _SHARED_KEY.search(name)
    if m is None:
        return None
    return int(m.group("idx")), m.group("w"), m.group("kind")


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
        self._shared = {}    # layer -> {"w1": codes, "w1s": block scales, ...} (host copies)
        self._shared_dev = {}

    def capture_shared(self, name: str, tensor: torch.Tensor) -> bool:
        """Keep a host copy of a shared-expert FP8 tensor (the weight stream still
        delivers it to its own module); True if ``name`` is one."""
        parsed = parse_shared_name(name)
        if parsed is None:
            return False
        layer, w, kind = parsed
        self._shared.setdefault(layer, {})[w + ("s" if kind == "scale" else "")] = tensor.detach().to("cpu")
        # a re-captured tensor (weight reload) invalidates the layer's prepared copy on every device
        for key in [k for k in self._shared_dev if k[0] == layer]:
            del self._shared_dev[key]
        return True

    def get_shared(self, layer: int, device):
        """The shared expert of ``layer`` prepared for the fused layer launch
        (``dsv4_hip.ops.prepare_shared_expert``), or None until all six tensors
        were captured."""
        parts = self._shared.get(int(layer))
        if parts is None or len(parts) < 6:
            return None
        key = (int(layer), str(device))
        prep = self._shared_dev.get(key)
        if prep is None:
            from dsv4_hip import ops
            d = {k: v.to(device) for k, v in parts.items()}
            prep = ops.prepare_shared_expert(d["w1"], d["w1s"], d["w3"], d["w3s"], d["w2"], d["w2s"])
            self._shared_dev[key] = prep
        return prep

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

    def resident_table(self, layer: int, n_experts: int):
        """Pointer table of every expert of ``layer`` while all registered experts fit
        the slot cache (None otherwise); see ``ExpertBank.resident_table``."""
        return self.bank.resident_table(layer, n_experts)

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
