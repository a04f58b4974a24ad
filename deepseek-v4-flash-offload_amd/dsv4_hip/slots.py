"""Python handle of the native expert slot cache (csrc/slots.cpp).

A record is one expert's six packed tensors laid out back to back (256-byte
aligned fields), identical in the pinned host pool and in every device slot,
so a miss is a single host-to-device copy. The three packed weight fields are
stored in the MFMA-tiled layout the grouped GEMMs stream fastest (tiled once,
on the host, when the expert is registered; env DSV4_TILED_WEIGHTS=0 keeps the
checkpoint layout); the slot table tags them, and the views handed to callers
(get_packed, the bf16 dequant path) are untiled back to the checkpoint layout.
"""

import ctypes
import os

import numpy as np
import torch

from . import _lib
from ._lib import call, stream_handle

FIELDS = ("w1p", "w1s", "w2p", "w2s", "w3p", "w3s")
PACKED = ("w1p", "w2p", "w3p")


def tile_host(a):
    """Packed E2M1 bytes [N, K/2] in the MFMA-tiled layout (``dsv4_mxfp4_tile_weights``):
    ``tiled[nt][j][ji][g][r][e] = a[16 nt + r][128 j + 32 g + 16 ji + e]``."""
    N, KH = a.shape
    return np.ascontiguousarray(a.reshape(N // 16, 16, KH // 128, 4, 2, 16).transpose(0, 2, 4, 3, 1, 5)).reshape(N, KH)


def _align(n, a=256):
    return (n + a - 1) // a * a


class SlotLayout:
    """Field offsets/shapes/dtypes of one expert record; ``tiled``: the packed
    fields are stored MFMA-tiled (when every packed field has 16-row tiles and
    256-wide K stages, and DSV4_TILED_WEIGHTS is not 0)."""

    def __init__(self, tensors, tiled=None):
        self.shapes, self.dtypes, self.offsets, self.nbytes = {}, {}, {}, {}
        o = 0
        for k in FIELDS:
            t = tensors[k]
            self.shapes[k] = tuple(t.shape)
            self.dtypes[k] = t.dtype
            self.nbytes[k] = t.numel() * t.element_size()
            self.offsets[k] = o
            o = _align(o + self.nbytes[k])
        self.record_bytes = _align(o)
        if tiled is None:
            tiled = os.environ.get("DSV4_TILED_WEIGHTS", "1") != "0"
        self.tiled = bool(tiled) and all(
            len(self.shapes[k]) == 2 and self.shapes[k][0] % 16 == 0 and self.shapes[k][1] % 128 == 0
            and self.nbytes[k] == self.shapes[k][0] * self.shapes[k][1] for k in PACKED)

    def matches(self, tensors):
        return all(tuple(tensors[k].shape) == self.shapes[k] and
                   tensors[k].numel() * tensors[k].element_size() == self.nbytes[k] for k in FIELDS)


class SlotCache:
    def __init__(self, device, n_slots, layout: SlotLayout, pin=True):
        self.device = torch.device(device)
        self.layout = layout
        self.n_slots = int(n_slots)
        self.pool = torch.empty(self.n_slots * layout.record_bytes, dtype=torch.uint8, device=self.device)
        h = ctypes.c_void_p()
        call("dsv4_slots_create", self.device.index or 0, layout.record_bytes, self.n_slots,
             ctypes.c_void_p(self.pool.data_ptr()), 1 if pin else 0, ctypes.byref(h))
        self.h = h
        self.keys_registered = set()
        offs = np.array([layout.offsets[k] for k in FIELDS], dtype=np.int64)
        self._slot_ptrs = (self.pool.data_ptr() + np.arange(self.n_slots, dtype=np.int64)[:, None]
                           * layout.record_bytes + offs[None, :])

    def close(self):
        if self.h:
            _lib.lib().dsv4_slots_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- host pool -------------------------------------------------------
    def register(self, layer, eid, tensors):
        """Copies the six CPU tensors into the expert's host record; returns whether it is pinned."""
        if not self.layout.matches(tensors):
            raise ValueError(f"expert ({layer}, {eid}): tensor shapes differ from the registered layout")
        rec = ctypes.c_void_p()
        pinned = ctypes.c_int(0)
        call("dsv4_slots_host_record", self.h, int(layer), int(eid), 1, ctypes.byref(rec), ctypes.byref(pinned))
        buf = np.ctypeslib.as_array((ctypes.c_uint8 * self.layout.record_bytes).from_address(rec.value))
        for k in FIELDS:
            t = tensors[k].detach().to("cpu").contiguous()
            src = t.view(torch.uint8).numpy().reshape(-1) if t.element_size() == 1 else \
                t.view(-1).view(torch.uint8).numpy()
            o = self.layout.offsets[k]
            if self.layout.tiled and k in PACKED:  # tiled straight into the record
                src = np.ascontiguousarray(src)
                N, KH = self.layout.shapes[k]
                call("dsv4_mxfp4_tile_host", src.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(rec.value + o),
                     N, 2 * KH)
            else:
                buf[o:o + src.size] = src
        self.keys_registered.add((int(layer), int(eid)))
        return bool(pinned.value)

    def has(self, layer, eid):
        return (int(layer), int(eid)) in self.keys_registered

    # -- device slots ------------------------------------------------------
    def _stream(self):
        return stream_handle(self.device)

    def acquire(self, layer, eids):
        """Makes experts resident; returns (slots int32 array, n_miss)."""
        e = np.ascontiguousarray(eids, dtype=np.int32)
        slots = np.empty_like(e)
        nm = ctypes.c_int(0)
        call("dsv4_slots_acquire", self.h, int(layer), e.ctypes.data_as(ctypes.c_void_p), int(e.size),
             self._stream(), slots.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nm))
        return slots, nm.value

    def prefetch(self, layer, eids):
        e = np.ascontiguousarray(eids, dtype=np.int32)
        n = ctypes.c_int(0)
        call("dsv4_slots_prefetch", self.h, int(layer), e.ctypes.data_as(ctypes.c_void_p), int(e.size),
             ctypes.byref(n))
        return n.value

    def release(self):
        call("dsv4_slots_release", self.h, self._stream())

    def _natural(self, k, v):
        """A field of a record as the caller registered it: tiled packed fields are
        untiled into a new tensor, everything else is a view."""
        if self.layout.tiled and k in PACKED:
            from . import ops
            v = ops.tile_weights(v.view(torch.uint8).view(self.layout.shapes[k]), inverse=True).view(-1)
        return v.view(self.layout.dtypes[k]).view(self.layout.shapes[k])

    def slot_views(self, slot):
        """Device tensors of one slot in the registered shapes/dtypes (views into the
        pool; packed fields are checkpoint-layout copies when the pool is tiled)."""
        base = slot * self.layout.record_bytes
        out = {}
        for k in FIELDS:
            o = base + self.layout.offsets[k]
            out[k] = self._natural(k, self.pool[o:o + self.layout.nbytes[k]])
        return out

    def slot_copy(self, slot):
        """Like ``slot_views``, but every field is a new tensor that later acquires
        cannot overwrite (the copies are enqueued on the current stream, before
        any later copy into the slot can start)."""
        out = self.slot_views(slot)
        for k in FIELDS:
            if not (self.layout.tiled and k in PACKED):  # untiled fields are new tensors already
                out[k] = out[k].clone()
        return out

    def table(self, eids, slots, n_experts):
        """Device pointer table [E, 6] for the grouped GEMMs (pinned host staging, async copy)."""
        tab = torch.zeros((n_experts, len(FIELDS)), dtype=torch.int64, pin_memory=True)
        ptrs = self._slot_ptrs[np.asarray(slots, dtype=np.int64)]
        if self.layout.tiled:  # tag the packed fields as MFMA-tiled
            ptrs = ptrs | np.array([_lib.TILED_WEIGHTS if k in PACKED else 0 for k in FIELDS], dtype=np.int64)
        tab.numpy()[np.asarray(eids, dtype=np.int64)] = ptrs
        return tab.to(self.device, non_blocking=True)

    def copy_record(self, layer, eid, dst):
        call("dsv4_slots_copy_record", self.h, int(layer), int(eid), ctypes.c_void_p(dst.data_ptr()), self._stream())

    def record_bytes_views(self, buf):
        """The fields of a record copied into ``buf`` as uint8 views in the registered
        shapes, packed fields in the stored layout (MFMA-tiled when ``layout.tiled``)."""
        out = {}
        for k in FIELDS:
            o = self.layout.offsets[k]
            N = self.layout.shapes[k][0]
            out[k] = buf[o:o + self.layout.nbytes[k]].view(N, -1)
        return out

    def record_views(self, buf):
        """The fields of a record copied into ``buf``, as registered (see slot_views)."""
        out = {}
        for k in FIELDS:
            o = self.layout.offsets[k]
            out[k] = self._natural(k, buf[o:o + self.layout.nbytes[k]])
        return out

    def lookup(self, layer, eid):
        s = ctypes.c_int32(-1)
        call("dsv4_slots_lookup", self.h, int(layer), int(eid), ctypes.byref(s))
        return s.value

    def keys(self):
        out = np.empty(self.n_slots, dtype=np.int64)
        n = ctypes.c_int(0)
        call("dsv4_slots_keys", self.h, out.ctypes.data_as(ctypes.c_void_p), self.n_slots, ctypes.byref(n))
        return [(int(k >> 32), int(k & 0xFFFFFFFF)) for k in out[:n.value]]

    def sync(self):
        call("dsv4_slots_sync", self.h)

    def invalidate(self):
        """Forget every resident expert; reads already enqueued on the current
        stream finish before any slot is overwritten."""
        call("dsv4_slots_invalidate", self.h, self._stream())

    def stats(self):
        s = np.zeros(9, dtype=np.int64)
        call("dsv4_slots_stats", self.h, s.ctypes.data_as(ctypes.c_void_p))
        keys = ("hits", "misses", "evictions", "prefetched", "bytes_h2d", "copies", "cached", "capacity", "pinned")
        return {k: int(v) for k, v in zip(keys, s)}

    def reset_stats(self):
        call("dsv4_slots_reset_stats", self.h)


class HostLRU:
    """The native LRU core alone (no GPU): used to check the policy on the host."""

    def __init__(self, capacity):
        h = ctypes.c_void_p()
        call("dsv4_lru_create", int(capacity), ctypes.byref(h))
        self.h = h
        self.capacity = capacity

    def access(self, key):
        hit, slot, ev = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int64(0)
        call("dsv4_lru_access", self.h, int(key), ctypes.byref(hit), ctypes.byref(slot), ctypes.byref(ev))
        return bool(hit.value), slot.value, (None if ev.value < 0 else int(ev.value))

    def keys(self):
        out = np.empty(max(self.capacity, 1), dtype=np.int64)
        n = ctypes.c_int(0)
        call("dsv4_lru_keys", self.h, out.ctypes.data_as(ctypes.c_void_p), max(self.capacity, 1), ctypes.byref(n))
        return [int(k) for k in out[:n.value]]

    def __del__(self):
        try:
            _lib.lib().dsv4_lru_destroy(self.h)
        except Exception:
            pass
