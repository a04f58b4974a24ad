"""GPU: lifetimes of slot-cache contents (offload.py:122-133 semantics).

* ``invalidate`` may drop every resident expert while work the caller already
  enqueued still reads a slot; a copy into that slot made afterwards must wait
  for those reads.
* ``get_packed`` hands out tensors the caller owns (the reference returns the
  ``.to(device)`` copies it cached): a later acquire that reuses the slot does
  not change them.
* A layer that routes to more experts than the packed slot cache holds runs in
  parts and gives the same output, bit for bit, as the one-part layer; at
  2048 routed rows and more (64-row blocks) as well, and from 16,384 routed
  rows, where the one-part layer runs its hot experts on the large-tile kernel,
  bit for bit in a4w4 and within the GEMM bar in the bf16 profile.
"""

import types

import numpy as np
import pytest
import torch
from torch import nn

from offload import ExpertBank
import dsv4_plugin.models.deepseek_v4 as mod
from dsv4_plugin.core.engine import ExpertOffloadEngine
from dsv4_hip import synth
from dsv4_hip.slots import FIELDS, SlotCache, SlotLayout
from oracle import mxfp4 as Q
from oracle import moe as M

pytestmark = pytest.mark.gpu


def _expert(seed, n1=128, k1=512, n2=512, k2=128):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, (n, k) in (("w1", (n1, k1)), ("w2", (n2, k2)), ("w3", (n1, k1))):
        out[name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, generator=g)
        out[name + "s"] = torch.randint(100, 150, (n, k // 32), dtype=torch.uint8, generator=g)
    return out


def _busy(dev, n=6):
    """Enqueue a few milliseconds of unrelated work on the current stream."""
    a = torch.randn(4096, 4096, device=dev)
    for _ in range(n):
        a = a @ a
        a = a / a.abs().max()
    return a


def test_invalidate_orders_later_copies_after_enqueued_reads(gpu):
    n_slots = 4
    tens = {e: _expert(40 + e) for e in range(12)}
    layout = SlotLayout(tens[0], tiled=False)
    cache = SlotCache(gpu, n_slots, layout, pin=True)
    for e, t in tens.items():
        cache.register(7, e, t)
    pool2d = cache.pool.view(n_slots, layout.record_bytes)
    first = np.arange(4, dtype=np.int32)
    slots, nm = cache.acquire(7, first)
    assert nm == 4
    _busy(gpu)                                            # keeps the compute stream busy
    seen = pool2d.index_select(0, torch.from_numpy(slots.astype(np.int64)).to(gpu))   # reads the 4 slots
    cache.invalidate()                                    # drops them while the read is queued
    slots2, nm2 = cache.acquire(7, np.arange(4, 8, dtype=np.int32))   # reuses the same 4 slots
    assert nm2 == 4 and sorted(slots2.tolist()) == sorted(slots.tolist())
    torch.cuda.synchronize()
    got = seen.cpu().numpy()
    off = layout.offsets
    for i, e in enumerate(first):
        for k in FIELDS:
            want = tens[int(e)][k].numpy().reshape(-1)
            assert np.array_equal(got[i, off[k]:off[k] + want.size], want), (int(e), k)
    cache.close()


@pytest.mark.parametrize("tiled", ["1", "0"])
def test_get_packed_returns_tensors_later_acquires_do_not_change(gpu, monkeypatch, tiled):
    monkeypatch.setenv("DSV4_PACKED_SLOTS", "2")
    monkeypatch.setenv("DSV4_TILED_WEIGHTS", tiled)
    bank = ExpertBank(capacity=1, device="cuda:0")
    tens = {e: _expert(90 + e) for e in range(6)}
    for e, t in tens.items():
        bank.register(2, e, *(t[k] for k in FIELDS))
    p0 = bank.get_packed(2, 0)
    for e in range(1, 6):                                 # evicts expert 0's slot several times
        bank.get_packed(2, e)
    torch.cuda.synchronize()
    for k in FIELDS:
        assert np.array_equal(p0[k].cpu().numpy(), tens[0][k].numpy()), k
    assert bank.stats()["packed_evictions"] >= 4


def _plugin(engine, E, K, layer, D):
    m = mod.OffloadDeepseekV4MoE.__new__(mod.OffloadDeepseekV4MoE)
    nn.Module.__init__(m)
    m.hash, m.topk, m.renormalize, m.scoring_func = False, K, True, "sqrtsoftplus"
    m.routed_scaling_factor, m.swiglu_limit, m.n_routed_experts = 1.5, 10.0, E
    m.is_sequence_parallel, m.shared_experts, m.layer_idx, m.engine = False, None, layer, engine
    g = torch.Generator().manual_seed(layer)
    m.gate = types.SimpleNamespace(weight=(torch.randn(E, D, generator=g) * 0.05).to("cuda:0"),
                                   e_score_correction_bias=(torch.randn(E, generator=g) * 0.01).to("cuda:0"),
                                   tid2eid=None)
    return m


def _engine(monkeypatch, slots, E, D, I, layer, host, shared=None):
    monkeypatch.setenv("DSV4_PACKED_SLOTS", str(slots))
    eng = ExpertOffloadEngine(slot_capacity=4, device="cuda:0")
    for e in range(E):
        for w in ("w1", "w2", "w3"):
            eng.capture(f"layers.{layer}.ffn.experts.{e}.{w}.weight", torch.from_numpy(host[e][w + "p"]).view(torch.int8))
            eng.capture(f"layers.{layer}.ffn.experts.{e}.{w}.scale",
                        torch.from_numpy(host[e][w + "s"]).view(torch.float8_e8m0fnu))
    if shared is not None:
        for w in ("w1", "w2", "w3"):
            eng.capture_shared(f"layers.{layer}.ffn.shared_experts.{w}.weight", torch.from_numpy(shared[w]))
            eng.capture_shared(f"layers.{layer}.ffn.shared_experts.{w}.scale", torch.from_numpy(shared[w + "s"]))
    return eng


@pytest.mark.parametrize("profile", ["bf16", "a4w4", "bf16_shared"])
def test_layer_with_more_routed_experts_than_slots_runs_in_parts(gpu, monkeypatch, profile):
    E, K, D, I, T, layer = 32, 6, 1024, 512, 16, 5
    host = {e: synth.expert_weights(e, D, I) for e in range(E)}
    sh = synth.shared_expert_weights(55, D, I) if profile == "bf16_shared" else None
    monkeypatch.setattr(mod, "_MXFP4_GMM", profile == "a4w4")
    monkeypatch.setattr(mod, "_FUSE_SHARED", sh is not None)
    monkeypatch.setattr(mod, "_FUSED_ROUTE", False)
    x = (synth.bf16_normal(np.random.default_rng(8), (T, D)).float() * 0.5).to(torch.bfloat16).to(gpu)
    small = _engine(monkeypatch, 7, E, D, I, layer, host, sh)        # 7 slots: the layer runs in parts
    big = _engine(monkeypatch, 64, E, D, I, layer, host, sh)         # every expert fits: one part
    m_small, m_big = _plugin(small, E, K, layer, D), _plugin(big, E, K, layer, D)
    w, idx = m_small._route(x, None)
    n_routed = len(np.unique(idx.cpu().numpy()))
    assert n_routed > 7
    y_small = m_small.forward(x)
    y_big = m_big.forward(x)
    torch.cuda.synchronize()
    bits = lambda t: t.cpu().view(torch.int16).numpy()  # noqa: E731
    assert np.array_equal(bits(y_small), bits(y_big))
    s = small.stats()
    assert s["packed_misses"] == n_routed and s["packed_cached"] == 7
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    if profile == "a4w4":
        ref = M.routed_a4w4(xb, idx.cpu().numpy(), w.cpu().numpy(), host, n_experts=E, rule="ocp_floor")["y"]
        tol = 2e-2
    elif profile == "bf16":
        ref = M.routed_bf16(xb, idx.cpu().numpy(), w.cpu().numpy(), host, n_experts=E)["y"]
        tol = 1e-2
    else:
        ref = M.routed_plus_shared_bf16(xb, idx.cpu().numpy(), w.cpu().numpy(), host, sh, n_experts=E)[0]
        tol = 1e-2
    want = Q.bf16_bits_to_f32(ref)
    got = Q.bf16_bits_to_f32(bits(y_small).view(np.uint16))
    err = float(np.abs(got - want).max() / np.abs(want).max())
    print(f"parts profile={profile} rel_err={err:.3e}")
    assert err <= tol


@pytest.mark.parametrize("T,profile", [(256, "bf16"), (256, "a4w4"), (2048, "bf16"), (2048, "a4w4")])
def test_prefill_sized_layer_in_parts_matches_one_part(gpu, monkeypatch, T, profile):
    """2048 routed rows (64-row blocks) and 16,384 (the one-part layer splits its
    hot experts onto the large-tile kernel; hidden and inter 1024 allow it)."""
    E, K, D, I, layer = 32, 8, 1024, 1024, 6
    host = {e: synth.expert_weights(e, D, I) for e in range(E)}
    monkeypatch.setattr(mod, "_MXFP4_GMM", profile == "a4w4")
    monkeypatch.setattr(mod, "_FUSE_SHARED", False)
    monkeypatch.setattr(mod, "_FUSED_ROUTE", False)
    x = (synth.bf16_normal(np.random.default_rng(9), (T, D)).float() * 0.5).to(torch.bfloat16).to(gpu)
    small = _engine(monkeypatch, 7, E, D, I, layer, host)
    big = _engine(monkeypatch, 64, E, D, I, layer, host)
    m_small, m_big = _plugin(small, E, K, layer, D), _plugin(big, E, K, layer, D)
    _, idx = m_small._route(x, None)
    counts = np.bincount(idx.cpu().numpy().reshape(-1), minlength=E)
    print(f"parts T={T} profile={profile}: {int((counts > 0).sum())} experts, max rows {int(counts.max())}",
          flush=True)
    y_small = m_small.forward(x)
    y_big = m_big.forward(x)
    torch.cuda.synchronize()
    a = y_small.float().cpu().numpy()
    b = y_big.float().cpu().numpy()
    assert np.isfinite(a).all() and np.isfinite(b).all()
    if profile == "a4w4" or T * K < 16384:
        assert np.array_equal(y_small.cpu().view(torch.int16).numpy(), y_big.cpu().view(torch.int16).numpy())
    else:
        assert (counts >= 128).any()                 # the one-part layer does split
        ref = np.maximum(np.abs(b), np.sqrt(np.mean(b * b)))
        worst = float((np.abs(a - b) / ref).max())
        print(f"parts vs one part (bf16, split) worst {worst:.3e}")
        assert worst <= 3e-2
