"""GPU: the allocation-free layer entry point against the workspace one.

``dsv4_moe_layer_forward_noalloc`` runs the routed layer on the library's
static per-device scratch array instead of a caller workspace. Called through
the C ABI twice in a row (the second call smaller, so it runs on what the
first left in the scratch), in both profiles, its output equals
``dsv4_moe_layer_forward``'s bit for bit; a call that needs more workspace
than the scratch holds is rejected before anything is launched, and so is a
call from a second stream that the caller has not declared ordered after the
first.
"""

import ctypes

import numpy as np
import pytest
import torch

from dsv4_hip import _lib, ops, synth, PROFILE_A4W4, PROFILE_BF16, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(T, K, E, D, I, seed, dev):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(seed))
    w = synth.routing_weights(T, K, seed + 1)
    x = synth.bf16_normal(np.random.default_rng(seed + 2), (T, D)).to(dev)
    return x, torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)


def _table(E, D, I, gpu, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    experts = {}
    for e in range(E):
        d = {}
        for name, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
            d[name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=gpu, generator=g)
            d[name + "s"] = torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=gpu, generator=g)
        experts[e] = d
    return ops.expert_table(experts, E, gpu), experts


@pytest.mark.parametrize("profile", [PROFILE_BF16, PROFILE_A4W4])
def test_noalloc_layer_equals_workspace_layer_twice(gpu, profile):
    E, D, I = 64, 1024, 512
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    table, experts = _table(E, D, I, gpu, 11)
    for T, K, seed in ((96, 8, 1), (5, 6, 2)):          # second call smaller than the first
        x, ids, w = _case(T, K, E, D, I, seed, gpu)
        n = ctypes.c_int64(0)
        _lib.call("dsv4_moe_layer_workspace_bytes", T, K, E, D, I, profile, ctypes.byref(n))
        assert n.value <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(n.value, dtype=torch.uint8, device=gpu)
        y_ws = torch.empty(T, D, dtype=torch.bfloat16, device=gpu)
        y_na = torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu)
        print(f"noalloc profile={profile} T={T} K={K}", flush=True)
        _lib.call("dsv4_moe_layer_forward", profile, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K, E, D, I,
                  _p(table), ctypes.c_float(10.0), _p(ws), n.value, _p(y_ws), st)
        _lib.call("dsv4_moe_layer_forward_noalloc", profile, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K, E, D,
                  I, _p(table), ctypes.c_float(10.0), _p(y_na), 0, st)
        torch.cuda.synchronize()
        assert torch.equal(y_na.view(torch.int16), y_ws.view(torch.int16)), (profile, T)
        assert torch.isfinite(y_na.float()).all()


def test_noalloc_layer_rejects_calls_beyond_its_scratch(gpu):
    lib = _lib.lib()
    T, K, E, D, I = 2048, 8, 256, 4096, 2048
    n = ctypes.c_int64(0)
    _lib.call("dsv4_moe_layer_workspace_bytes", T, K, E, D, I, PROFILE_BF16, ctypes.byref(n))
    assert n.value > _lib.NOALLOC_SCRATCH_BYTES
    dummy = torch.empty(16, dtype=torch.uint8, device=gpu)
    rc = lib.dsv4_moe_layer_forward_noalloc(PROFILE_BF16, RULE_OCP_FLOOR, _p(dummy), _p(dummy), 1, _p(dummy), T, K,
                                            E, D, I, _p(dummy), ctypes.c_float(10.0), _p(dummy), 0, None)
    assert rc == -3 and "scratch" in lib.dsv4_last_error().decode()


def test_noalloc_layer_refuses_an_unordered_second_stream(gpu):
    """The scratch belongs to the stream of the device's last call: a call from
    another stream is refused before anything is enqueued, unless the caller
    passes DSV4_NOALLOC_STREAMS_ORDERED; the flagged call then owns it."""
    E, D, I, T, K = 64, 1024, 512, 16, 8
    lib = _lib.lib()
    table, experts = _table(E, D, I, gpu, 12)
    x, ids, w = _case(T, K, E, D, I, 7, gpu)
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    s2 = torch.cuda.Stream(gpu)
    st2 = ctypes.c_void_p(s2.cuda_stream)
    args = lambda y: (PROFILE_BF16, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K, E, D, I, _p(table),  # noqa: E731
                      ctypes.c_float(10.0), _p(y))
    y1 = torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu)
    y2 = torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu)
    print("noalloc streams: first call on the current stream", flush=True)
    _lib.call("dsv4_moe_layer_forward_noalloc", *args(y1), 0, st)
    rc = lib.dsv4_moe_layer_forward_noalloc(*args(y2), 0, st2)
    msg = lib.dsv4_last_error().decode()
    assert rc == -5 and "stream" in msg, (rc, msg)
    assert lib.dsv4_moe_layer_forward_noalloc(*args(y2), 2, st2) == -3      # unknown flag bit
    torch.cuda.synchronize(gpu)
    assert torch.isnan(y2.float()).all()                                     # nothing was enqueued
    s2.wait_stream(torch.cuda.current_stream(gpu))
    print("noalloc streams: ordered call on a second stream", flush=True)
    _lib.call("dsv4_moe_layer_forward_noalloc", *args(y2), _lib.NOALLOC_STREAMS_ORDERED, st2)
    _lib.call("dsv4_moe_layer_forward_noalloc", *args(y2), 0, st2)           # s2 owns the scratch now
    torch.cuda.synchronize(gpu)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert lib.dsv4_moe_layer_forward_noalloc(*args(y1), 0, st) == -5
    _lib.call("dsv4_moe_layer_forward_noalloc", *args(y1), _lib.NOALLOC_STREAMS_ORDERED, st)   # hand it back
    torch.cuda.synchronize(gpu)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    del experts
