"""GPU: the layer's concurrent hot/cold launches against the one-stream order.

From 16,384 routed rows in the bf16 profile the layer runs the experts with at
least 128 rows on the large-tile kernel, on a side stream forked from the
caller's stream after the align and joined before the combine, while the
tiled kernel takes the other experts on the caller's stream. The allocation-
free entry point keeps every launch on the caller's stream, so the two entry
points on the same inputs compare the concurrent schedule with the serial
one: the outputs must agree bit for bit (the two kernels write disjoint rows).
Called twice in a row, with the second call's inputs changed, so that a join
that did not hold would show up as stale rows of the first call.

Under stream capture the layer keeps every launch on the capturing stream (the
library's side stream would otherwise join that capture): a split layer
captured into a graph and replayed, with eager work between the replays,
gives the eager output bit for bit on every replay.
"""

import ctypes

import numpy as np
import pytest
import torch

from dsv4_hip import _lib, ops, synth, PROFILE_BF16, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_concurrent_split_equals_one_stream(gpu):
    T, K, E, D, I = 2048, 8, 64, 1024, 1024  # 16,384 routed rows: the bf16 split's threshold
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    experts = {}
    for e in range(E):
        d = {}
        for name, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
            d[name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=gpu, generator=g)
            d[name + "s"] = torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=gpu, generator=g)
        experts[e] = d
    table = ops.expert_table(experts, E, gpu)
    n = ctypes.c_int64(0)
    _lib.call("dsv4_moe_layer_workspace_bytes", T, K, E, D, I, PROFILE_BF16, ctypes.byref(n))
    assert n.value <= _lib.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(n.value, dtype=torch.uint8, device=gpu)
    for seed in (1, 2):
        ids_np = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3 + seed), np.random.default_rng(seed))
        counts = np.bincount(ids_np.reshape(-1), minlength=E)
        assert (counts >= 128).any() and (counts < 128).any()  # both launches have work
        ids = torch.from_numpy(ids_np).to(gpu)
        w = torch.from_numpy(synth.routing_weights(T, K, seed + 10)).to(gpu)
        x = synth.bf16_normal(np.random.default_rng(seed + 20), (T, D)).to(gpu)
        y_side = torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu)
        y_one = torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu)
        print(f"concurrent split seed={seed}: {int((counts >= 128).sum())} hot experts", flush=True)
        _lib.call("dsv4_moe_layer_forward", PROFILE_BF16, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K, E, D, I,
                  _p(table), ctypes.c_float(10.0), _p(ws), n.value, _p(y_side), st)
        _lib.call("dsv4_moe_layer_forward_noalloc", PROFILE_BF16, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K,
                  E, D, I, _p(table), ctypes.c_float(10.0), _p(y_one), 0, st)
        torch.cuda.synchronize(gpu)
        a = y_side.view(torch.int16).cpu().numpy()
        b = y_one.view(torch.int16).cpu().numpy()
        assert np.isfinite(y_one.float().cpu().numpy()).all()
        assert np.array_equal(a, b), f"{int((a != b).sum())} elements differ"


def test_split_layer_captured_in_a_graph_replays_exactly(gpu):
    T, K, E, D, I = 2048, 8, 64, 1024, 1024   # 16,384 routed rows: the split runs
    g = torch.Generator(device=gpu)
    g.manual_seed(9)
    experts = {}
    for e in range(E):
        d = {}
        for name, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
            d[name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=gpu, generator=g)
            d[name + "s"] = torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=gpu, generator=g)
        experts[e] = d
    table = ops.expert_table(experts, E, gpu)
    ids_np = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 4), np.random.default_rng(3))
    counts = np.bincount(ids_np.reshape(-1), minlength=E)
    assert (counts >= 128).any() and (counts < 128).any()
    ids = torch.from_numpy(ids_np).to(gpu)
    w = torch.from_numpy(synth.routing_weights(T, K, 13)).to(gpu)
    x = synth.bf16_normal(np.random.default_rng(23), (T, D)).to(gpu)
    n = ctypes.c_int64(0)
    _lib.call("dsv4_moe_layer_workspace_bytes", T, K, E, D, I, PROFILE_BF16, ctypes.byref(n))
    ws = torch.empty(n.value, dtype=torch.uint8, device=gpu)
    y_eager = torch.empty(T, D, dtype=torch.bfloat16, device=gpu)
    y_graph = torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu)

    def layer(y):
        st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
        _lib.call("dsv4_moe_layer_forward", PROFILE_BF16, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K, E, D, I,
                  _p(table), ctypes.c_float(10.0), _p(ws), n.value, _p(y), st)

    print("graph capture of the split layer: eager", flush=True)
    layer(y_eager)
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    print("graph capture of the split layer: capture", flush=True)
    with torch.cuda.graph(graph):
        layer(y_graph)
    torch.cuda.synchronize(gpu)
    want = y_eager.view(torch.int16).cpu()
    for rep in range(3):
        y_graph.fill_(float("nan"))
        layer(y_eager)                                   # eager work between the replays
        print(f"graph capture of the split layer: replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize(gpu)
        assert torch.equal(y_graph.view(torch.int16).cpu(), want), f"replay {rep}"
    del graph
