"""GPU: decode-sized layers captured into one HIP graph and replayed.

A serving loop captures its decode step once and replays it. Eight decode layers
(8 tokens, top-8 of 64 experts, each layer with its own weights, routing and
output) are captured into one graph in each profile: the bf16 profile (the
16-row kernels with the FP8 quantisation of h as its own launch), a4w4 (h
quantised in the gate/up epilogue) and pure bf16. The graph is replayed three
times with eager calls of the same layers (on other outputs) and a host
synchronisation between the replays; every replay's outputs must equal the
eager outputs bit for bit, and the graph's outputs start as NaN so that a
replay that skipped a layer would show."""

import ctypes

import numpy as np
import pytest
import torch

from dsv4_hip import _lib, ops, synth, PROFILE_A4W4, PROFILE_BF16, PROFILE_BF16_PURE, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("profile", [PROFILE_BF16, PROFILE_A4W4, PROFILE_BF16_PURE])
def test_decode_layers_captured_in_a_graph_replay_exactly(gpu, profile):
    L, T, K, E, D, I = 8, 8, 8, 64, 1024, 512
    g = torch.Generator(device=gpu)
    g.manual_seed(31 + profile)
    layers = []
    for li in range(L):
        experts = {}
        for e in range(E):
            d = {}
            for name, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
                d[name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=gpu, generator=g)
                d[name + "s"] = torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=gpu, generator=g)
            experts[e] = d
        rng = np.random.default_rng(100 * profile + li)
        ids = torch.from_numpy(synth.zipf_topk(T, K, E, synth.rank_permutation(E, li), rng)).to(gpu)
        w = torch.from_numpy(synth.routing_weights(T, K, 7 + li)).to(gpu)
        x = synth.bf16_normal(rng, (T, D)).to(gpu)
        layers.append((ops.expert_table(experts, E, gpu, tiled=li % 2 == 0), ids, w, x))
    n = ctypes.c_int64(0)
    _lib.call("dsv4_moe_layer_workspace_bytes", T, K, E, D, I, profile, ctypes.byref(n))
    ws = torch.empty(n.value, dtype=torch.uint8, device=gpu)
    y_eager = [torch.empty(T, D, dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    y_graph = [torch.full((T, D), float("nan"), dtype=torch.bfloat16, device=gpu) for _ in range(L)]

    def run(ys):
        st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
        for (table, ids, w, x), y in zip(layers, ys):
            _lib.call("dsv4_moe_layer_forward", profile, RULE_OCP_FLOOR, _p(x), _p(ids), 1, _p(w), T, K, E, D, I,
                      _p(table), ctypes.c_float(10.0), _p(ws), n.value, _p(y), st)

    print(f"decode graph, profile {profile}: eager", flush=True)
    run(y_eager)
    torch.cuda.synchronize(gpu)
    want = [y.view(torch.int16).cpu() for y in y_eager]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    print(f"decode graph, profile {profile}: capture", flush=True)
    with torch.cuda.graph(graph, stream=side):
        run(y_graph)
    torch.cuda.synchronize(gpu)
    for rep in range(3):
        for y in y_graph:
            y.fill_(float("nan"))
        run(y_eager)                                   # eager work between the replays
        torch.cuda.synchronize(gpu)
        print(f"decode graph, profile {profile}: replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize(gpu)
        for li, y in enumerate(y_graph):
            assert torch.equal(y.view(torch.int16).cpu(), want[li]), f"replay {rep}, layer {li}"
    del graph
