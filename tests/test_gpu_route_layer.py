"""GPU: the routed layer with its router in one C call
(``dsv4_moe_routed_layer_forward``, ``OffloadDeepseekV4MoE._routed`` with its
``_route``, ``deepseek_v4.py:118-245``) against ``dsv4_moe_route`` followed by
``dsv4_moe_layer_forward(_shared)`` on the routed ids.

Up to 16 tokens the top-k, the expert layout and the quantisation of x share
one launch; above, the router's own launches run first. Either way the ids,
weights and layer output must equal the two-call path bit for bit (the same
per-token top-k code, the same layout, the same GEMMs); the two-call path is
itself pinned to the oracle by the router and layer tests."""

import numpy as np
import pytest
import torch

from dsv4_hip import ops, synth, PROFILE_A4W4, PROFILE_BF16, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu


def _device_experts(E, D, I, dev, seed):
    """Random MXFP4 experts generated on the device (every expert of the layer is
    present, as when the whole layer sits in the slot cache). The pointer table
    holds raw addresses: callers keep the returned tensors alive while it is used."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    ex = {}
    for e in range(E):
        d = {}
        for name, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
            d[name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=g)
            d[name + "s"] = torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=dev, generator=g)
        ex[e] = d
    return ex


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy()


CASES = [  # T, E, D, I, K, scoring, bias, profile
    (1, 256, 4096, 2048, 8, "sqrtsoftplus", True, PROFILE_BF16),
    (8, 256, 4096, 2048, 8, "sqrtsoftplus", True, PROFILE_BF16),   # the decode layer
    (16, 256, 1024, 512, 8, "softmax", False, PROFILE_A4W4),
    (8, 64, 1024, 512, 6, "sigmoid", True, PROFILE_BF16),
    (5, 512, 512, 512, 8, "sqrtsoftplus", True, PROFILE_A4W4),     # widest expert count
    (17, 256, 1024, 512, 8, "sqrtsoftplus", True, PROFILE_BF16),   # router launches first
    (300, 128, 1024, 512, 8, "softmax", True, PROFILE_BF16),       # 2400 rows: chunked align, 64-row blocks
]


@pytest.mark.parametrize("T,E,D,I,K,scoring,use_bias,profile", CASES)
def test_routed_layer_equals_route_then_layer(gpu, T, E, D, I, K, scoring, use_bias, profile):
    rng = np.random.default_rng(T * 7 + E)
    x = synth.bf16_normal(rng, (T, D)).to(gpu)
    gate = torch.from_numpy((rng.standard_normal((E, D)) * 0.03).astype(np.float32)).to(gpu)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(gpu) if use_bias else None
    experts = _device_experts(E, D, I, gpu, T + E)
    table = ops.expert_table(experts, E, gpu)
    runner = ops.LayerRunner(gpu, E, D, I)
    w_ref, ids_ref = ops.route(x, gate, K, scoring, bias=bias, renormalize=True, scale=1.5)
    y_ref = runner.forward(x, ids_ref, w_ref, table, profile=profile, rule=RULE_OCP_FLOOR).clone()
    y, w, ids = runner.forward_routed(x, gate, K, table, scoring, bias=bias, renormalize=True, scale=1.5,
                                      profile=profile, rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids_ref)
    assert torch.equal(w.view(torch.int32), w_ref.view(torch.int32))
    assert np.array_equal(_bits(y), _bits(y_ref))
    # repeated call on the same runner (workspace reused) gives the same bits
    y2, _, _ = runner.forward_routed(x, gate, K, table, scoring, bias=bias, renormalize=True, scale=1.5,
                                     profile=profile, rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y2), _bits(y_ref))
    del experts


@pytest.mark.parametrize("T", [6, 40])
def test_routed_layer_hash_table_with_bad_ids(gpu, T):
    E, D, I, K, V = 64, 1024, 512, 4, 500
    rng = np.random.default_rng(T)
    x = synth.bf16_normal(rng, (T, D)).to(gpu)
    gate = torch.from_numpy((rng.standard_normal((E, D)) * 0.03).astype(np.float32)).to(gpu)
    tab = np.stack([rng.permutation(E)[:K] for _ in range(V)]).astype(np.int64)
    tab[7, 1] = E + 3                       # a table entry outside [0, E)
    inp = rng.integers(0, V, T)
    inp[0] = 7
    inp[T - 1] = V + 9                      # an input id outside the vocabulary
    tab_d, inp_d = torch.from_numpy(tab).to(gpu), torch.from_numpy(inp).to(gpu)
    experts = _device_experts(E, D, I, gpu, 3)
    table = ops.expert_table(experts, E, gpu)
    runner = ops.LayerRunner(gpu, E, D, I)
    st_ref = torch.zeros(1, dtype=torch.int32, device=gpu)
    st = torch.zeros(1, dtype=torch.int32, device=gpu)
    w_ref, ids_ref = ops.route(x, gate, K, "sqrtsoftplus", tid2eid=tab_d, input_ids=inp_d, status=st_ref)
    y_ref = runner.forward(x, ids_ref, w_ref, table).clone()
    y, w, ids = runner.forward_routed(x, gate, K, table, "sqrtsoftplus", tid2eid=tab_d, input_ids=inp_d, status=st)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids_ref) and torch.equal(w.view(torch.int32), w_ref.view(torch.int32))
    assert np.array_equal(_bits(y), _bits(y_ref))
    assert int(st.item()) == int(st_ref.item()) == 2
    assert int(ids[T - 1].min()) == -1 and float(w[T - 1].abs().sum()) == 0.0
    del experts


@pytest.mark.parametrize("T", [8, 300])
def test_routed_layer_with_shared_expert(gpu, T):
    E, D, I, K = 64, 1024, 512, 8
    rng = np.random.default_rng(50 + T)
    x = synth.bf16_normal(rng, (T, D)).to(gpu)
    gate = torch.from_numpy((rng.standard_normal((E, D)) * 0.03).astype(np.float32)).to(gpu)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(gpu)
    experts = _device_experts(E, D, I, gpu, 9)
    table = ops.expert_table(experts, E, gpu)
    sh = {k: torch.from_numpy(v).to(gpu) for k, v in synth.shared_expert_weights(4, D, I).items()}
    prep = ops.prepare_shared_expert(sh["w1"], sh["w1s"], sh["w3"], sh["w3s"], sh["w2"], sh["w2s"])
    runner = ops.LayerRunner(gpu, E, D, I)
    w_ref, ids_ref = ops.route(x, gate, K, "sqrtsoftplus", bias=bias)
    y_ref = runner.forward(x, ids_ref, w_ref, table, shared=prep).clone()
    y, w, ids = runner.forward_routed(x, gate, K, table, "sqrtsoftplus", bias=bias, shared=prep)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids_ref)
    assert np.array_equal(_bits(y), _bits(y_ref))
    del experts


def test_routed_layer_rejects_bad_arguments(gpu):
    E, D, I = 64, 512, 512
    runner = ops.LayerRunner(gpu, E, D, I)
    x = torch.zeros(2, D, dtype=torch.bfloat16, device=gpu)
    gate = torch.zeros(E, D, dtype=torch.float32, device=gpu)
    table = torch.zeros(E, 6, dtype=torch.int64, device=gpu)
    with pytest.raises(ValueError, match="gate weight"):
        runner.forward_routed(x, gate[:, :256], 4, table)
    with pytest.raises(RuntimeError, match="input_ids"):
        runner.forward_routed(x, gate, 4, table, tid2eid=torch.zeros(10, 4, dtype=torch.int32, device=gpu))
    with pytest.raises(Exception, match="top-k"):
        runner.forward_routed(x, gate, 65, table)
