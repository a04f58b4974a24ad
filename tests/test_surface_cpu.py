"""Host-side behaviour of the plugin surface (CPU only): checkpoint-key parsing,
the load_weights tee, the CPU ExpertBank degrade path, patch installation,
and the native LRU core against the oracle LRU."""

import types

import numpy as np
import pytest
import torch

import dsv4_plugin.core.engine as eng
import dsv4_plugin.models.deepseek_v4 as mod
from dsv4_plugin.core.engine import ExpertOffloadEngine, is_expert_weight, parse_expert_name
from dsv4_hip.slots import HostLRU
from oracle.lru import LRUOracle
from offload import ExpertBank

N_LAYERS, N_EXPERTS = 43, 256


def synthetic_weight_map():
    """Every routed-expert key of a 43-layer x 256-expert checkpoint, one MTP block,
    plus non-expert keys (the names of test_plugin_load.py:40-66)."""
    keys = []
    for l in range(N_LAYERS):
        for e in range(N_EXPERTS):
            for w in ("w1", "w2", "w3"):
                for kind in ("weight", "scale"):
                    keys.append(f"layers.{l}.ffn.experts.{e}.{w}.{kind}")
        keys += [f"layers.{l}.ffn.gate.weight", f"layers.{l}.attn.wq_a.weight",
                 f"layers.{l}.ffn.shared_experts.w1.weight"]
    for e in range(N_EXPERTS):
        for w in ("w1", "w2", "w3"):
            for kind in ("weight", "scale"):
                keys.append(f"mtp.0.ffn.experts.{e}.{w}.{kind}")
    keys += ["embed.weight", "head.weight", "mtp.0.norm.weight"]
    return keys


def test_name_coverage_and_parse():
    wm = synthetic_weight_map()
    main = [k for k in wm if is_expert_weight(k)]
    mtp = [k for k in wm if ".ffn.experts." in k and not is_expert_weight(k)]
    assert len(main) == N_LAYERS * N_EXPERTS * 6
    assert all(k.startswith("mtp.") for k in mtp) and len(mtp) == N_EXPERTS * 6
    assert parse_expert_name("layers.42.ffn.experts.255.w2.scale") == (42, 255, "w2", "scale")
    assert parse_expert_name("mtp.0.ffn.experts.7.w1.weight") == (-1, 7, "w1", "weight")
    assert parse_expert_name("model.layers.3.ffn.experts.1.w3.weight") == (3, 1, "w3", "weight")
    assert parse_expert_name("layers.3.ffn.shared_experts.w1.weight") is None
    assert is_expert_weight("mtp.0.ffn.experts.7.w1.weight", include_mtp=True)


def test_tee_split_captures_every_expert(capsys):
    # test_plugin_load.py:69-99 with a recording stub in place of the wrapped loader
    wm = synthetic_weight_map()
    engine = ExpertOffloadEngine(slot_capacity=64, device="cpu")
    saved_engine, eng._ENGINE = eng._ENGINE, engine
    received = []

    def stub_original(self, weights):
        for name, _ in weights:
            received.append(name)
        return set()

    saved = mod._ORIG_LOAD_WEIGHTS
    mod._ORIG_LOAD_WEIGHTS = stub_original
    try:
        it = ((k, torch.zeros(1, dtype=torch.uint8)) for k in wm)
        mod._offload_load_weights(object(), it)
    finally:
        mod._ORIG_LOAD_WEIGHTS = saved
        eng._ENGINE = saved_engine
    non_main = {k for k in wm if not is_expert_weight(k)}
    assert engine.captured == N_LAYERS * N_EXPERTS
    assert set(received) == non_main and len(received) == len(wm) - N_LAYERS * N_EXPERTS * 6
    assert engine.stats()["parked"] == 0 and engine.bank.num_experts() == N_LAYERS * N_EXPERTS


def test_cpu_bank_degrades_pin_and_refuses_compute(capsys):
    bank = ExpertBank(capacity=4, device="cpu", pin=True)
    t = [torch.zeros(4, 2, dtype=torch.uint8)] * 6
    bank.register(0, 0, *t)
    assert bank.has(0, 0) and not bank.has(0, 1) and bank.num_experts() == 1
    if not torch.cuda.is_available():  # pin_memory needs a GPU: the reference's degrade branch
        assert bank.pin is False and "pin_memory failed" in capsys.readouterr().out
    with pytest.raises(RuntimeError, match="ROCm device"):
        bank.get(0, 0)
    with pytest.raises(RuntimeError, match="ROCm device"):
        bank.get_packed(0, 0)
    s = bank.stats()
    for k in ("hits", "misses", "evictions", "hit_rate", "cached", "capacity", "packed_hits", "packed_misses",
              "packed_hit_rate", "packed_cached", "packed_capacity", "pinned"):
        assert k in s
    assert s["packed_capacity"] == 16


def test_packed_capacity_env(monkeypatch):
    monkeypatch.setenv("DSV4_PACKED_SLOTS", "7")
    assert ExpertBank(capacity=4, device="cpu").packed_capacity == 7


def test_native_lru_matches_oracle_random_sequences():
    rng = np.random.default_rng(0)
    for cap in (1, 3, 16, 64):
        nat, ora = HostLRU(cap), LRUOracle(cap)
        keys = rng.zipf(1.3, size=5000) % 97
        for k in keys:
            h1, _, ev1 = nat.access(int(k))
            h2, ev2 = ora.access(int(k))
            assert h1 == h2 and ev1 == ev2
        assert nat.keys() == list(ora.cache.keys())


def test_native_lru_known_answer_and_capacity_zero():
    # test_offload.py:67-86 on the native core
    lru = HostLRU(4)
    for e in range(4):
        assert lru.access(e)[0] is False
    assert lru.access(0)[0] is True
    hit, _, ev = lru.access(100)
    assert not hit and ev == 1
    assert lru.keys() == [2, 3, 0, 100]
    z = HostLRU(0)
    assert z.access(5) == (False, -1, None) and z.access(5) == (False, -1, None)


def test_install_patches_without_vllm_is_noop():
    assert mod.v4 is None  # no vLLM in this image
    mod._PATCHED = False
    mod.install_patches()
    assert mod._PATCHED
    import dsv4_plugin
    dsv4_plugin.register_model()  # idempotent


def test_moe_module_constructs_without_vllm(monkeypatch):
    cfg = types.SimpleNamespace(routed_scaling_factor=1.5, swiglu_limit=10.0, n_routed_experts=16,
                                n_shared_experts=1, num_experts_per_tok=4, norm_topk_prob=True,
                                scoring_func="sqrtsoftplus", hidden_size=512, num_hash_layers=3,
                                vocab_size=100)
    pc = types.SimpleNamespace(use_sequence_parallel_moe=False, enable_eplb=False,
                               eplb_config=types.SimpleNamespace(num_redundant_experts=0))
    monkeypatch.setattr(eng, "_ENGINE", ExpertOffloadEngine(slot_capacity=4, device="cpu"))
    m = mod.OffloadDeepseekV4MoE(cfg, pc, prefix="model.layers.5.mlp")
    assert m.layer_idx == 5 and not m.hash and m.gate.weight.shape == (16, 512)
    h = mod.OffloadDeepseekV4MoE(cfg, pc, prefix="model.layers.1.mlp")
    assert h.hash and h.gate.tid2eid.shape == (100, 4)
    with pytest.raises(RuntimeError, match="input_ids"):
        h._route(torch.zeros(2, 512), None)
    # routing runs on the HIP router only: host tensors raise instead of taking a CPU path
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        m._route(torch.randn(3, 512), None)


def test_tee_keeps_a_copy_of_the_shared_expert():
    # shared-expert keys still reach the wrapped loader (its shared MLP loads them);
    # the engine keeps a host copy per layer for the fused launch
    from dsv4_plugin.core.engine import parse_shared_name
    assert parse_shared_name("model.layers.7.ffn.shared_experts.w2.scale") == (7, "w2", "scale")
    assert parse_shared_name("layers.7.ffn.experts.3.w2.scale") is None
    assert parse_shared_name("mtp.0.ffn.shared_experts.w1.weight") is None
    engine = ExpertOffloadEngine(slot_capacity=4, device="cpu")
    saved_engine, eng._ENGINE = eng._ENGINE, engine
    received = []

    def stub_original(self, weights):
        received.extend(name for name, _ in weights)

    names = [f"model.layers.{l}.ffn.shared_experts.{w}.{k}" for l in (1, 2) for w in ("w1", "w2", "w3")
             for k in ("weight", "scale")]
    names += ["model.layers.1.attn.wq.weight", "model.layers.1.ffn.experts.0.w1.weight"]
    saved = mod._ORIG_LOAD_WEIGHTS
    mod._ORIG_LOAD_WEIGHTS = stub_original
    try:
        mod._offload_load_weights(object(), ((n, torch.full((2, 2), i, dtype=torch.uint8))
                                             for i, n in enumerate(names)))
    finally:
        mod._ORIG_LOAD_WEIGHTS = saved
        eng._ENGINE = saved_engine
    assert received == [n for n in names if ".ffn.experts." not in n]
    assert sorted(engine._shared) == [1, 2] and sorted(engine._shared[1]) == ["w1", "w1s", "w2", "w2s", "w3", "w3s"]
    assert int(engine._shared[2]["w3s"][0, 0]) == names.index("model.layers.2.ffn.shared_experts.w3.scale")
    assert engine.get_shared(5, "cpu") is None      # nothing captured for layer 5


def test_recaptured_shared_tensor_drops_every_prepared_copy_of_its_layer():
    # get_shared caches per (layer, device); a re-captured tensor of layer 1 must drop
    # layer 1's prepared copies on every device and leave other layers' alone
    engine = ExpertOffloadEngine(slot_capacity=4, device="cpu")
    for l in (1, 2):
        for w in ("w1", "w2", "w3"):
            for k in ("weight", "scale"):
                engine.capture_shared(f"layers.{l}.ffn.shared_experts.{w}.{k}", torch.zeros(2, 2, dtype=torch.uint8))
    engine._shared_dev = {(1, "cuda:0"): "old", (1, "cuda:1"): "old", (2, "cuda:0"): "kept"}
    assert engine.capture_shared("layers.1.ffn.shared_experts.w2.weight", torch.ones(2, 2, dtype=torch.uint8))
    assert engine._shared_dev == {(2, "cuda:0"): "kept"}
    assert int(engine._shared[1]["w2"][0, 0]) == 1


def test_resident_table_needs_a_device_bank():
    # the router-in-layer path needs every expert on the device; a host bank never offers it
    bank = ExpertBank(capacity=4, device="cpu")
    assert bank.resident_table(0, 8) is None
