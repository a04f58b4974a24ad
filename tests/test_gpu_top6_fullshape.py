"""GPU: the plugin's routed layer at the reference model's own routing and
expert shape: top-6 of 256 experts, hidden 4096, inter 2048, 8 tokens
(model_npu.py:61; the parity case of test_moe_align.py:103,147-150).

The layer is driven through ``OffloadDeepseekV4MoE.forward`` with the router
on the device (sqrtsoftplus scores, renormalised, scaled by 1.5), once with a
score-correction bias and once as a hash layer (``tid2eid`` rows picked by the
input ids), in both profiles, on both of the plugin's paths: the one-call
routed layer over the resident pointer table and ``_route`` -> host ids ->
acquired slots -> layer. Only the experts the router picks are registered
(their 13.4 MB records pinned on the host, MFMA-tiled in the slots, as
``_offload_load_weights`` would store them). The oracle runs the reference
path on the same ids and weights: a4w4 bit for bit, bf16 profile within 1e-2
normwise and 3e-2 per element of max(|ref|, rms(ref)).
"""

import types

import numpy as np
import pytest
import torch
from torch import nn

import dsv4_plugin.models.deepseek_v4 as mod
from dsv4_plugin.core.engine import ExpertOffloadEngine
from dsv4_hip import synth
from oracle import moe as M
from oracle import mxfp4 as Q
from _parity import elementwise_rel

pytestmark = pytest.mark.gpu

E, K, D, I, T, LAYER = 256, 6, 4096, 2048, 8, 4


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _plugin(is_hash):
    m = mod.OffloadDeepseekV4MoE.__new__(mod.OffloadDeepseekV4MoE)
    nn.Module.__init__(m)
    m.hash, m.topk, m.renormalize, m.scoring_func = is_hash, K, True, "sqrtsoftplus"
    m.routed_scaling_factor, m.swiglu_limit, m.n_routed_experts = 1.5, 10.0, E
    m.is_sequence_parallel, m.shared_experts, m.layer_idx, m.engine = False, None, LAYER, None
    g = torch.Generator().manual_seed(17 + int(is_hash))
    m.gate = types.SimpleNamespace(
        weight=(torch.randn(E, D, generator=g) * 0.02).to("cuda:0"),
        e_score_correction_bias=None if is_hash else (torch.randn(E, generator=g) * 0.01).to("cuda:0"),
        tid2eid=(torch.argsort(torch.rand(1000, E, generator=g), dim=1)[:, :K].to(torch.int32).to("cuda:0")
                 if is_hash else None))    # K distinct experts per token id
    return m


@pytest.mark.parametrize("is_hash", [False, True])
def test_top6_full_shape_layer_both_profiles(gpu, monkeypatch, is_hash):
    m = _plugin(is_hash)
    x = synth.bf16_normal(np.random.default_rng(31), (T, D)).to(gpu)
    input_ids = torch.randint(0, 1000, (T,), generator=torch.Generator().manual_seed(5)).to(gpu)
    w, idx = m._route(x, input_ids)
    ids = idx.cpu().numpy().astype(np.int64)
    wt = w.cpu().numpy().astype(np.float32)
    uniq = np.unique(ids)
    print(f"top-6 full shape hash={is_hash}: {uniq.size} experts routed", flush=True)
    assert ids.shape == (T, K) and uniq.size > K
    monkeypatch.setenv("DSV4_PACKED_SLOTS", "64")
    eng = ExpertOffloadEngine(slot_capacity=4, device="cuda:0")
    host = {int(e): synth.expert_weights(int(e), D, I) for e in uniq}
    for e, hw in host.items():
        for nm in ("w1", "w2", "w3"):
            eng.capture(f"layers.{LAYER}.ffn.experts.{e}.{nm}.weight", torch.from_numpy(hw[nm + "p"]).view(torch.int8))
            eng.capture(f"layers.{LAYER}.ffn.experts.{e}.{nm}.scale",
                        torch.from_numpy(hw[nm + "s"]).view(torch.float8_e8m0fnu))
    m.engine = eng
    xb = _bits(x)
    refs = {"bf16": M.routed_bf16(xb, ids, wt, host, n_experts=E)["y"],
            "a4w4": M.routed_a4w4(xb, ids, wt, host, n_experts=E, rule="ocp_floor")["y"]}
    for profile in ("bf16", "a4w4"):
        monkeypatch.setattr(mod, "_MXFP4_GMM", profile == "a4w4")
        for fused in (True, False):
            monkeypatch.setattr(mod, "_FUSED_ROUTE", fused)
            print(f"top-6 layer hash={is_hash} profile={profile} one_call={fused}", flush=True)
            y = m.forward(x, input_ids)
            torch.cuda.synchronize()
            got = Q.bf16_bits_to_f32(_bits(y))
            want = Q.bf16_bits_to_f32(refs[profile])
            if profile == "a4w4":
                assert np.array_equal(_bits(y), refs[profile])
            else:
                nw = float(np.abs(got - want).max() / np.abs(want).max())
                er = elementwise_rel(got, want)
                print(f"  normwise {nw:.3e} elementwise {er:.3e}")
                assert nw <= 1e-2 and er <= 3e-2
    s = eng.stats()
    assert s["packed_misses"] == uniq.size and s["packed_cached"] == uniq.size   # each record copied once
