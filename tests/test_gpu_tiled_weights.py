"""MFMA-tiled weight layout (``dsv4_mxfp4_tile_weights``) and the grouped GEMMs
reading it.

The layout is pure data movement, so the bar is bit equality: the kernel
against a numpy statement of the layout, the inverse round trip, and the routed
layer on tiled weights against the same layer on the checkpoint layout (the
MFMAs receive the same operand bytes either way), for the 16-row decode kernel
and the 64-row prefill kernel, both profiles, and with the shared expert's
(untiled) E4M3 weights in the same launches."""

import numpy as np
import pytest
import torch

from dsv4_hip import ops, synth, PROFILE_A4W4, PROFILE_BF16, RULE_OCP_FLOOR, Dsv4Error


def tile_np(w):
    """tiled[nt][j][ji][g][r][e] = w[16 nt + r][128 j + 32 g + 16 ji + e]."""
    N, KH = w.shape
    nst = KH // 128
    return np.ascontiguousarray(w.reshape(N // 16, 16, nst, 4, 2, 16).transpose(0, 2, 4, 3, 1, 5)).reshape(N, KH)


def test_tile_np_matches_the_index_formula():
    rng = np.random.default_rng(0)
    N, K = 32, 512
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    t = tile_np(w).reshape(-1)
    nst = K // 256
    for nt in range(N // 16):
        for j in range(nst):
            for ji in range(2):
                for g in range(4):
                    for r in range(16):
                        off = ((nt * nst + j) * 2 + ji) * 1024 + (r + 16 * g) * 16
                        src = w[16 * nt + r, 128 * j + 32 * g + 16 * ji: 128 * j + 32 * g + 16 * ji + 16]
                        assert np.array_equal(t[off:off + 16], src)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(16, 256), (2048, 4096), (4096, 2048), (48, 768)])
def test_tile_weights_matches_numpy_and_round_trips(gpu, N, K):
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    wd = torch.from_numpy(w).to(gpu)
    t = ops.tile_weights(wd)
    back = ops.tile_weights(t, inverse=True)
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), tile_np(w))
    assert np.array_equal(back.cpu().numpy(), w)


@pytest.mark.gpu
def test_tile_weights_rejects_bad_shapes(gpu):
    with pytest.raises(Dsv4Error, match="rows % 16"):
        ops.tile_weights(torch.zeros(24, 128, dtype=torch.uint8, device=gpu))
    with pytest.raises(Dsv4Error, match="K % 256"):
        ops.tile_weights(torch.zeros(16, 64, dtype=torch.uint8, device=gpu))
    from dsv4_hip import _lib
    buf = torch.zeros(16, 256, dtype=torch.uint8, device=gpu)
    rc = _lib.lib().dsv4_mxfp4_tile_weights(buf.data_ptr(), buf.data_ptr() + 16, 16, 256, 0, None)
    assert rc != 0 and b"overlap" in _lib.lib().dsv4_last_error()


def _tiled_copy(devw):
    return {e: {k: (ops.tile_weights(v) if k.endswith("p") else v) for k, v in d.items()} for e, d in devw.items()}


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy()


# (T, K, E, D, I): decode at full size (16-row kernel), small, 2048 and 2400 routed rows (64-row kernel)
LAYERS = [(8, 8, 256, 4096, 2048), (5, 4, 32, 1024, 512), (256, 8, 32, 1024, 512), (300, 8, 64, 2048, 1024)]


@pytest.mark.gpu
@pytest.mark.parametrize("profile", [PROFILE_BF16, PROFILE_A4W4])
@pytest.mark.parametrize("T,K,E,D,I", LAYERS)
def test_layer_on_tiled_weights_equals_checkpoint_layout(gpu, profile, T, K, E, D, I):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(T + E))
    w = synth.routing_weights(T, K, 17)
    x = synth.bf16_normal(np.random.default_rng(T), (T, D)).to(gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(T + D)
    devw = {}
    for e in np.unique(ids):
        devw[int(e)] = {}
        for name, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
            devw[int(e)][name + "p"] = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=gpu, generator=g)
            devw[int(e)][name + "s"] = torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=gpu, generator=g)
    tiled = _tiled_copy(devw)
    runner = ops.LayerRunner(gpu, E, D, I)
    ids_d, w_d = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
    y_nat = runner.forward(x, ids_d, w_d, ops.expert_table(devw, E, gpu), profile=profile,
                           rule=RULE_OCP_FLOOR).clone()
    y_til = runner.forward(x, ids_d, w_d, ops.expert_table(tiled, E, gpu, tiled=True), profile=profile,
                           rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y_til), _bits(y_nat))
    del devw, tiled


@pytest.mark.gpu
@pytest.mark.parametrize("profile", [PROFILE_BF16, PROFILE_A4W4])
@pytest.mark.parametrize("T", [8, 300])
def test_mixed_layouts_in_one_launch(gpu, profile, T):
    # the 16-row kernel picks its weight loads per block from the table tag:
    # tiled and checkpoint-layout experts side by side in one table
    E, K, D, I = 32, 8, 1024, 512
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 5), np.random.default_rng(T + 9))
    w = synth.routing_weights(T, K, 19)
    x = synth.bf16_normal(np.random.default_rng(T + 2), (T, D)).to(gpu)
    devw = {int(e): {k: torch.from_numpy(v).to(gpu) for k, v in synth.expert_weights(int(e), D, I).items()}
            for e in np.unique(ids)}
    tiled = _tiled_copy(devw)
    runner = ops.LayerRunner(gpu, E, D, I)
    ids_d, w_d = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
    tab_nat = ops.expert_table(devw, E, gpu)
    tab_til = ops.expert_table(tiled, E, gpu, tiled=True)
    mixed = torch.where((torch.arange(E, device=gpu) % 2 == 0)[:, None], tab_til, tab_nat)
    y_nat = runner.forward(x, ids_d, w_d, tab_nat, profile=profile, rule=RULE_OCP_FLOOR).clone()
    y_mix = runner.forward(x, ids_d, w_d, mixed, profile=profile, rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y_mix), _bits(y_nat))
    del devw, tiled


@pytest.mark.gpu
@pytest.mark.parametrize("T", [8, 300])
def test_tiled_routed_weights_with_the_shared_expert(gpu, T):
    E, K, D, I = 32, 8, 1024, 512
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(T))
    w = synth.routing_weights(T, K, 18)
    x = synth.bf16_normal(np.random.default_rng(T + 1), (T, D)).to(gpu)
    devw = {int(e): {k: torch.from_numpy(v).to(gpu) for k, v in synth.expert_weights(int(e), D, I).items()}
            for e in np.unique(ids)}
    tiled = _tiled_copy(devw)
    sh = {k: torch.from_numpy(v).to(gpu) for k, v in synth.shared_expert_weights(5, D, I).items()}
    prep = ops.prepare_shared_expert(sh["w1"], sh["w1s"], sh["w3"], sh["w3s"], sh["w2"], sh["w2s"])
    runner = ops.LayerRunner(gpu, E, D, I)
    ids_d, w_d = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
    y_nat = runner.forward(x, ids_d, w_d, ops.expert_table(devw, E, gpu), shared=prep).clone()
    y_til = runner.forward(x, ids_d, w_d, ops.expert_table(tiled, E, gpu, tiled=True), shared=prep)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y_til), _bits(y_nat))
    del devw, tiled


def test_host_tiler_matches_numpy():
    # the host tiler writes pinned records before their first copy to the device
    import ctypes
    from dsv4_hip import _lib
    from dsv4_hip.slots import tile_host
    rng = np.random.default_rng(3)
    for N, K in ((16, 256), (64, 1024), (48, 512)):
        w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
        out = np.zeros_like(w)
        rc = _lib.lib().dsv4_mxfp4_tile_host(w.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p), N, K)
        assert rc == 0
        assert np.array_equal(out, tile_np(w)) and np.array_equal(tile_host(w), tile_np(w))
    bad = np.zeros((24, 128), np.uint8)
    assert _lib.lib().dsv4_mxfp4_tile_host(bad.ctypes.data_as(ctypes.c_void_p), bad.ctypes.data_as(ctypes.c_void_p),
                                           24, 256) != 0


@pytest.mark.gpu
def test_bank_stores_tiled_records_and_serves_checkpoint_views(gpu, monkeypatch):
    from offload import ExpertBank
    monkeypatch.setenv("DSV4_PACKED_SLOTS", "16")
    E, D, I, T, K, layer = 16, 1024, 512, 8, 4, 2
    bank = ExpertBank(capacity=2, device="cuda:0")
    host = {e: synth.expert_weights(100 + e, D, I) for e in range(E)}
    for e in range(E):
        h = host[e]
        bank.register(layer, e, *[torch.from_numpy(h[k]) for k in ("w1p", "w1s", "w2p", "w2s", "w3p", "w3s")])
    assert bank._layout.tiled
    p = bank.get_packed(layer, 3)                                   # checkpoint layout for the caller
    assert np.array_equal(p["w1p"].cpu().numpy().view(np.uint8), host[3]["w1p"])
    assert np.array_equal(p["w2p"].cpu().numpy().view(np.uint8), host[3]["w2p"])
    bf = bank.get(layer, 5)                                         # bf16 dequant of an untiled copy
    from oracle import mxfp4 as Q
    assert np.array_equal(_bits(bf["w3"]).view(np.uint16), Q.dequant_fp4_weight(host[5]["w3p"], host[5]["w3s"]))
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(1))
    w = synth.routing_weights(T, K, 2)
    x = synth.bf16_normal(np.random.default_rng(3), (T, D)).to(gpu)
    table, _ = bank.acquire_table(layer, ids.reshape(-1), E)
    devw = {e: {k: torch.from_numpy(v).to(gpu) for k, v in host[e].items()} for e in range(E)}
    runner = ops.LayerRunner(gpu, E, D, I)
    ids_d, w_d = torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu)
    y_bank = runner.forward(x, ids_d, w_d, table).clone()
    y_nat = runner.forward(x, ids_d, w_d, ops.expert_table(devw, E, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y_bank), _bits(y_nat))
    del devw
