"""GPU parity: the shared expert folded into the routed layer's grouped GEMMs
(``dsv4_moe_layer_forward_shared``) against the oracle's
``routed_plus_shared_bf16`` (``deepseek_v4.py:262-264`` with the FP8 shared
expert of ``model_npu.py:469-489``), tolerance 1e-2 max-relative as for the
bf16 profile; the block-scale expansion is compared bit for bit."""

import numpy as np
import pytest
import torch

from oracle import moe as M
from oracle import mxfp4 as Q
from dsv4_hip import ops, synth

pytestmark = pytest.mark.gpu

TOL = 1e-2


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _layer(E, D, I, needed, dev):
    host = {int(e): synth.expert_weights(int(e), D, I) for e in needed}
    devw = {e: {k: torch.from_numpy(v).to(dev) for k, v in d.items()} for e, d in host.items()}
    return host, devw, ops.expert_table(devw, E, dev)


def _shared(D, I, seed, dev):
    sh = synth.shared_expert_weights(seed, D, I)
    d = {k: torch.from_numpy(v).to(dev) for k, v in sh.items()}
    prep = ops.prepare_shared_expert(d["w1"], d["w1s"], d["w3"], d["w3s"], d["w2"], d["w2s"])
    return sh, prep


@pytest.mark.parametrize("n,k", [(300, 416), (4096, 2048), (2048, 4096), (128, 32)])
def test_expand_block_scales_bit_exact(gpu, n, k):
    rng = np.random.default_rng(n + k)
    blk = rng.integers(0, 256, size=((n + 127) // 128, (k + 127) // 128), dtype=np.uint8)
    got = ops.expand_block_scales(torch.from_numpy(blk).to(gpu), n, k)
    torch.cuda.synchronize()
    want = np.repeat(np.repeat(blk, 128, 0)[:n], 4, 1)[:, :k // 32]
    assert np.array_equal(got.cpu().numpy(), want)


# (T, K, E, D, I): decode at full size, small shapes, 2048 routed rows (64-row
# blocks, tiled kernel, h quantised in its epilogue), one token, 2400 routed
# rows (chunked align with the shared group)
CASES = [(8, 8, 256, 4096, 2048), (24, 4, 16, 1024, 512), (256, 8, 16, 1024, 512),
         (300, 6, 24, 2048, 1024), (1, 8, 64, 1024, 512), (300, 8, 64, 1024, 512)]


@pytest.mark.parametrize("T,K,E,D,I", CASES)
def test_layer_with_shared_expert_vs_oracle(gpu, T, K, E, D, I):
    seed = 400 + T
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(seed))
    w = synth.routing_weights(T, K, seed + 1)
    x = synth.bf16_normal(np.random.default_rng(seed + 2), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    host, devw, table = _layer(E, D, I, np.unique(ids), gpu)
    sh, prep = _shared(D, I, seed + 3, gpu)
    runner = ops.LayerRunner(gpu, E, D, I)
    y = runner.forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), table,
                       shared=prep)
    # the shared expert alone: zero routing weights make every routed row zero
    y0 = runner.forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.zeros(T, K, device=gpu), table,
                        shared=prep)
    # the routed-only layer through the same runner (workspace reused at another size)
    yr = runner.forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), table)
    torch.cuda.synchronize()
    want, want_r, want_s = M.routed_plus_shared_bf16(xb, ids, w, host, sh, n_experts=E)
    f = Q.bf16_bits_to_f32
    assert rel(f(_bits(y0)), f(want_s)) <= TOL, rel(f(_bits(y0)), f(want_s))
    assert rel(f(_bits(yr)), f(want_r)) <= TOL
    assert rel(f(_bits(y)), f(want)) <= TOL, rel(f(_bits(y)), f(want))
    # y is the bf16 sum of the two parts the kernels produced
    both = (torch.from_numpy(_bits(yr).view(np.int16)).view(torch.bfloat16)
            + torch.from_numpy(_bits(y0).view(np.int16)).view(torch.bfloat16))
    assert np.array_equal(_bits(y), both.view(torch.int16).numpy().view(np.uint16))


def test_layer_with_shared_rejects_a4w4_and_bad_scales(gpu):
    E, D, I = 16, 512, 512
    sh = synth.shared_expert_weights(1, D, I)
    d = {k: torch.from_numpy(v).to(gpu) for k, v in sh.items()}
    with pytest.raises(ValueError, match="do not tile"):
        ops.expand_block_scales(d["w1s"][:, :2], I, D)
    prep = ops.prepare_shared_expert(d["w1"], d["w1s"], d["w3"], d["w3s"], d["w2"], d["w2s"])
    runner = ops.LayerRunner(gpu, E, D, I)
    x = torch.zeros(2, D, dtype=torch.bfloat16, device=gpu)
    ids = torch.zeros(2, 2, dtype=torch.int64, device=gpu)
    with pytest.raises(ValueError, match="bf16 profile"):
        runner.forward(x, ids, torch.ones(2, 2, device=gpu), torch.zeros(E, 6, dtype=torch.int64, device=gpu),
                       profile=ops._lib.PROFILE_A4W4, shared=prep)
