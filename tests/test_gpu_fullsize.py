"""GPU: the routed layer at its full configured sizes, checked on sampled tokens.

A token's output depends only on its own row of x, its routed ids and weights:
x and h are quantised per row block, the GEMMs are per row, and the unpermute
sums each token's rows on their own. So a full-size launch can be checked
against the oracle run on a few of its tokens. Sizes: 256 experts, top-8,
hidden 4096, inter 2048, at
* 2048 tokens in both profiles: 16,384 routed rows, 64-row blocks, the chunked
  align, Zipf-hot experts spread over dozens of blocks;
* 64 tokens in the a4w4 profile: 512 routed rows on the 16-row kernel.
Expert weights are random bytes generated on the device and stored MFMA-tiled,
as the slot cache stores them. The oracle reads checkpoint-layout copies of the
sampled tokens' experts. Tolerances (max relative error): 1e-2 for bf16, 2e-2
for a4w4."""

import numpy as np
import pytest
import torch

from dsv4_hip import ops, synth, PROFILE_A4W4, PROFILE_BF16, RULE_OCP_FLOOR
from oracle import moe as M
from oracle import mxfp4 as Q

pytestmark = pytest.mark.gpu

E, K, D, I = 256, 8, 4096, 2048
TOL = {"bf16": 1e-2, "a4w4": 2e-2}


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _device_experts(dev, seed):
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


@pytest.mark.parametrize("profile,T", [("bf16", 2048), ("a4w4", 2048), ("a4w4", 64)])
def test_full_size_layer_on_sampled_tokens(gpu, profile, T):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(T))
    w = synth.routing_weights(T, K, T + 1)
    x = synth.bf16_normal(np.random.default_rng(T + 2), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    experts = _device_experts(gpu, T + 3)
    tiled = {e: {k: (ops.tile_weights(v) if k.endswith("p") else v) for k, v in d.items()} for e, d in experts.items()}
    table = ops.expert_table(tiled, E, gpu, tiled=True)
    runner = ops.LayerRunner(gpu, E, D, I)
    prof = PROFILE_BF16 if profile == "bf16" else PROFILE_A4W4
    y = runner.forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), table,
                       profile=prof, rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    got_all = Q.bf16_bits_to_f32(_bits(y))
    # the token routed to the hottest expert's last row block, plus the ends and the middle
    hot = np.bincount(ids.reshape(-1), minlength=E).argmax()
    last_hot = int(np.nonzero((ids == hot).any(axis=1))[0][-1])
    sample = np.array(sorted({0, T // 2, T - 1, last_hot}))
    host = {int(e): {k: v.cpu().numpy() for k, v in experts[int(e)].items()} for e in np.unique(ids[sample])}
    if profile == "bf16":
        ref = M.routed_bf16(xb[sample], ids[sample], w[sample], host, n_experts=E)
    else:
        ref = M.routed_a4w4(xb[sample], ids[sample], w[sample], host, n_experts=E, rule="ocp_floor")
    want = Q.bf16_bits_to_f32(ref["y"])
    got = got_all[sample]
    err = float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))
    assert err <= TOL[profile], (profile, T, err)
    assert np.isfinite(got_all).all()
    del experts, tiled
