"""GPU: the routed layer at its full configured sizes, checked on sampled tokens.

A token's output depends only on its own row of x, its routed ids and weights:
x and h are quantised per row block, the GEMMs are per row, and the unpermute
sums each token's rows on their own. So a full-size launch can be checked
against the oracle run on a few of its tokens. Sizes: 256 experts, top-8,
hidden 4096, inter 2048, at
* 2048 tokens in both profiles: 16,384 routed rows, 64-row blocks, the chunked
  align, Zipf-hot experts spread over dozens of blocks;
* 16384 tokens in both profiles: 131,072 routed rows; experts with at least 256
  rows (the Zipf-hot ones, up to ~14,000 rows) run in 256-row blocks on the
  large-tile kernel, the others in 64-row blocks;
* 64 tokens in the a4w4 profile: 512 routed rows on the 16-row kernel;
* 2048 and 16384 tokens in the pure-bf16 variant (no FP8 round trips): bf16
  activations in 64-row blocks on the tiled kernel; at 16384 tokens (from
  65,536 routed rows) the hot experts on the large-tile bf16 kernel (32x32x16
  bf16 MFMAs).
Expert weights are random bytes generated on the device and stored MFMA-tiled,
as the slot cache stores them. The oracle reads checkpoint-layout copies of the
sampled tokens' experts. The sample at 2048 tokens: the tokens of the first and
last routed row of every M block of the 16 hottest experts (the block edges of
every hot expert; ~260 tokens) plus 32 random ones; at 16384 tokens the same for
the 8 hottest experts in their 256-row blocks; at 64 tokens, all of them.
Tolerances: max relative error (normwise) 1e-2 for bf16 and pure bf16, 2e-2 for
a4w4; per element, bf16 within 3e-2 and pure bf16 within 2e-2 of
max(|ref|, rms(ref)), a4w4 bit for bit."""

import numpy as np
import pytest
import torch

from dsv4_hip import ops, synth, PROFILE_A4W4, PROFILE_BF16, PROFILE_BF16_PURE, RULE_OCP_FLOOR
from oracle import moe as M
from oracle import mxfp4 as Q
from _parity import elementwise_rel

pytestmark = pytest.mark.gpu

E, K, D, I = 256, 8, 4096, 2048
TOL = {"bf16": 1e-2, "a4w4": 2e-2, "bf16_pure": 1e-2}
# per element, floor rms(ref) (_parity.elementwise_rel); a4w4 exact
ELEM_TOL = {"bf16": 3e-2, "a4w4": 0.0, "bf16_pure": 2e-2}


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


@pytest.mark.parametrize("profile,T", [("bf16", 2048), ("a4w4", 2048), ("a4w4", 64), ("bf16", 4096),
                                       ("a4w4", 4096), ("bf16", 16384), ("a4w4", 16384), ("bf16_pure", 2048),
                                       ("bf16_pure", 16384)])
def test_full_size_layer_on_sampled_tokens(gpu, profile, T):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(T))
    w = synth.routing_weights(T, K, T + 1)
    x = synth.bf16_normal(np.random.default_rng(T + 2), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    experts = _device_experts(gpu, T + 3)
    tiled = {e: {k: (ops.tile_weights(v) if k.endswith("p") else v) for k, v in d.items()} for e, d in experts.items()}
    table = ops.expert_table(tiled, E, gpu, tiled=True)
    runner = ops.LayerRunner(gpu, E, D, I)
    prof = {"bf16": PROFILE_BF16, "a4w4": PROFILE_A4W4, "bf16_pure": PROFILE_BF16_PURE}[profile]
    y = runner.forward(x.to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), table,
                       profile=prof, rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    got_all = Q.bf16_bits_to_f32(_bits(y))
    sample = _sample_tokens(ids, T, profile)
    print(f"full size {profile} T={T}: checking {sample.size} tokens", flush=True)
    host = {int(e): {k: v.cpu().numpy() for k, v in experts[int(e)].items()} for e in np.unique(ids[sample])}
    if profile == "bf16":
        ref = M.routed_bf16(xb[sample], ids[sample], w[sample], host, n_experts=E, workers=16)
    elif profile == "bf16_pure":
        ref = M.routed_bf16(xb[sample], ids[sample], w[sample], host, n_experts=E, workers=16, fp8_act=False)
    else:
        ref = M.routed_a4w4(xb[sample], ids[sample], w[sample], host, n_experts=E, rule="ocp_floor", workers=16)
    want = Q.bf16_bits_to_f32(ref["y"])
    got = got_all[sample]
    err = float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))
    er = elementwise_rel(got, want)
    print(f"full size {profile} T={T}: normwise rel {err:.3e}, elementwise rel {er:.3e}", flush=True)
    assert err <= TOL[profile], (profile, T, err)
    assert er <= ELEM_TOL[profile], (profile, T, er)
    if profile == "a4w4":      # every product and partial sum is exact in fp32: bit for bit
        assert np.array_equal(_bits(y)[sample], ref["y"])
    assert np.isfinite(got_all).all()
    del experts, tiled


def _sample_tokens(ids, T, profile, n_hot=16, n_random=32):
    """Tokens of the first and last routed row of every M block of the n_hot
    hottest experts (rows of an expert in flat-index order, blocks of the
    layer's block size: 64 rows from 2048 routed rows on, else 16), plus
    n_random random tokens; every token when T <= 64. The large-tile split
    (from 16,384 routed rows; only the 8 hottest experts are then taken)
    gives its experts blocks of the rows one workgroup takes: bf16, experts
    with at least 128 rows, 128 rows (half a hot block); pure bf16 (from
    65,536 routed rows), experts with at least 128 rows in whole 256-row
    blocks; a4w4, experts with at
    least 128 rows in 128-row halves below 32,768 routed rows, then at least
    256 rows (128 from 65,536) in whole 256-row blocks."""
    if T <= 64:
        return np.arange(T)
    R = ids.size
    flat = ids.reshape(-1)
    counts = np.bincount(flat, minlength=E)
    picks = set()
    fp8 = profile == "bf16"
    pure = profile == "bf16_pure"
    split = R >= (65536 if pure else 16384)  # the layer's large-tile split
    hot_min = 128 if (fp8 or pure or R < 32768 or R >= 65536) else 256
    if split:
        n_hot = 8
    for e in np.argsort(-counts, kind="stable")[:n_hot]:
        tok = np.nonzero(flat == e)[0] // ids.shape[1]
        big = 256 if pure else 128 if (fp8 or R < 32768) else 256
        bm = big if (split and tok.size >= hot_min) else (64 if R >= 2048 else 16)
        for b in range(0, tok.size, bm):
            picks.add(int(tok[b]))
            picks.add(int(tok[min(b + bm, tok.size) - 1]))
    picks.update(int(t) for t in np.random.default_rng(T + 7).choice(T, n_random, replace=False))
    return np.array(sorted(picks))
