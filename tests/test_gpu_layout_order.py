"""GPU: a row's GEMM result does not depend on where it sits in its block.

The C ABI's grouped GEMMs take any ``sorted_ids`` layout in which every block
holds rows of one expert and padding marks (the flat-index count R) anywhere.
moe_align puts an expert's padding at the end of its last block, and the
tiled kernel skips the 16-row subtiles that hold only padding (their A loads
and MFMAs), so a layout whose padding sits first or in the middle of a block
exercises the per-subtile mask. Reversing, or rotating, the rows inside every
block must leave h and the down outputs unchanged bit for bit, for every
kernel: 16-row decode blocks, 64/128-row tiled blocks, 256-row large tiles,
in both profiles.
"""

import dataclasses

import numpy as np
import pytest
import torch

from oracle import mxfp4 as Q
from dsv4_hip import ops, synth, AFMT_E2M1, AFMT_E4M3

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _permuted(al, how):
    sid = al.sorted_ids.view(al.max_blocks, al.block_m)
    if how == "reverse":
        p = sid.flip(1)
    else:  # rotate by 24 rows: an expert's padding lands mid-block
        p = sid.roll(24 % al.block_m, dims=1)
    return dataclasses.replace(al, sorted_ids=p.contiguous().view(-1))


@pytest.mark.parametrize("profile", ["bf16", "a4w4"])
@pytest.mark.parametrize("T,K,E,D,I,bm", [(24, 4, 16, 1024, 512, 16), (300, 6, 24, 2048, 1024, 64),
                                          (200, 8, 16, 1024, 512, 128), (300, 6, 24, 2048, 1024, 256)])
def test_gemm_rows_independent_of_block_position(gpu, profile, T, K, E, D, I, bm):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(7 + T))
    w = synth.routing_weights(T, K, 8 + T)
    xb = synth.bf16_normal(np.random.default_rng(9 + T), (T, D)).view(torch.int16).numpy().view(np.uint16)
    devw = {int(e): {k: _dev(v, gpu) for k, v in synth.expert_weights(int(e), D, I).items()} for e in np.unique(ids)}
    table = ops.expert_table(devw, E, gpu)
    al = ops.moe_align(_dev(ids, gpu), _dev(w, gpu), E, bm)
    if profile == "bf16":
        _, codes, _, k = Q.act_quant(xb, 128)
        a, a_s, afmt = _dev(codes, gpu), _dev(np.repeat((k + 127).astype(np.uint8), 4, axis=-1), gpu), AFMT_E4M3
    else:
        _, packed, sc = Q.ocp_mx_quant(xb, 32)
        a, a_s, afmt = _dev(packed, gpu), _dev(sc, gpu), AFMT_E2M1
    wf = _dev(w.reshape(-1), gpu)
    h0 = ops.gemm_gateup(afmt, a, a_s, K, al, table, D, I, wf, 10.0)
    # the down GEMM's input: h quantised on the host (the same for every layout)
    torch.cuda.synchronize()
    hb = _bits(h0)
    if profile == "bf16":
        _, hc, _, hk = Q.act_quant(hb, 128)
        ha, has = _dev(hc, gpu), _dev(np.repeat((hk + 127).astype(np.uint8), 4, axis=-1), gpu)
    else:
        _, hp, hsc = Q.ocp_mx_quant(hb, 32)
        ha, has = _dev(hp, gpu), _dev(hsc, gpu)
    y0 = ops.gemm_down(afmt, ha, has, al, table, I, D)
    torch.cuda.synchronize()
    y0b = _bits(y0)
    assert np.isfinite(Q.bf16_bits_to_f32(y0b)).all()
    for how in ("reverse", "rotate"):
        alp = _permuted(al, how)
        h1 = ops.gemm_gateup(afmt, a, a_s, K, alp, table, D, I, wf, 10.0)
        y1 = ops.gemm_down(afmt, ha, has, alp, table, I, D)
        torch.cuda.synchronize()
        dh = int((_bits(h1) != hb).sum())
        dy = int((_bits(y1) != y0b).sum())
        print(f"{profile} bm={bm} {how}: h differs in {dh}, y in {dy} elements", flush=True)
        assert dh == 0 and dy == 0
