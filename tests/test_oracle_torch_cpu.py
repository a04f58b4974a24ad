"""CPU: the torch restatement the bench times as its CPU baseline agrees with
the numpy oracle - its quantisers and dequant bit for bit, its routed layers
within the GEMM tolerance (torch sums in fp32, the oracle in float64)."""

import numpy as np
import torch

from oracle import moe as M
from oracle import mxfp4 as Q
from oracle import torch_cpu as TC
from dsv4_hip import synth


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_quantisers_and_dequant_bit_exact():
    rng = np.random.default_rng(3)
    x = synth.bf16_normal(rng, (16, 512))
    x[3] *= 1e-3
    x[5, :128] = 0.0
    xb = _bits(x)
    assert np.array_equal(_bits(TC.act_quant_rt(x)), Q.act_quant(xb, 128)[0])
    assert np.array_equal(_bits(TC.mx_quant_rt(x)), Q.ocp_mx_quant(xb, 32)[0])
    p = rng.integers(0, 256, (64, 256), dtype=np.uint8)
    s = rng.integers(100, 150, (64, 16), dtype=np.uint8)
    assert np.array_equal(_bits(TC.dequant(p, s)), Q.dequant_fp4_weight(p, s))


def test_routed_layers_match_the_oracle():
    T, K, E, D, I = 24, 6, 16, 512, 256
    x, ids, w = synth.layer_inputs(T, K, E, D)
    xb = _bits(x)
    ex = {int(e): synth.expert_weights(int(e), D, I) for e in np.unique(ids)}
    for fn_t, fn_o, tol in ((TC.routed_bf16, M.routed_bf16, 1e-2),
                            (TC.routed_a4w4, lambda *a, **k: M.routed_a4w4(*a, rule="ocp_floor", **k), 2e-2)):
        got = fn_t(xb, ids, w, ex).float().numpy()
        want = Q.bf16_bits_to_f32(fn_o(xb, ids, w, ex, n_experts=E)["y"])
        assert float(np.abs(got - want).max() / np.abs(want).max()) <= tol
