"""GPU parity: MXFP4 dequant, FP8 act_quant round trip and MXFP4 activation quant,
all bit-exact against the oracle (NaN only arises from E8M0 byte 255 and is
emitted as 0x7FC0 by both); and the config-0 dequant + bf16 GEMV, within 1e-2."""

import numpy as np
import pytest
import torch

from oracle import moe as M_
from oracle import mxfp4 as Q
from dsv4_hip import ops, synth, RULE_CEIL_DIV6, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _bf16_dev(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(dev)


def _u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(dev)


def test_dequant_config0_bitexact(gpu):
    packed, scales, _ = synth.dequant_config0()
    out = ops.dequant_mxfp4(_u8(packed, gpu), _u8(scales, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), Q.dequant_fp4_weight(packed, scales))


def test_dequant_exhaustive_byte_scale_table(gpu):
    b = np.tile(np.arange(256, dtype=np.uint8), (256, 16))
    s = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)
    out = ops.dequant_mxfp4(_u8(b, gpu), _u8(s, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), Q.dequant_fp4_weight(b, s))


@pytest.mark.parametrize("n,k", [(1, 32), (3, 96), (4096, 2048), (257, 4096)])
def test_dequant_shapes_and_tails(gpu, n, k):
    rng = np.random.default_rng(n + k)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(0, 256, (n, k // 32), dtype=np.uint8)
    out = ops.dequant_mxfp4(_u8(packed, gpu).view(torch.int8), _u8(scales, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), Q.dequant_fp4_weight(packed, scales))


@pytest.mark.parametrize("tiled", [False, True])
def test_dequant_multi_one_launch_equals_each_tensor(gpu, tiled):
    # one launch for several tensors (an expert's w1, w2, w3 at the config-1 shapes,
    # plus odd shapes and an empty one), checkpoint or MFMA-tiled source layout: each
    # output bit for bit the oracle's dequant of that tensor
    rng = np.random.default_rng(21 + int(tiled))
    shapes = [(2048, 4096), (4096, 2048), (2048, 4096), (16, 256), (0, 512), (48, 1024)]
    if not tiled:
        shapes += [(3, 96), (1, 32)]
    host = [(rng.integers(0, 256, (n, k // 2), dtype=np.uint8), rng.integers(0, 256, (n, k // 32), dtype=np.uint8))
            for n, k in shapes]
    pairs = []
    for p_, s_ in host:
        pt = _u8(p_, gpu)
        if tiled and p_.size:
            pt = ops.tile_weights(pt)
        pairs.append((pt, _u8(s_, gpu)))
    outs = ops.dequant_mxfp4_multi(pairs, tiled=tiled)
    torch.cuda.synchronize()
    for (p_, s_), o in zip(host, outs):
        assert tuple(o.shape) == (p_.shape[0], 2 * p_.shape[1])
        assert np.array_equal(_bits(o), Q.dequant_fp4_weight(p_, s_)), p_.shape


def test_expert_bank_get_miss_is_one_dequant_launch(gpu, monkeypatch):
    # offload.py:77-84: the bf16 get of a missing expert (one record copy, one dequant
    # launch for w1, w2, w3 read from the MFMA-tiled record) equals the oracle bit for bit
    from offload import ExpertBank
    calls = []
    real = ops.dequant_mxfp4_multi
    monkeypatch.setattr(ops, "dequant_mxfp4_multi", lambda *a, **k: calls.append(1) or real(*a, **k))
    monkeypatch.setenv("DSV4_PACKED_SLOTS", "2")
    bank = ExpertBank(capacity=1, device="cuda:0")
    w = synth.expert_weights(3, 1024, 512)
    bank.register(0, 3, *(torch.from_numpy(w[k]) for k in ("w1p", "w1s", "w2p", "w2s", "w3p", "w3s")))
    assert bank._layout.tiled
    d = bank.get(0, 3)
    torch.cuda.synchronize()
    assert len(calls) == 1
    for nm in ("w1", "w2", "w3"):
        assert np.array_equal(_bits(d[nm]), Q.dequant_fp4_weight(w[nm + "p"], w[nm + "s"])), nm


def _all_finite_bf16_rows(cols):
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = Q.bf16_bits_to_f32(b)
    b = np.where(np.isfinite(v), b, 0).astype(np.uint16)
    return b.reshape(-1, cols)


def test_fp8_act_quant_all_bf16_patterns(gpu):
    for cols in (128, 4096):
        xb = _all_finite_bf16_rows(cols)
        rt, codes, s, k = Q.act_quant(xb, 128)
        x = _bf16_dev(xb, gpu)
        r = ops.fp8_act_quant(x, 128, rt=torch.empty_like(x), want_codes=True, want_scale=True, want_e8m0x4=True)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(r["rt"]), rt)
        assert np.array_equal(r["codes"].cpu().numpy(), codes)
        assert np.array_equal(r["scale"].cpu().numpy(), s)
        assert np.array_equal(r["e8m0x4"].cpu().numpy(), np.repeat((k + 127).astype(np.uint8), 4, axis=-1))


@pytest.mark.parametrize("scale", [1.0, 3.0, 1e-3, 1e-7, 1e4, 3e37])
def test_fp8_act_quant_random_and_inplace(gpu, scale):
    rng = np.random.default_rng(int(abs(np.log(scale))) + 1)
    xf = (rng.standard_normal((64, 512)) * scale).astype(np.float32)
    xb = Q.f32_to_bf16_bits(xf)
    rt = Q.act_quant(xb, 128)[0]
    x = _bf16_dev(xb, gpu)
    ops.fp8_act_quant(x, 128, rt=x)   # inplace: rt aliases x
    torch.cuda.synchronize()
    assert np.array_equal(_bits(x), rt)


@pytest.mark.parametrize("rule,name", [(RULE_CEIL_DIV6, "ceil_div6"), (RULE_OCP_FLOOR, "ocp_floor")])
def test_mxfp4_quant_all_bf16_patterns(gpu, rule, name):
    xb = _all_finite_bf16_rows(32)
    dq, packed, sc = Q.dynamic_mx_quant(xb, name)
    x = _bf16_dev(xb, gpu)
    p, s, d = ops.mxfp4_act_quant(x, rule, dq=torch.empty_like(x))
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), sc)
    assert np.array_equal(p.cpu().numpy(), packed)
    assert np.array_equal(_bits(d), dq)


@pytest.mark.parametrize("rule,name", [(RULE_CEIL_DIV6, "ceil_div6"), (RULE_OCP_FLOOR, "ocp_floor")])
@pytest.mark.parametrize("scale", [1.0, 1e-30, 1e30])
def test_mxfp4_quant_random(gpu, rule, name, scale):
    rng = np.random.default_rng(7)
    xf = (rng.standard_normal((130, 4096)) * scale).astype(np.float32)
    xf[5] = 0.0
    xf[6, :32] = -0.0
    xb = Q.f32_to_bf16_bits(xf)
    dq, packed, sc = Q.dynamic_mx_quant(xb, name)
    x = _bf16_dev(xb, gpu)
    p, s, d = ops.mxfp4_act_quant(x, rule, dq=torch.empty_like(x))
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), sc)
    assert np.array_equal(p.cpu().numpy(), packed)
    assert np.array_equal(_bits(d), dq)


def test_cpu_tensor_is_rejected(gpu):
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.dequant_mxfp4(torch.zeros(4, 16, dtype=torch.uint8), torch.zeros(4, 1, dtype=torch.uint8))


@pytest.mark.parametrize("M", [1, 3, 16])
def test_mxfp4_gemv_config0(gpu, M):
    # config 0: bf16 x @ dequant(W)^T against the oracle (fp64 sum of the exact
    # products, rounded once), tolerance 1e-2 max-relative
    packed, scales, x0 = synth.dequant_config0()
    x = x0 if M == 1 else synth.bf16_normal(np.random.default_rng(40 + M), (M, 4096))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    y = ops.mxfp4_gemv(x.to(gpu), _u8(packed, gpu), _u8(scales, gpu))
    torch.cuda.synchronize()
    got = Q.bf16_bits_to_f32(_bits(y))
    want = Q.bf16_bits_to_f32(M_.dequant_gemv(xb, packed, scales))
    assert got.shape == (M, 2048)
    assert np.abs(got - want).max() <= 1e-2 * np.abs(want).max()


def test_mxfp4_gemv_rejects_bad_shapes(gpu):
    with pytest.raises(ValueError):
        ops.mxfp4_gemv(torch.zeros(1, 64, dtype=torch.bfloat16, device=gpu),
                       torch.zeros(8, 16, dtype=torch.uint8, device=gpu), torch.zeros(8, 2, dtype=torch.uint8, device=gpu))
    with pytest.raises(ops._lib.Dsv4Error, match="at most 16"):
        ops.mxfp4_gemv(torch.zeros(17, 64, dtype=torch.bfloat16, device=gpu),
                       torch.zeros(8, 32, dtype=torch.uint8, device=gpu), torch.zeros(8, 2, dtype=torch.uint8, device=gpu))
