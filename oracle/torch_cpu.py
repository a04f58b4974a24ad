"""torch CPU restatement of the reference's routed-expert path: the CPU baseline.

Test and measurement infrastructure only (the CPU-baseline leg of the bench and
the CPU tests import it); nothing in the product path does. It runs the
reference's torch arithmetic on the host cores, the way its CPU path would:

* ``act_quant`` FP8 E4M3 round trip, per 128       - ``npu_ops.py:73-104``
* ``dequant_fp4_weight`` (table lookup, E8M0 scale) - ``npu_ops.py:129-158``
* ``_routed`` bf16 profile                         - ``deepseek_v4.py:150-197``:
  stable sort of the flat expert ids, gather, per-group ``torch.matmul`` in fp32
  on the bf16-valued operands (standing in for ``npu_grouped_matmul``; bf16
  outputs), clamp + SwiGLU x routing weight, FP8 round trip of h, down GEMM,
  unweighted fp32 ``index_add_``
* a4w4 profile, simulated (the reference has no CPU kernel for it:
  ``deepseek_v4.py:199-245``): OCP MX quantise -> dequantise -> fp32 matmul

Inputs follow ``oracle.moe``: x as bf16 bit patterns (uint16), ids/weights as
numpy arrays, experts as dicts of packed checkpoint tensors. Per-group products
are summed in fp32 by torch's BLAS (the numpy oracle sums in float64), so the
outputs agree with the oracle within the GEMM tolerance, not bit for bit.
"""

import numpy as np
import torch

_FP4 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=torch.float32)
_TBL256 = torch.stack([_FP4[torch.arange(256) & 15], _FP4[torch.arange(256) >> 4]], dim=-1)  # [256, 2]
_E2M1_POS = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=torch.float64)


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16)


def _pow2_ceil(v):
    """2**ceil(log2 v) for positive fp32 v (exact, via frexp)."""
    m, e = torch.frexp(v)
    return torch.ldexp(torch.ones_like(v), torch.where(m == 0.5, e - 1, e))


def act_quant_rt(x):
    """Per-128 FP8 round trip of a bf16 [R, C] tensor (``npu_ops.py:73-104``)."""
    R, C = x.shape
    xf = x.float().view(R, C // 128, 128)
    amax = xf.abs().amax(-1, keepdim=True).clamp(min=1e-4)
    s = _pow2_ceil(torch.clamp(amax * torch.tensor(1.0 / 448.0, dtype=torch.float32), min=2.0 ** -126))
    y = (xf / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).float() * s
    return y.view(R, C).to(torch.bfloat16)


def dequant(w_packed, scale):
    """[N, K/2] packed + [N, K/32] E8M0 -> bf16 [N, K] (``npu_ops.py:129-158``)."""
    p = torch.from_numpy(np.ascontiguousarray(w_packed).view(np.uint8)).long()
    s = torch.from_numpy(np.ascontiguousarray(scale).view(np.uint8)).to(torch.int32)
    N, K2 = p.shape
    vals = _TBL256[p].view(N, K2 * 2 // 32, 32)
    sc = torch.ldexp(torch.ones(1), (s - 127).to(torch.float32)).unsqueeze(-1)
    return (vals * sc).view(N, 2 * K2).to(torch.bfloat16)


def mx_quant_rt(x):
    """OCP MX v1.0 MXFP4 round trip of a bf16 [R, C] tensor per 32 elements
    (shared exponent floor(log2 amax) - 2, saturate to 6, nearest even)."""
    R, C = x.shape
    xf = x.double().view(R, C // 32, 32)
    amax = xf.abs().amax(-1, keepdim=True)
    _, e = torch.frexp(amax)
    shared = torch.where(amax == 0, torch.full_like(e, -127), torch.clamp(e - 3, -127, 127))
    X = torch.ldexp(torch.ones_like(amax), shared.double())
    a = torch.clamp(xf.abs() / X, max=6.0)
    _, ea = torch.frexp(a)
    E = torch.where(a < 1.0, torch.zeros_like(ea), ea - 1)
    q = torch.round(torch.ldexp(a, (1 - E).double())) * torch.ldexp(torch.ones_like(a), (E - 1).double())
    return (torch.sign(xf) * q * X).float().view(R, C).to(torch.bfloat16)


def _routed(x_bits, topk_ids, topk_w, experts, quant, swiglu_limit):
    x = _bf16(x_bits)
    T, D = x.shape
    ids = torch.from_numpy(np.asarray(topk_ids, np.int64))
    K = ids.shape[1]
    flat_e = ids.reshape(-1)
    flat_w = torch.from_numpy(np.asarray(topk_w, np.float32)).reshape(-1)
    order = torch.argsort(flat_e, stable=True)                          # :155-158
    s_e, s_w, row = flat_e[order], flat_w[order], order // K
    counts = torch.bincount(flat_e, minlength=int(flat_e.max()) + 1 if flat_e.numel() else 1)
    xq = quant(x)                                                       # :170 / :212
    xs = xq[row].float()                                                # :171 / :213
    y = torch.zeros(T, D, dtype=torch.float32)
    o = 0
    hs, ws = [], []
    for e in torch.nonzero(counts).flatten().tolist():
        c = int(counts[e])
        ex = experts[int(e)]
        w1 = dequant(ex["w1p"], ex["w1s"]).float()
        w3 = dequant(ex["w3p"], ex["w3s"]).float()
        w2 = dequant(ex["w2p"], ex["w2s"]).float()
        xa = xs[o:o + c]
        gate = torch.matmul(xa, w1.t()).to(torch.bfloat16).float()      # :177-179
        up = torch.matmul(xa, w3.t()).to(torch.bfloat16).float()        # :180-182
        if swiglu_limit and swiglu_limit > 0:
            up = up.clamp(-swiglu_limit, swiglu_limit)
            gate = gate.clamp(max=swiglu_limit)
        h = (torch.nn.functional.silu(gate) * up * s_w[o:o + c, None]).to(torch.bfloat16)   # :184-187
        hs.append(h)
        ws.append(w2)
        o += c
    o = 0
    outs = []
    for h, w2 in zip(hs, ws):
        hq = quant(h).float()                                           # :188 / :240
        outs.append(torch.matmul(hq, w2.t()).to(torch.bfloat16))        # :191-193 / :241
        o += h.shape[0]
    out = torch.cat(outs) if outs else torch.zeros(0, D, dtype=torch.bfloat16)
    y.index_add_(0, row, out.float())                                   # :195-197
    return y.to(torch.bfloat16)


def routed_bf16(x_bits, topk_ids, topk_w, experts, swiglu_limit=10.0):
    """bf16 profile of ``_routed``; bf16 [T, D] tensor."""
    return _routed(x_bits, topk_ids, topk_w, experts, act_quant_rt, swiglu_limit)


def routed_a4w4(x_bits, topk_ids, topk_w, experts, swiglu_limit=10.0):
    """a4w4 profile (OCP MX scales), simulated with fp32 matmuls; bf16 [T, D] tensor."""
    return _routed(x_bits, topk_ids, topk_w, experts, mx_quant_rt, swiglu_limit)
