"""numpy restatement of the routed expert computation (test oracle only).

* ``routed_bf16``  - ``deepseek_v4.py:150-197`` (bf16 profile: FP8 round trip of
  x, grouped gate/up GEMM with bf16 outputs, clamp + SwiGLU x routing weight,
  FP8 round trip of h, grouped down GEMM, unweighted fp32 ``index_add_``).
* ``routed_a4w4``  - ``deepseek_v4.py:199-245`` (a4w4 profile: MXFP4
  activations x MXFP4 weights, same SwiGLU and combine). The closed
  ``npu_dynamic_mx_quant`` is replaced by ``mxfp4.dynamic_mx_quant(rule)``.
* ``baseline_loop_bf16`` - ``model_npu.py:492-533`` (``MoE.forward`` with the
  per-expert ``_expert`` loop), the reference's own parity baseline.
* ``grouped_gemm`` - ``npu_grouped_matmul(x=[x], weight=[w_g^T...],
  group_list_type=1)``: per-group ``x_g @ W_g^T`` (``_bench_gmm.py:8-22``).
* ``shared_expert_bf16`` - ``model_npu.py:469-489`` (the FP8 shared expert),
  and ``routed_plus_shared_bf16`` - ``deepseek_v4.py:262-264`` (routed output
  plus shared output, bf16 + bf16).

GEMM products are accumulated in float64 and rounded once to fp32 then bf16;
the reference accumulates in fp32 on the NPU, so GEMM outputs are compared
within a tolerance, never bit for bit.
"""

import numpy as np

from . import mxfp4 as Q
from .routing import moe_align, unpermute


def silu_f32(g):
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def swiglu(gate_f32, up_f32, w_f32, limit):
    """``deepseek_v4.py:184-187``: clamp(up, +-limit), clamp(gate, max=limit),
    silu(gate) * up * w, all in fp32."""
    gate = np.asarray(gate_f32, np.float32)
    up = np.asarray(up_f32, np.float32)
    if limit and limit > 0:
        up = np.clip(up, -limit, limit).astype(np.float32)
        gate = np.minimum(gate, np.float32(limit)).astype(np.float32)
    return (silu_f32(gate) * up * np.asarray(w_f32, np.float32)[:, None]).astype(np.float32)


def matmul_nt(a_f32, w_f32):
    """a [M,K] @ w[N,K]^T in float64, rounded to fp32."""
    return (np.asarray(a_f32, np.float64) @ np.asarray(w_f32, np.float64).T).astype(np.float32)


def grouped_gemm(x_f32, weights_f32, group_list):
    """Per-group ``x_g @ W_g^T`` over consecutive row groups; fp32 result.

    ``weights_f32[g]`` is ``[N, K]`` (the F.linear weight; the reference passes
    ``w.t()``). Empty groups contribute nothing."""
    x = np.asarray(x_f32, np.float32)
    N = weights_f32[0].shape[0] if len(weights_f32) else 0
    out = np.zeros((x.shape[0], N), np.float32)
    o = 0
    for w, c in zip(weights_f32, group_list):
        c = int(c)
        if c:
            out[o:o + c] = matmul_nt(x[o:o + c], w)
        o += c
    return out


def _expert_f32(experts, e):
    ex = experts[int(e)]
    return (Q.dequant_fp4_weight_f32(ex["w1p"], ex["w1s"]),
            Q.dequant_fp4_weight_f32(ex["w3p"], ex["w3s"]),
            Q.dequant_fp4_weight_f32(ex["w2p"], ex["w2s"]))


def _map(fn, items, workers):
    """``list(map(fn, items))``, on a thread pool when ``workers > 1`` (the
    per-expert numpy work releases the GIL; results do not depend on it)."""
    if workers <= 1 or len(items) <= 1:
        return [fn(i) for i in items]
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=workers) as ex:
        return list(ex.map(fn, items))


def routed_bf16(x_bf16, topk_ids, topk_w, experts, n_experts=256, swiglu_limit=10.0,
                fp8_act=True, workers=1):
    """bf16 profile of ``_routed``. Returns a dict of every intermediate.

    ``experts[e]`` holds the packed checkpoint tensors ``w{1,2,3}{p,s}``
    (``[N, K/2]`` uint8 + ``[N, K/32]`` UE8M0 bytes). ``workers`` runs the
    per-expert dequant and GEMMs on that many host threads (the reference's CPU
    path uses every core, ``ds4_npu_moe.py``); each expert's rows are computed
    the same way either way."""
    x_bf16 = np.asarray(x_bf16, np.uint16)
    T = x_bf16.shape[0]
    al = moe_align(topk_ids, topk_w, n_experts)
    xq = Q.act_quant(x_bf16, 128)[0] if fp8_act else x_bf16          # :170
    x_sorted = Q.bf16_bits_to_f32(xq[al["row"]])                     # :171
    R = x_sorted.shape[0]
    I = experts[int(al["active"][0])]["w1p"].shape[0] if R else 0
    D = x_bf16.shape[1]
    gate = np.zeros((R, I), np.float32)
    up = np.zeros((R, I), np.float32)
    starts = np.concatenate([[0], np.cumsum(al["group_list"])]).astype(np.int64)
    groups = [(int(e), int(starts[i]), int(starts[i + 1]))
              for i, e in enumerate(al["active"])]
    W = {}

    def gate_up(g):
        e, a, b = g
        W[e] = _expert_f32(experts, e)
        w1, w3, _ = W[e]
        gate[a:b] = Q.f32_to_bf16_f32(matmul_nt(x_sorted[a:b], w1))   # :177-179
        up[a:b] = Q.f32_to_bf16_f32(matmul_nt(x_sorted[a:b], w3))     # :180-182

    _map(gate_up, groups, workers)
    h = swiglu(gate, up, al["s_w"], swiglu_limit)                        # :184-187
    h_bf16 = Q.f32_to_bf16_bits(h)
    hq = Q.act_quant(h_bf16, 128)[0] if fp8_act else h_bf16             # :188
    hq_f = Q.bf16_bits_to_f32(hq)
    out = np.zeros((R, D), np.float32)

    def down(g):
        e, a, b = g
        out[a:b] = matmul_nt(hq_f[a:b], W[e][2])                        # :191-193

    _map(down, groups, workers)
    out_bf16 = Q.f32_to_bf16_bits(out)
    y = unpermute(out_bf16, al["row"], T)                                # :195-197
    return {"align": al, "xq": xq, "gate": gate, "up": up, "h": h, "h_bf16": h_bf16,
            "hq": hq, "out": out_bf16, "y": y}


def routed_a4w4(x_bf16, topk_ids, topk_w, experts, n_experts=256, swiglu_limit=10.0,
                rule="ocp_floor", workers=1):
    """a4w4 profile of ``_routed_mxfp4`` (``deepseek_v4.py:199-245``). ``workers``
    as in ``routed_bf16``."""
    x_bf16 = np.asarray(x_bf16, np.uint16)
    T, D = x_bf16.shape
    al = moe_align(topk_ids, topk_w, n_experts)
    _, xp, xs = Q.dynamic_mx_quant(x_bf16, rule)                         # :212
    xa = Q.fp4_codes_to_f32(xp, xs)[al["row"]]                           # :213-214
    R = xa.shape[0]
    I = experts[int(al["active"][0])]["w1p"].shape[0] if R else 0
    gate = np.zeros((R, I), np.float32)
    up = np.zeros((R, I), np.float32)
    starts = np.concatenate([[0], np.cumsum(al["group_list"])]).astype(np.int64)
    groups = [(int(e), int(starts[i]), int(starts[i + 1])) for i, e in enumerate(al["active"])]
    W = {}

    def gate_up(g):
        e, a, b = g
        W[e] = _expert_f32(experts, e)
        w1, w3, _ = W[e]
        gate[a:b] = Q.f32_to_bf16_f32(matmul_nt(xa[a:b], w1))           # :231
        up[a:b] = Q.f32_to_bf16_f32(matmul_nt(xa[a:b], w3))             # :232

    _map(gate_up, groups, workers)
    h = swiglu(gate, up, al["s_w"], swiglu_limit)                        # :234-237
    h_bf16 = Q.f32_to_bf16_bits(h)
    _, hp, hs = Q.dynamic_mx_quant(h_bf16, rule)                         # :240
    ha = Q.fp4_codes_to_f32(hp, hs)
    out = np.zeros((R, D), np.float32)

    def down(g):
        e, a, b = g
        out[a:b] = matmul_nt(ha[a:b], W[e][2])                           # :241

    _map(down, groups, workers)
    out_bf16 = Q.f32_to_bf16_bits(out)
    y = unpermute(out_bf16, al["row"], T)                                # :243-245
    return {"align": al, "xp": xp, "xs": xs, "gate": gate, "up": up, "h": h,
            "h_bf16": h_bf16, "hp": hp, "hs": hs, "out": out_bf16, "y": y}


def baseline_loop_bf16(x_bf16, topk_ids, topk_w, experts, n_experts=256, swiglu_limit=10.0):
    """``model_npu.MoE.forward`` (``:516-533``) with ``_expert`` (``:505-514``):
    for each expert in ascending id, the tokens that picked it (row-major
    ``torch.where`` order), FP8 round trip, gate/up/down, ``index_add_``."""
    x_bf16 = np.asarray(x_bf16, np.uint16)
    ids = np.asarray(topk_ids).astype(np.int64)
    w = np.asarray(topk_w, np.float32)
    T, D = x_bf16.shape
    y = np.zeros((T, D), np.float32)
    for i in range(n_experts):
        idx, top = np.nonzero(ids == i)
        if len(idx) == 0:
            continue
        w1, w3, w2 = _expert_f32(experts, i)
        xq = Q.bf16_bits_to_f32(Q.act_quant(x_bf16[idx], 128)[0])
        gate = Q.f32_to_bf16_f32(matmul_nt(xq, w1))
        up = Q.f32_to_bf16_f32(matmul_nt(xq, w3))
        h = swiglu(gate, up, w[idx, top], swiglu_limit)
        hq = Q.bf16_bits_to_f32(Q.act_quant(Q.f32_to_bf16_bits(h), 128)[0])
        val = Q.f32_to_bf16_f32(matmul_nt(hq, w2))
        np.add.at(y, idx, val)
    return Q.f32_to_bf16_bits(y)


def dequant_gemv(x_bf16, w_packed, scale):
    """Config-0 check: bf16 ``x @ dequant(W)^T`` -> bf16 bits."""
    wf = Q.dequant_fp4_weight_f32(w_packed, scale)
    return Q.f32_to_bf16_bits(matmul_nt(Q.bf16_bits_to_f32(x_bf16), wf))


def shared_expert_bf16(x_bf16, sh, swiglu_limit=10.0):
    """``model_npu.py:469-489`` Expert(mode="fp8"): every Linear takes the FP8
    round trip of its input (``:114-117``) and the weight dequantised to bf16
    (``npu_ops.py:161-167``); SwiGLU with the clamp and no routing weight.
    ``sh`` holds ``w{1,2,3}`` E4M3 codes and ``w{1,2,3}s`` 128x128 block
    scales. Returns bf16 bits [T, D]."""
    x_bf16 = np.asarray(x_bf16, np.uint16)
    w1 = Q.dequant_fp8_weight_f32(sh["w1"], sh["w1s"])
    w3 = Q.dequant_fp8_weight_f32(sh["w3"], sh["w3s"])
    w2 = Q.dequant_fp8_weight_f32(sh["w2"], sh["w2s"])
    xq = Q.bf16_bits_to_f32(Q.act_quant(x_bf16, 128)[0])                 # :115
    gate = Q.f32_to_bf16_f32(matmul_nt(xq, w1))                          # :479
    up = Q.f32_to_bf16_f32(matmul_nt(xq, w3))                            # :480
    h = swiglu(gate, up, np.ones(xq.shape[0], np.float32), swiglu_limit)  # :481-486 (x 1.0 is exact)
    hq = Q.bf16_bits_to_f32(Q.act_quant(Q.f32_to_bf16_bits(h), 128)[0])  # :489 -> :115
    return Q.f32_to_bf16_bits(matmul_nt(hq, w2))


def routed_plus_shared_bf16(x_bf16, topk_ids, topk_w, experts, sh, n_experts=256, swiglu_limit=10.0):
    """``deepseek_v4.py:262-264``: ``out = self._routed(hs) + self.shared_experts(hs)``,
    a bf16 + bf16 addition (rounded once, from the exact fp32 sum)."""
    yr = routed_bf16(x_bf16, topk_ids, topk_w, experts, n_experts=n_experts, swiglu_limit=swiglu_limit)["y"]
    ys = shared_expert_bf16(x_bf16, sh, swiglu_limit)
    return Q.f32_to_bf16_bits(Q.bf16_bits_to_f32(yr) + Q.bf16_bits_to_f32(ys)), yr, ys
