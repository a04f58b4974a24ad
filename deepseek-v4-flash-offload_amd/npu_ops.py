"""MoE expert-path operators of ``npu_ops`` on MI355X (HIP kernels, gfx950).

Same names, signatures and results as the reference module for the expert
path (``npu_ops.py:16-158``): ``FP4_TABLE``, ``FP4_POS``, ``FP8_MAX``,
``FP4_MAX``, ``e8m0_to_fp32``, ``act_quant``, ``fp4_act_quant`` and
``dequant_fp4_weight``, all bit-exact with the reference's torch math. New
entry points for the operations the reference runs inline or in closed
``torch_npu`` ops: ``dynamic_mx_quant`` (``npu_dynamic_mx_quant`` call sites),
``moe_align`` / ``moe_permute`` / ``moe_unpermute`` (the sort/gather/combine of
``deepseek_v4.py:155-197``) and ``grouped_matmul`` (``npu_grouped_matmul``).

Tensors must be on a ROCm device: there is no CPU implementation.
"""

import torch

from dsv4_hip import ops as _ops
from dsv4_hip import _lib

FP4_TABLE = torch.tensor(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=torch.float32,
)
FP4_POS = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=torch.float32)
FP8_MAX = 448.0
FP4_MAX = 6.0

SCALE_RULES = {"ceil_div6": _lib.RULE_CEIL_DIV6, "ocp_floor": _lib.RULE_OCP_FLOOR}


def e8m0_to_fp32(scale: torch.Tensor) -> torch.Tensor:
    """UE8M0 scale -> float32 = 2 ** (byte - 127) (byte 0 -> 2^-127, 255 -> inf).

    Built from exponent bits on the device, which is exact (the reference
    evaluates ``torch.pow``); integer-exponent tensors use ``2 ** (s - 127)``."""
    _ops._dev(scale, "e8m0_to_fp32")
    if scale.dtype == getattr(torch, "float8_e8m0fnu", None) or scale.dtype == torch.uint8:
        u = scale.view(torch.uint8).to(torch.int32)
        bits = torch.where(u == 0, torch.full_like(u, 0x00400000), u << 23)
        return bits.view(torch.float32)
    return torch.pow(2.0, scale.float() - 127.0)


def act_quant(x: torch.Tensor, block_size: int = 128, scale_fmt: str = "ue8m0",
              scale_dtype=None, inplace: bool = False):
    """Block-wise FP8 (E4M3) quantisation with power-of-two scales (``npu_ops.py:73-104``).

    ``inplace=True`` writes the quantise-dequantise round trip into ``x`` and
    returns ``x``; otherwise returns ``(y float8_e4m3fn, scale fp32 [..., N/128])``.
    ``scale_dtype`` is accepted and ignored, as in the reference."""
    N = x.shape[-1]
    assert N % block_size == 0, (N, block_size)
    if scale_fmt is None:
        raise NotImplementedError("act_quant: only power-of-two (ue8m0) scales are implemented")
    _ops._dev(x, "act_quant")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"act_quant: bf16 activations required, got {x.dtype}")
    src = x.contiguous()
    if inplace:
        _ops.fp8_act_quant(src, block_size, rt=src)
        if src is not x:
            x.copy_(src)
        return x
    r = _ops.fp8_act_quant(src, block_size, want_codes=True, want_scale=True)
    return r["codes"].view(torch.float8_e4m3fn), r["scale"]


def fp4_act_quant(x: torch.Tensor, block_size: int = 32, inplace: bool = False):
    """Block-wise FP4 quantisation, scale 2^ceil(log2(amax/6)) (``npu_ops.py:107-121``)."""
    N = x.shape[-1]
    assert N % block_size == 0, (N, block_size)
    if block_size != 32:
        raise NotImplementedError("fp4_act_quant: block_size 32 only")
    if not inplace:
        raise NotImplementedError("non-inplace fp4 pack not needed on this path")
    _ops._dev(x, "fp4_act_quant")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"fp4_act_quant: bf16 activations required, got {x.dtype}")
    src = x.contiguous()
    _ops.mxfp4_act_quant(src, _lib.RULE_CEIL_DIV6, dq=src)
    if src is not x:
        x.copy_(src)
    return x


def dequant_fp4_weight(w_packed: torch.Tensor, scale: torch.Tensor, out_dtype=torch.bfloat16) -> torch.Tensor:
    """[N, K/2] packed E2M1 + [N, K/32] UE8M0 -> [N, K] (``npu_ops.py:142-158``)."""
    out = _ops.dequant_mxfp4(w_packed, scale)
    return out if out_dtype == torch.bfloat16 else out.to(out_dtype)


# ---------------------------------------------------------------------------
# new entry points of the expert path
# ---------------------------------------------------------------------------
def dynamic_mx_quant(x: torch.Tensor, scale_rule: str = "ocp_floor", dst_type=None):
    """MXFP4 activation quantisation in place of ``torch_npu.npu_dynamic_mx_quant``
    (``deepseek_v4.py:212, 240``): returns ``(packed uint8 [..., K/2], scale uint8
    [..., K/32])``. ``scale_rule`` picks ``"ocp_floor"`` (2^(floor(log2 amax)-2))
    or ``"ceil_div6"`` (the reference's own ``fp4_act_quant`` rule)."""
    if scale_rule not in SCALE_RULES:
        raise ValueError(f"unknown scale_rule {scale_rule!r}")
    packed, scale, _ = _ops.mxfp4_act_quant(x.contiguous(), SCALE_RULES[scale_rule])
    return packed, scale


def moe_align(topk_ids: torch.Tensor, topk_weights, n_experts: int, block_m: int = 16):
    """Stable sort of the routed entries by expert plus the padded block layout.

    The result carries the reference's views (``order``, ``s_e``, ``s_w``,
    ``row``, ``counts``, ``active``/``num_active``) of ``deepseek_v4.py:155-164``
    with the stable order, and ``sorted_ids``/``block_expert``/
    ``num_post_padded`` for the grouped GEMM."""
    return _ops.moe_align(topk_ids, topk_weights, n_experts, block_m)


def moe_permute(x: torch.Tensor, row: torch.Tensor) -> torch.Tensor:
    """``x[row]`` (``deepseek_v4.py:171``)."""
    return _ops.moe_permute(x, row)


def moe_unpermute(out: torch.Tensor, row: torch.Tensor, num_tokens: int) -> torch.Tensor:
    """``zeros(T, D, fp32).index_add_(0, row, out.float()).bf16()`` (``deepseek_v4.py:195-197``)."""
    return _ops.moe_unpermute(out, row, num_tokens)


def grouped_matmul(x, weight, group_list, scale=None, per_token_scale=None, group_list_type=1,
                   output_dtype=torch.bfloat16, fp8_roundtrip=False, **unused):
    """Grouped ``x_g @ W_g^T`` over consecutive row groups, for MXFP4 weights.

    Keyword form of ``npu_grouped_matmul`` (``deepseek_v4.py:177-193,224-229``):
    ``x=[x]``, ``weight=[...]`` per-group packed ``[N, K/2]`` (or the
    reference's stacked ``[g, K/2, N]`` transposed view), ``scale=[...]`` their
    ``[N, K/32]`` E8M0, ``group_list`` per-group row counts
    (``group_list_type=1``). Output bf16 ``[M, N]``. Activations:

    * packed E2M1 ``[M, K/2]`` with ``per_token_scale=[[M, K/32]]`` (a4w4,
      ``deepseek_v4.py:224-229``);
    * bf16 ``[M, K]`` with ``fp8_roundtrip=True``: x is first replaced by its
      per-128 FP8 round trip (``act_quant(x, 128, "ue8m0", None, True)``), as
      the bf16 profile does before each of its grouped GEMMs
      (``deepseek_v4.py:170,188``), and the product runs on the FP8 x FP4 MFMA;
    * bf16 ``[M, K]`` as it is (the default): ``x @ bf16(dequant(W))^T`` with
      fp32 accumulation on the bf16 MFMA - the product
      ``npu_grouped_matmul(x=[bf16], weight=[bf16 w.t()])`` computes on the
      bf16-dequantised weights (``deepseek_v4.py:174-182``), no quantisation of
      x."""
    if group_list_type != 1:
        raise NotImplementedError("grouped_matmul: group_list_type=1 (counts) only")
    if output_dtype != torch.bfloat16:
        raise NotImplementedError("grouped_matmul: bf16 output only")
    xs = x[0] if isinstance(x, (list, tuple)) else x
    ws = list(weight)
    ss = list(scale) if scale is not None else None
    if len(ws) == 1 and ws[0].dim() == 3:
        # stacked [g, K/2, N] transposed view of [g, N, K/2]; scales [g, K/64, N, 2] of [g, N, K/64, 2]
        ws = [w.transpose(0, 1) for w in ws[0]]
        if ss is not None and len(ss) == 1 and ss[0].dim() == 4:
            ss = [s.transpose(0, 1).reshape(s.shape[1], -1) for s in ss[0]]
    if ss is None or len(ss) != len(ws):
        raise ValueError("grouped_matmul: one E8M0 scale tensor per packed weight is required")
    counts = [int(c) for c in (group_list.tolist() if torch.is_tensor(group_list) else group_list)]
    if len(counts) != len(ws):
        raise ValueError("grouped_matmul: group_list length must match the number of weights")
    dev = xs.device
    M = sum(counts)
    N, K2 = ws[0].shape
    K = 2 * K2
    # one "token" per row, routed to its group: the grouped GEMM of the layer
    # with K=1 picks, no SwiGLU (down-projection kernel)
    ids = torch.repeat_interleave(torch.arange(len(ws), device=dev), torch.tensor(counts, device=dev))
    ids = ids.to(torch.int32).view(M, 1)
    table = _ops.expert_table({g: {"w1p": w, "w1s": s, "w2p": w, "w2s": s, "w3p": w, "w3s": s}
                               for g, (w, s) in enumerate(zip(ws, ss)) if counts[g]},
                              len(ws), dev)
    # the layer's block rule: 16-row blocks (single-wave kernel) below 2048 rows,
    # 64-row blocks (LDS-tiled kernel, weight fragments reused over 4 row tiles) above
    al = _ops.moe_align(ids, None, len(ws), 64 if M >= 2048 else _lib.GEMM_BLOCK_M)
    if per_token_scale is not None:
        xa = xs.view(torch.uint8).contiguous()
        xsc = per_token_scale[0] if isinstance(per_token_scale, (list, tuple)) else per_token_scale
        xsc = xsc.reshape(M, K // 32).view(torch.uint8).contiguous()
        afmt = _lib.AFMT_E2M1
    else:
        if xs.dtype != torch.bfloat16:
            raise NotImplementedError(
                "grouped_matmul: activations must be packed E2M1 with per_token_scale, or bf16 "
                f"(x dtype {xs.dtype})")
        if fp8_roundtrip:
            q = _ops.fp8_act_quant(xs.contiguous(), 128, want_codes=True, want_e8m0x4=True)
            xa, xsc, afmt = q["codes"], q["e8m0x4"], _lib.AFMT_E4M3
        else:  # bf16 x bf16-dequantised weights on the bf16 MFMA
            xa, xsc, afmt = xs.contiguous(), None, _lib.AFMT_BF16
    return _ops.gemm_down(afmt, xa, xsc, al, table, K, N)
