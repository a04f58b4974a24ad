"""torch-facing wrappers of the HIP kernels.

Tensors must live on a ROCm device; outputs are allocated with torch on the
input's device and every kernel is enqueued on torch's current stream for that
device. There is no CPU implementation: a CPU tensor raises.
"""

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import call, stream_handle

_E8M0 = getattr(torch, "float8_e8m0fnu", None)


def _dev(t: torch.Tensor, what: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the HIP MoE path needs a ROCm device tensor (got {t.device}); "
                           "there is no CPU implementation")
    return t


def _u8(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.uint8 and t.is_contiguous():
        return t
    if t.dtype in (torch.uint8, torch.int8) or (_E8M0 is not None and t.dtype == _E8M0):
        return t.contiguous().view(torch.uint8)
    raise TypeError(f"expected a byte tensor (uint8/int8/e8m0), got {t.dtype}")


def _p(t: Optional[torch.Tensor]):
    # the bound entry points declare pointer arguments c_void_p, which takes the int as is
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor):
    return stream_handle(t.device)


# ---------------------------------------------------------------------------
# dequant / quant
# ---------------------------------------------------------------------------
def dequant_mxfp4(w_packed: torch.Tensor, scale: torch.Tensor, out: Optional[torch.Tensor] = None):
    """[N, K/2] packed + [N, K/32] E8M0 -> bf16 [N, K] (bit-exact)."""
    _dev(w_packed, "dequant_mxfp4")
    wp, sc = _u8(w_packed), _u8(scale)
    if wp.dim() != 2 or sc.dim() != 2:
        raise ValueError("dequant_mxfp4 expects 2-D packed and scale tensors")
    N, K2 = wp.shape
    K = 2 * K2
    if sc.shape != (N, K // 32):
        raise ValueError(f"scale shape {tuple(sc.shape)} does not match packed {tuple(wp.shape)}")
    if out is None:
        out = torch.empty((N, K), dtype=torch.bfloat16, device=wp.device)
    call("dsv4_mxfp4_dequant_bf16", _p(wp), _p(sc), _p(out), N, K, _stream(wp))
    return out


def dequant_mxfp4_multi(pairs, tiled: bool = False):
    """Several ``(packed [N, K/2], scale [N, K/32])`` pairs -> a list of bf16 ``[N, K]``
    tensors in ONE launch (bit-exact, as ``dequant_mxfp4``): an expert's w1, w2, w3.
    ``tiled``: the packed bytes are in the MFMA-tiled layout (``tile_weights``), as
    the slot records store them; the outputs are the checkpoint layout either way."""
    pairs = list(pairs)
    n = len(pairs)
    if not 1 <= n <= 8:
        raise ValueError(f"dequant_mxfp4_multi: {n} tensors (1..8)")
    wps, scs, outs = [], [], []
    for w_packed, scale in pairs:
        _dev(w_packed, "dequant_mxfp4_multi")
        wp, sc = _u8(w_packed), _u8(scale)
        if wp.dim() != 2 or sc.shape != (wp.shape[0], wp.shape[1] // 16):
            raise ValueError(f"scale shape {tuple(sc.shape)} does not match packed {tuple(wp.shape)}")
        wps.append(wp)
        scs.append(sc)
        outs.append(torch.empty((wp.shape[0], 2 * wp.shape[1]), dtype=torch.bfloat16, device=wp.device))
    arr = ctypes.c_void_p * n
    i64 = ctypes.c_int64 * n
    tag = _lib.TILED_WEIGHTS if tiled else 0
    call("dsv4_mxfp4_dequant_bf16_multi", n, arr(*[t.data_ptr() | tag for t in wps]), arr(*[t.data_ptr() for t in scs]),
         arr(*[t.data_ptr() for t in outs]), i64(*[t.shape[0] for t in wps]), i64(*[2 * t.shape[1] for t in wps]),
         _stream(wps[0]))
    return outs


def mxfp4_gemv(x: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``bf16(x @ dequant(W)^T)`` for up to 16 bf16 rows of x, fp32 accumulation."""
    _dev(x, "mxfp4_gemv")
    x = x.to(torch.bfloat16).contiguous()
    wp, sc = _u8(w_packed), _u8(scale)
    M, K = x.shape
    N = wp.shape[0]
    if wp.shape[1] * 2 != K or sc.shape != (N, K // 32):
        raise ValueError(f"mxfp4_gemv: weight {tuple(wp.shape)} / scales {tuple(sc.shape)} do not match K={K}")
    y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    call("dsv4_mxfp4_gemv_bf16", _p(x), M, _p(wp), _p(sc), N, K, _p(y), _stream(x))
    return y


def fp8_act_quant(x: torch.Tensor, block_size: int = 128, rt: Optional[torch.Tensor] = None,
                  want_codes: bool = False, want_scale: bool = False, want_e8m0x4: bool = False):
    """Per-128 FP8 E4M3 quantisation of a bf16 tensor (last dim blocked).

    Returns a dict with the requested outputs: ``rt`` (bf16 round trip, may be
    ``x`` itself for the inplace form), ``codes`` (uint8), ``scale`` (fp32 per
    block) and ``e8m0x4`` (uint8 per 32 elements)."""
    _dev(x, "fp8_act_quant")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"fp8_act_quant: bf16 input required, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError("fp8_act_quant: input must be contiguous")
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    res = {}
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device) if want_codes else None
    scale = torch.empty((*x.shape[:-1], cols // block_size), dtype=torch.float32,
                        device=x.device) if want_scale else None
    e8 = torch.empty((*x.shape[:-1], cols // 32), dtype=torch.uint8, device=x.device) if want_e8m0x4 else None
    call("dsv4_fp8_act_quant", _p(x), rows, cols, block_size, _p(rt), _p(codes), _p(scale), _p(e8), _stream(x))
    if rt is not None:
        res["rt"] = rt
    if codes is not None:
        res["codes"] = codes
    if scale is not None:
        res["scale"] = scale
    if e8 is not None:
        res["e8m0x4"] = e8
    return res


def mxfp4_act_quant(x: torch.Tensor, rule: int, dq: Optional[torch.Tensor] = None, want_packed: bool = True):
    """Per-32 MXFP4 quantisation. Returns (packed uint8 [.., K/2], scale uint8 [.., K/32], dq)."""
    _dev(x, "mxfp4_act_quant")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"mxfp4_act_quant: bf16 input required, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError("mxfp4_act_quant: input must be contiguous")
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    packed = torch.empty((*x.shape[:-1], cols // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty((*x.shape[:-1], cols // 32), dtype=torch.uint8, device=x.device)
    call("dsv4_mxfp4_act_quant", _p(x), rows, cols, int(rule), _p(packed), _p(scale), _p(dq), _stream(x))
    return packed, scale, dq


# ---------------------------------------------------------------------------
# routing layout
# ---------------------------------------------------------------------------
@dataclass
class AlignResult:
    """Device tensors of one moe_align call (all int32 unless noted)."""
    T: int
    K: int
    E: int
    block_m: int
    max_blocks: int
    sorted_ids: torch.Tensor
    block_expert: torch.Tensor
    num_post_padded: torch.Tensor
    order: torch.Tensor
    s_e: torch.Tensor
    s_w: torch.Tensor          # fp32
    row: torch.Tensor
    counts: torch.Tensor
    expert_start: torch.Tensor
    active: torch.Tensor       # [E], ascending active ids then -1
    num_active: torch.Tensor
    padded_pos: torch.Tensor
    status: torch.Tensor

    def check(self):
        """Host-synchronising check of the kernel's status word."""
        s = int(self.status.item())
        if s & (1 << 30):
            raise RuntimeError("moe_align: max_blocks too small")
        if s:
            raise ValueError(f"moe_align: {s} expert id(s) outside [0, {self.E})")

    def active_list(self) -> torch.Tensor:
        """``active`` trimmed to its length (host sync)."""
        return self.active[: int(self.num_active.item())]


def route(x: torch.Tensor, gate_w: torch.Tensor, topk: int, scoring: str = "sqrtsoftplus",
          bias: Optional[torch.Tensor] = None, renormalize: bool = True, scale: float = 1.5,
          tid2eid: Optional[torch.Tensor] = None, input_ids: Optional[torch.Tensor] = None,
          status: Optional[torch.Tensor] = None):
    """Router of ``deepseek_v4.py:118-148`` on the device: ``(weights fp32 [T, K],
    ids int32 [T, K])``. ``x`` [T, D] bf16 or fp32 (other dtypes are cast to fp32,
    as ``hs.float()`` does), ``gate_w`` [E, D] fp32;
    ``bias`` [E] fp32 or None; ``tid2eid`` [vocab, K] int32/int64 with
    ``input_ids`` [T] on hash layers. ``status`` (int32 [1], optional) is
    incremented once per out-of-range input id or table entry."""
    _dev(x, "route")
    if scoring not in _lib.SCORING:
        raise ValueError(f"route: unknown scoring function {scoring!r}")
    x = x.reshape(-1, x.shape[-1])
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    T, D = x.shape
    w = gate_w.to(torch.float32).contiguous()
    if w.dim() != 2 or w.shape[1] != D:
        raise ValueError(f"route: gate weight {tuple(w.shape)} does not match hidden size {D}")
    E = w.shape[0]
    b = None if bias is None else bias.to(torch.float32).contiguous()
    tab, ids_in, vocab = None, None, 0
    if tid2eid is not None:
        if input_ids is None:
            raise RuntimeError("hash-layer routing needs input_ids")
        tab = tid2eid.contiguous()
        if tab.dtype not in (torch.int32, torch.int64) or tab.dim() != 2 or tab.shape[1] != topk:
            raise ValueError("route: tid2eid must be int32/int64 [vocab, topk]")
        ids_in = input_ids.reshape(-1).contiguous()
        if ids_in.dtype not in (torch.int32, torch.int64):
            ids_in = ids_in.to(torch.int64)
        if ids_in.numel() != T:
            raise ValueError(f"route: {ids_in.numel()} input ids for {T} tokens")
        vocab = tab.shape[0]
    dev = x.device
    out_w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    out_ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    ws = torch.empty(max(int(_lib.lib().dsv4_moe_route_workspace_bytes(T, D, E)), 4), dtype=torch.uint8,
                     device=dev)
    call("dsv4_moe_route", _p(x), 1 if x.dtype == torch.float32 else 0, _p(w), _p(b), _p(tab), 1 if tab is not None and tab.dtype == torch.int64 else 0,
         vocab, _p(ids_in), 1 if ids_in is not None and ids_in.dtype == torch.int64 else 0, T, D, E, topk,
         _lib.SCORING[scoring], 1 if renormalize else 0, float(scale), _p(out_w), _p(out_ids), _p(status), _p(ws),
         _stream(x))
    return out_w, out_ids


def max_blocks(R: int, E: int, block_m: int) -> int:
    return int(_lib.lib().dsv4_moe_align_max_blocks(R, E, block_m))


def moe_align(topk_ids: torch.Tensor, topk_w: Optional[torch.Tensor], n_experts: int,
              block_m: int = _lib.GEMM_BLOCK_M) -> AlignResult:
    _dev(topk_ids, "moe_align")
    if topk_ids.dim() != 2:
        raise ValueError("moe_align expects topk_ids of shape [T, K]")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"moe_align: int32/int64 ids required, got {topk_ids.dtype}")
    ids = topk_ids.contiguous()
    T, K = ids.shape
    R = T * K
    dev = ids.device
    w = None
    if topk_w is not None:
        w = topk_w.to(torch.float32).contiguous()
        if w.shape != ids.shape:
            raise ValueError("moe_align: topk_w shape must match topk_ids")
    mb = max_blocks(R, n_experts, block_m)
    i32 = dict(dtype=torch.int32, device=dev)
    res = AlignResult(
        T=T, K=K, E=n_experts, block_m=block_m, max_blocks=mb,
        sorted_ids=torch.empty(mb * block_m, **i32), block_expert=torch.empty(mb, **i32),
        num_post_padded=torch.empty(1, **i32), order=torch.empty(R, **i32), s_e=torch.empty(R, **i32),
        s_w=torch.empty(R, dtype=torch.float32, device=dev), row=torch.empty(R, **i32),
        counts=torch.empty(n_experts, **i32), expert_start=torch.empty(n_experts, **i32),
        active=torch.empty(n_experts, **i32), num_active=torch.empty(1, **i32),
        padded_pos=torch.empty(R, **i32), status=torch.empty(1, **i32))
    nws = int(_lib.lib().dsv4_moe_align_workspace_bytes(T, K, n_experts))
    ws = torch.empty(max(nws, 4), dtype=torch.uint8, device=dev)
    call("dsv4_moe_align_ws", _p(ids), 1 if ids.dtype == torch.int64 else 0, _p(w), T, K, n_experts, block_m, mb,
         _p(res.sorted_ids), _p(res.block_expert), _p(res.num_post_padded), _p(res.order), _p(res.s_e),
         _p(res.s_w if w is not None else None), _p(res.row), _p(res.counts), _p(res.expert_start),
         _p(res.active), _p(res.num_active), _p(res.padded_pos), _p(res.status), _p(ws), ws.numel(), _stream(ids))
    if w is None:
        res.s_w.zero_()
    return res


def moe_permute(x: torch.Tensor, row: torch.Tensor) -> torch.Tensor:
    """``x[row]`` for row-major x whose rows are a multiple of 16 bytes."""
    _dev(x, "moe_permute")
    x = x.contiguous()
    row = row.to(torch.int32).contiguous()
    n = row.numel()
    out = torch.empty((n, *x.shape[1:]), dtype=x.dtype, device=x.device)
    row_bytes = x[0].numel() * x.element_size() if x.shape[0] else 0
    call("dsv4_moe_permute", _p(x), x.shape[0], _p(row), n, row_bytes, _p(out), _stream(x))
    return out


def moe_unpermute(out_sorted: torch.Tensor, row: torch.Tensor, T: int, kmax: Optional[int] = None,
                  check: bool = True):
    """``zeros(T, D).index_add_(0, row, out.float()).bf16()`` (bit-exact).

    A token may receive up to ``kmax`` rows (default: R, capped at
    ``UNPERMUTE_MAX_ROWS`` = 64). With ``check`` (default) the call reads back
    the kernel's count of dropped rows (a host sync) and raises where
    ``index_add_`` would not have dropped them: ``IndexError`` for a row whose
    token is outside [0, T), ``ValueError`` for a token with more than ``kmax``
    rows."""
    _dev(out_sorted, "moe_unpermute")
    if out_sorted.dtype != torch.bfloat16:
        raise TypeError("moe_unpermute: bf16 rows required")
    out_sorted = out_sorted.contiguous()
    row = row.to(torch.int32).contiguous()
    R, D = out_sorted.shape
    if row.numel() != R:
        raise ValueError(f"moe_unpermute: {row.numel()} row indices for {R} rows")
    if kmax is None:
        kmax = max(1, min(R, _lib.UNPERMUTE_MAX_ROWS))
    ws = torch.empty(int(_lib.lib().dsv4_moe_unpermute_workspace_bytes(T, kmax)), dtype=torch.uint8,
                     device=out_sorted.device)
    y = torch.empty((T, D), dtype=torch.bfloat16, device=out_sorted.device)
    status = torch.zeros(1, dtype=torch.int32, device=out_sorted.device)
    call("dsv4_moe_unpermute", _p(out_sorted), _p(row), R, T, kmax, D, _p(ws), _p(y), _p(status), _stream(out_sorted))
    if check and T > 0 and R > 0:
        dropped = int(status.item())
        if dropped:
            if bool(((row < 0) | (row >= T)).any()):
                raise IndexError(f"moe_unpermute: row index outside [0, {T})")
            raise ValueError(f"moe_unpermute: {dropped} row(s) beyond {kmax} rows per token were dropped")
    return y


def moe_combine(out_flat: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
    """Sum each token's K rows (row t*K+k) in ascending expert order -> bf16 [T, D]."""
    _dev(out_flat, "moe_combine")
    ids = topk_ids.contiguous()
    T, K = ids.shape
    D = out_flat.shape[-1]
    y = torch.empty((T, D), dtype=torch.bfloat16, device=out_flat.device)
    call("dsv4_moe_combine", _p(out_flat.contiguous()), _p(ids), 1 if ids.dtype == torch.int64 else 0, T, K, D,
         _p(y), _stream(out_flat))
    return y


# ---------------------------------------------------------------------------
# expert table + GEMMs + fused layer
# ---------------------------------------------------------------------------
_KEYS = ("w1p", "w1s", "w2p", "w2s", "w3p", "w3s")


def tile_weights(w_packed: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """Packed E2M1 weights [N, K/2] to the MFMA-tiled layout the grouped GEMMs
    stream fastest (``dsv4_mxfp4_tile_weights``), or back with ``inverse``:
    ``tiled[nt][j][ji][g][r][e] = w[16 nt + r][128 j + 32 g + 16 ji + e]``.
    Returns a new uint8 tensor of the same shape; N % 16 == 0, K % 256 == 0."""
    _dev(w_packed, "tile_weights")
    w = _u8(w_packed.contiguous())
    if w.dim() != 2:
        raise ValueError("tile_weights: [N, K/2] packed weights required")
    N, K = w.shape[0], w.shape[1] * 2
    out = torch.empty_like(w)
    call("dsv4_mxfp4_tile_weights", _p(w), _p(out), N, K, 1 if inverse else 0, _stream(w))
    return out


def expert_table(experts, n_experts: int, device, tiled: bool = False) -> torch.Tensor:
    """Device table [E, 6] (uint64 as int64) of the packed weight pointers.

    ``experts`` maps expert id -> dict with keys ``w{1,2,3}{p,s}`` (device
    tensors, contiguous, any byte dtype). Missing experts get null entries.
    ``tiled``: the packed fields hold the MFMA-tiled layout (``tile_weights``);
    their pointers carry the table's layout tag (bit 0). The returned tensor
    holds references to the weight tensors, so they live as long as the table
    (a table of raw pointers into freed tensors would read whatever the
    allocator put there next)."""
    tab = torch.zeros((n_experts, 6), dtype=torch.int64)
    refs = []
    items = experts.items() if hasattr(experts, "items") else enumerate(experts)
    for e, d in items:
        if d is None:
            continue
        for j, k in enumerate(_KEYS):
            t = d[k]
            _dev(t, "expert_table")
            if not t.is_contiguous():
                raise ValueError(f"expert {e} {k}: weights must be contiguous")
            if t.data_ptr() % 16:
                raise ValueError(f"expert {e} {k}: weights must be 16-byte aligned")
            tab[int(e), j] = t.data_ptr() | (_lib.TILED_WEIGHTS if tiled and k.endswith("p") else 0)
            refs.append(t)
    out = tab.to(device)
    out._dsv4_weights = refs
    return out


def gemm_gateup(afmt, a, a_scale, a_row_div, al: AlignResult, table, D, I, topk_w_flat, swiglu_limit, out=None):
    """h [R, I] bf16 by flat index (rows of ids the align skipped are left as they were in ``out``)."""
    R = al.T * al.K
    h = out if out is not None else torch.empty((R, I), dtype=torch.bfloat16, device=a.device)
    call("dsv4_moe_gemm_gateup", afmt, _p(a), _p(a_scale), a_row_div, _p(al.sorted_ids), _p(al.block_expert),
         _p(al.num_post_padded), R, al.block_m, al.max_blocks, _p(table), D, I, _p(topk_w_flat),
         float(swiglu_limit or 0.0), _p(h), _stream(a))
    return h


def gemm_down(afmt, a, a_scale, al: AlignResult, table, I, D, out=None):
    """[R, D] bf16 by flat index (rows of ids the align skipped are left as they were in ``out``)."""
    R = al.T * al.K
    if out is None:
        out = torch.empty((R, D), dtype=torch.bfloat16, device=a.device)
    call("dsv4_moe_gemm_down", afmt, _p(a), _p(a_scale), _p(al.sorted_ids), _p(al.block_expert),
         _p(al.num_post_padded), R, al.block_m, al.max_blocks, _p(table), I, D, _p(out), _stream(a))
    return out


def expand_block_scales(block_scales: torch.Tensor, n_rows: int, k: int) -> torch.Tensor:
    """128x128-block E8M0 scales [ceil(n/128), ceil(k/128)] -> per-32 layout [n, k/32]."""
    b = _u8(_dev(block_scales, "expand_block_scales"))
    if b.shape != ((n_rows + 127) // 128, (k + 127) // 128):
        raise ValueError(f"expand_block_scales: scales {tuple(b.shape)} do not tile a [{n_rows}, {k}] weight")
    out = torch.empty(n_rows, k // 32, dtype=torch.uint8, device=b.device)
    call("dsv4_expand_block_scales", _p(b), n_rows, k, _p(out), _stream(b))
    return out


def prepare_shared_expert(w1, w1s, w3, w3s, w2, w2s):
    """The shared expert's FP8 checkpoint tensors (``w{1,3}`` [I, D], ``w2`` [D, I]
    E4M3, 128x128 E8M0 block scales) on the device in the layout
    ``dsv4_moe_layer_forward_shared`` reads: codes as bytes, scales per 32."""
    out = {}
    for name, w, sc in (("w1", w1, w1s), ("w3", w3, w3s), ("w2", w2, w2s)):
        codes = w.contiguous().view(torch.uint8) if w.dtype != torch.uint8 else w.contiguous()
        _dev(codes, "prepare_shared_expert")
        n, k = codes.shape
        out[name] = codes
        out[name + "s"] = expand_block_scales(sc, n, k)
    I, D = out["w1"].shape
    if out["w3"].shape != (I, D) or out["w2"].shape != (D, I):
        raise ValueError("prepare_shared_expert: w1/w3 must be [I, D] and w2 [D, I]")
    return out


class LayerRunner:
    """Holds a reusable workspace for ``dsv4_moe_layer_forward`` (one routed layer)."""

    def __init__(self, device, n_experts: int, hidden: int, inter: int):
        self.device = torch.device(device)
        self.E, self.D, self.I = n_experts, hidden, inter
        self._ws = None

    def workspace(self, T, K, profile, shared=False):
        n = ctypes.c_int64(0)
        if shared:
            call("dsv4_moe_layer_shared_workspace_bytes", T, K, self.E, self.D, self.I, ctypes.byref(n))
        else:
            call("dsv4_moe_layer_workspace_bytes", T, K, self.E, self.D, self.I, profile, ctypes.byref(n))
        if self._ws is None or self._ws.numel() < n.value:
            self._ws = torch.empty(max(n.value, 256), dtype=torch.uint8, device=self.device)
        return self._ws

    def forward(self, x, topk_ids, topk_w, table, profile=_lib.PROFILE_BF16, rule=_lib.RULE_OCP_FLOOR,
                swiglu_limit=10.0, out=None, shared=None):
        """The routed layer; with ``shared`` (``prepare_shared_expert``) the shared
        expert runs as one more group of the same launches and is added to the
        routed output (bf16 profile only)."""
        _dev(x, "layer_forward")
        if x.dtype != torch.bfloat16 or not x.is_contiguous():
            raise TypeError("layer_forward: contiguous bf16 activations required")
        T, D = x.shape
        ids = topk_ids.contiguous()
        K = ids.shape[1]
        w = topk_w.to(torch.float32).contiguous()
        y = out if out is not None else torch.empty((T, D), dtype=torch.bfloat16, device=x.device)
        i64 = 1 if ids.dtype == torch.int64 else 0
        lim = float(swiglu_limit or 0.0)
        if shared is not None:
            if profile != _lib.PROFILE_BF16:
                raise ValueError("layer_forward: the shared expert is fused in the bf16 profile only")
            ws = self.workspace(T, K, profile, shared=True)
            call("dsv4_moe_layer_forward_shared", _p(x), _p(ids), i64, _p(w), T, K, self.E, D, self.I, _p(table),
                 _p(shared["w1"]), _p(shared["w1s"]), _p(shared["w3"]), _p(shared["w3s"]), _p(shared["w2"]),
                 _p(shared["w2s"]), lim, _p(ws), ws.numel(), _p(y), _stream(x))
            return y
        ws = self.workspace(T, K, profile)
        call("dsv4_moe_layer_forward", profile, rule, _p(x), _p(ids), i64, _p(w), T, K, self.E, D, self.I,
             _p(table), lim, _p(ws), ws.numel(), _p(y), _stream(x))
        return y

    def forward_routed(self, x, gate_w, topk, table, scoring="sqrtsoftplus", bias=None, renormalize=True,
                       scale=1.5, tid2eid=None, input_ids=None, status=None, profile=_lib.PROFILE_BF16,
                       rule=_lib.RULE_OCP_FLOOR, swiglu_limit=10.0, out=None, shared=None):
        """Router + routed layer in one C call (``dsv4_moe_routed_layer_forward``):
        ``_routed(hs, input_ids)`` of ``deepseek_v4.py:150-245`` with its ``_route``
        (``:118-148``), plus the shared expert when ``shared`` is given. Returns
        ``(y bf16 [T, D], weights fp32 [T, K], ids int32 [T, K])``, the same as
        ``route`` followed by ``forward`` on its ids. Arguments as in ``route``;
        x must be bf16."""
        _dev(x, "routed_layer_forward")
        if x.dtype != torch.bfloat16 or not x.is_contiguous():
            raise TypeError("routed_layer_forward: contiguous bf16 activations required")
        if scoring not in _lib.SCORING:
            raise ValueError(f"routed_layer_forward: unknown scoring function {scoring!r}")
        T, D = x.shape
        w = gate_w.to(torch.float32).contiguous()
        if w.dim() != 2 or w.shape != (self.E, D):
            raise ValueError(f"routed_layer_forward: gate weight {tuple(w.shape)} is not [{self.E}, {D}]")
        b = None if bias is None else bias.to(torch.float32).contiguous()
        tab, ids_in, vocab = None, None, 0
        if tid2eid is not None:
            if input_ids is None:
                raise RuntimeError("hash-layer routing needs input_ids")
            tab = tid2eid.contiguous()
            if tab.dtype not in (torch.int32, torch.int64) or tab.dim() != 2 or tab.shape[1] != topk:
                raise ValueError("routed_layer_forward: tid2eid must be int32/int64 [vocab, topk]")
            ids_in = input_ids.reshape(-1).contiguous()
            if ids_in.dtype not in (torch.int32, torch.int64):
                ids_in = ids_in.to(torch.int64)
            if ids_in.numel() != T:
                raise ValueError(f"routed_layer_forward: {ids_in.numel()} input ids for {T} tokens")
            vocab = tab.shape[0]
        if shared is not None and profile != _lib.PROFILE_BF16:
            raise ValueError("routed_layer_forward: the shared expert is fused in the bf16 profile only")
        n = ctypes.c_int64(0)
        call("dsv4_moe_routed_layer_workspace_bytes", T, topk, self.E, D, self.I, profile,
             1 if shared is not None else 0, ctypes.byref(n))
        if self._ws is None or self._ws.numel() < n.value:
            self._ws = torch.empty(max(n.value, 256), dtype=torch.uint8, device=self.device)
        ws = self._ws
        y = out if out is not None else torch.empty((T, D), dtype=torch.bfloat16, device=x.device)
        out_w = torch.empty(T, topk, dtype=torch.float32, device=x.device)
        out_ids = torch.empty(T, topk, dtype=torch.int32, device=x.device)
        sh = [None] * 6 if shared is None else [shared[k] for k in ("w1", "w1s", "w3", "w3s", "w2", "w2s")]
        call("dsv4_moe_routed_layer_forward", profile, rule, _p(x), T, topk, self.E, D, self.I, _p(w), _p(b),
             _p(tab), 1 if tab is not None and tab.dtype == torch.int64 else 0, vocab, _p(ids_in),
             1 if ids_in is not None and ids_in.dtype == torch.int64 else 0, _lib.SCORING[scoring],
             1 if renormalize else 0, float(scale), _p(table), *[_p(t) for t in sh], float(swiglu_limit or 0.0),
             _p(out_w), _p(out_ids), _p(status), _p(ws), ws.numel(), _p(y), _stream(x))
        return y, out_w, out_ids
