"""DeepSeek-V4 MoE takeover with offloaded experts, computed by the HIP expert path.

Surface of ``dsv4_plugin/models/deepseek_v4.py`` in the reference:
``OffloadDeepseekV4MoE(config, parallel_config, quant_config=None, prefix="",
is_draft_layer=False)`` with ``_route`` / ``_routed`` / ``_routed_mxfp4`` /
``forward``, the module toggle ``_MXFP4_GMM`` (read at call time, env
``DSV4_MXFP4_GMM``), ``_offload_load_weights``, ``_ORIG_LOAD_WEIGHTS`` and
``install_patches``.

Routing (``_route``) runs the HIP router (``dsv4_moe_route``) on device
tensors. The routed experts run as ONE call into ``libdsv4hip.so``
(``dsv4_moe_layer_forward``): moe_align, activation quantisation, the grouped
gate/up GEMM with the SwiGLU epilogue, the h quantisation, the grouped down
GEMM and the deterministic combine. Expert weights are read in place from the
engine's packed slots through a device pointer table (no restacking, no
per-expert host sync).

vLLM is optional: when a DeepSeek-V4 model module is importable the class
derives from its ``DeepseekV4MoE`` and ``install_patches`` swaps it in;
otherwise the class is a plain ``nn.Module`` (shared experts omitted) and
``install_patches`` is a no-op.
"""

import importlib
import os
import weakref

import numpy as np
import torch
from torch import nn

from dsv4_plugin.core.engine import get_engine, is_expert_weight
from dsv4_hip import ops as _ops
from dsv4_hip import _lib

_V4_MODULES = ("vllm_ascend.models.deepseek_v4", "vllm.model_executor.models.deepseek_v4")


def _find_v4():
    for name in _V4_MODULES:
        try:
            return importlib.import_module(name)
        except Exception:  # noqa: BLE001 - any import failure means "not available"
            continue
    return None


v4 = _find_v4()

_PATCHED = False
_MXFP4_GMM = os.environ.get("DSV4_MXFP4_GMM", "0") == "1"
# The bf16 profile's per-128 FP8 round trips of x and h (deepseek_v4.py:170,188),
# as the reference does; False runs the pure-bf16 variant (bf16 x and h against
# the bf16-dequantised weights, fp32 accumulation). Read at call time; env
# DSV4_FP8_ROUNDTRIP=0 turns them off.
_FP8_ROUNDTRIP = os.environ.get("DSV4_FP8_ROUNDTRIP", "1") != "0"
# activation scale rule of the a4w4 profile: "ocp_floor" or "ceil_div6"
_MX_RULE = os.environ.get("DSV4_MX_RULE", "ocp_floor")
_RULES = {"ocp_floor": _lib.RULE_OCP_FLOOR, "ceil_div6": _lib.RULE_CEIL_DIV6}

# Shared expert inside the routed launches (bf16 profile): when the engine
# captured the layer's FP8 shared-expert tensors from the weight stream, forward
# runs them as one more group of the grouped GEMMs instead of calling the
# shared MLP. Read at call time; env DSV4_FUSE_SHARED=1.
_FUSE_SHARED = os.environ.get("DSV4_FUSE_SHARED", "0") == "1"

# Predictive prefetch: layer L routes its input with layer L+1's gate (or reads
# layer L+1's tid2eid rows on hash layers, which is exact) and starts the copies
# of the experts that picks, after its own slots are acquired and before its
# GEMMs, so the copies overlap its compute. Read at call time; env
# DSV4_PREFETCH_NEXT=1. Layers register themselves by index.
_PREFETCH_NEXT = os.environ.get("DSV4_PREFETCH_NEXT", "0") == "1"

# When every expert of every layer fits the slot cache (on a 288 GB MI355X the
# whole routed expert set can), route and run the experts in one device call:
# top-k, expert layout and x quantisation share a launch and the routed ids
# never go to the host. The result equals _route + _run_experts bit for bit.
# Read at call time; env DSV4_FUSED_ROUTE=0 turns it off.
_FUSED_ROUTE = os.environ.get("DSV4_FUSED_ROUTE", "1") == "1"
_LAYERS = weakref.WeakValueDictionary()

_BASE = v4.DeepseekV4MoE if (v4 is not None and hasattr(v4, "DeepseekV4MoE")) else nn.Module
_RUNNERS = {}


def _runner(device, E, D, I):
    key = (str(device), E, D, I)
    r = _RUNNERS.get(key)
    if r is None:
        r = _RUNNERS[key] = _ops.LayerRunner(device, E, D, I)
    return r


class _ExpertsFacade:
    """Stand-in for the FusedMoE experts object that vLLM code may touch."""

    is_internal_router = False

    def __init__(self, moe):
        self._moe = moe

    def update_expert_map(self):
        pass


class _Gate(nn.Module):
    """Router parameters when vLLM is absent: fp32 weight [E, D], bias or tid2eid."""

    def __init__(self, hidden, n_experts):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(n_experts, hidden, dtype=torch.float32), requires_grad=False)
        self.e_score_correction_bias = None
        self.tid2eid = None


class OffloadDeepseekV4MoE(_BASE):
    """Routed MoE layer whose experts live in host memory and device slots."""

    def __init__(self, config, parallel_config, quant_config=None, prefix="", is_draft_layer=False):
        nn.Module.__init__(self)  # the base __init__ would place every expert on the device
        self.tp_size = v4.get_tensor_model_parallel_world_size() if v4 is not None else 1
        self.tp_rank = v4.get_tensor_model_parallel_rank() if v4 is not None else 0
        self.layer_idx = int(prefix.split(sep=".")[-2])
        self.routed_scaling_factor = getattr(config, "routed_scaling_factor", 1.5)
        self.swiglu_limit = getattr(config, "swiglu_limit", None)
        self.n_routed_experts = config.n_routed_experts
        self.n_shared_experts = config.n_shared_experts
        self.topk = config.num_experts_per_tok
        self.renormalize = config.norm_topk_prob
        self.num_expert_group = getattr(config, "n_group", 1)
        self.topk_group = getattr(config, "topk_group", 1)
        self.scoring_func = getattr(config, "scoring_func", "softmax")
        self.is_sequence_parallel = getattr(parallel_config, "use_sequence_parallel_moe", False)
        if v4 is not None:
            self.gate = v4.ReplicatedLinear(config.hidden_size, config.n_routed_experts, bias=False,
                                            quant_config=None, prefix=f"{prefix}.gate")
            self.gate.precast_fp32_weight = True
        else:
            self.gate = _Gate(config.hidden_size, config.n_routed_experts)
        eplb = getattr(parallel_config, "eplb_config", None)
        self.enable_eplb = getattr(parallel_config, "enable_eplb", False)
        self.n_redundant_experts = getattr(eplb, "num_redundant_experts", 0) if eplb is not None else 0
        self.n_logical_experts = self.n_routed_experts
        self.n_physical_experts = self.n_logical_experts + self.n_redundant_experts
        self.ep_size = 1
        self.n_local_physical_experts = self.n_physical_experts
        self.physical_expert_start = 0
        self.physical_expert_end = self.n_local_physical_experts
        if config.n_shared_experts is None or v4 is None:
            self.shared_experts = None
        else:
            self.shared_experts = v4.DeepseekV2MLP(
                hidden_size=config.hidden_size,
                intermediate_size=config.moe_intermediate_size * config.n_shared_experts,
                hidden_act=config.hidden_act, swiglu_limit=self.swiglu_limit, quant_config=quant_config,
                is_sequence_parallel=self.is_sequence_parallel, reduce_results=False,
                prefix=f"{prefix}.shared_experts")
        self.hash = self.layer_idx < getattr(config, "num_hash_layers", 0) and not is_draft_layer
        if self.hash:
            self.gate.tid2eid = nn.Parameter(
                torch.zeros(config.vocab_size, config.num_experts_per_tok, dtype=torch.int32), requires_grad=False)
            self.gate.e_score_correction_bias = None
        else:
            self.gate.tid2eid = None
            self.gate.e_score_correction_bias = nn.Parameter(
                torch.zeros(config.n_routed_experts, dtype=torch.float32))
        self.engine = get_engine()
        self.experts = _ExpertsFacade(self)
        _LAYERS[self.layer_idx] = self

    # -- routing ---------------------------------------------------------------
    def _route(self, hs: torch.Tensor, input_ids):
        """``noaux_tc`` + score function routing: biased scores choose, unbiased
        scores weigh, renormalise, scale (``deepseek_v4.py:118-148``), on the HIP
        router (``dsv4_moe_route``: ids int32, each token's picks in descending
        biased score). There is no host implementation: CPU tensors raise."""
        if self.hash and input_ids is None:
            raise RuntimeError("hash-layer routing needs input_ids (forward_context.input_ids is missing)")
        if not hs.is_cuda:
            raise RuntimeError(f"_route: the HIP router needs ROCm device tensors (got {hs.device}); "
                               "there is no CPU implementation")
        return _ops.route(hs, self.gate.weight, self.topk, self.scoring_func,
                          bias=None if self.hash else self.gate.e_score_correction_bias,
                          renormalize=bool(self.renormalize), scale=float(self.routed_scaling_factor),
                          tid2eid=self.gate.tid2eid if self.hash else None, input_ids=input_ids)

    # -- experts ---------------------------------------------------------------
    def _expert_table(self, indices: torch.Tensor, device):
        """Device pointer table of the routed experts and the intermediate size."""
        eng = self.engine
        E = self.n_routed_experts
        ids = indices.detach().to("cpu").numpy()
        if hasattr(eng, "acquire_table"):
            table, _ = eng.acquire_table(self.layer_idx, ids, E)
            inter = eng.bank._layout.shapes["w1p"][0]
            return table, inter
        packed = {int(e): eng.get_packed(self.layer_idx, int(e)) for e in np.unique(ids)}
        inter = next(iter(packed.values()))["w1p"].shape[0]
        return _ops.expert_table(packed, E, device), inter

    def _prefetch_next(self, hs, input_ids):
        """Start the copies of the experts layer ``layer_idx + 1`` is predicted to
        use; returns the number of copies started."""
        nxt = _LAYERS.get(self.layer_idx + 1)
        eng = self.engine
        if nxt is None or not hasattr(eng, "prefetch") or nxt.engine is not eng:
            return 0
        if nxt.hash:
            if input_ids is None:
                return 0
            ids = nxt.gate.tid2eid[input_ids.to(torch.long).flatten()]
        else:
            _, ids = nxt._route(hs, None)
        ids = ids.detach().to("cpu").numpy().reshape(-1)
        ids = np.unique(ids[(ids >= 0) & (ids < nxt.n_routed_experts)])
        return eng.prefetch(nxt.layer_idx, ids) if ids.size else 0

    def _run_experts(self, hs, weights, indices, profile, input_ids=None, shared=None):
        T, D = hs.shape
        x = hs if (hs.dtype == torch.bfloat16 and hs.is_contiguous()) else hs.to(torch.bfloat16).contiguous()
        if T == 0:
            return torch.zeros_like(hs)
        cap = getattr(getattr(self.engine, "bank", None), "packed_capacity", None)
        if cap is not None and hasattr(self.engine, "acquire_table"):
            ids_h = indices.detach().to("cpu").numpy().reshape(-1)
            uniq = np.unique(ids_h[(ids_h >= 0) & (ids_h < self.n_routed_experts)])
            if uniq.size > max(int(cap), 1):
                return self._run_experts_in_parts(x, weights, indices, profile, uniq, max(int(cap), 1),
                                                  shared).type_as(hs)
        table, inter = self._expert_table(indices, hs.device)
        if _PREFETCH_NEXT:
            self._prefetch_next(hs, input_ids)
        limit = self.swiglu_limit if (self.swiglu_limit and self.swiglu_limit > 0) else 0.0
        y = _runner(hs.device, self.n_routed_experts, D, inter).forward(
            x, indices, weights, table, profile=profile, rule=_RULES[_MX_RULE], swiglu_limit=limit, shared=shared)
        return y.type_as(hs)

    def _run_experts_in_parts(self, x, weights, indices, profile, uniq, cap, shared):
        """The routed layer when it routes to more experts than the packed slot cache
        holds (the reference's per-expert ``get_packed`` works at any capacity by
        evicting). The experts are acquired ``cap`` at a time; each part runs the
        grouped GEMMs on the routed rows of its experts (the other ids are masked
        out of its layout) into one buffer of per-row outputs, and a single combine
        sums every token's rows in ascending expert id. Each part takes the M-block
        size the one-part layer takes (16-row blocks below 2048 routed rows, 64 from
        there) with h quantised by its own launch, which the one-part layer's fused
        epilogue matches bit for bit, so the result equals the one-part layer bit for
        bit, except where the one-part layer sends its hot experts to the large-tile
        kernel (from 16,384 routed rows): there the bf16 profile's FP8 x FP4 MFMAs
        group the products of a sum differently and the two agree within the GEMM
        parity bar (the a4w4 products and partial sums are exact, so a4w4 stays bit
        for bit). With a fused shared expert, its output (the layer with no routed
        rows) is added as forward adds the shared MLP's."""
        T, D = x.shape
        K = indices.shape[1]
        E = self.n_routed_experts
        ids = indices.to(torch.int32).contiguous()
        w = weights.to(torch.float32).contiguous().reshape(-1)
        rule = _RULES[_MX_RULE]
        limit = self.swiglu_limit if (self.swiglu_limit and self.swiglu_limit > 0) else 0.0
        fp8 = profile == _lib.PROFILE_BF16
        pure = profile == _lib.PROFILE_BF16_PURE
        if fp8:
            q = _ops.fp8_act_quant(x, 128, want_codes=True, want_e8m0x4=True)
            xa, xs, afmt = q["codes"], q["e8m0x4"], _lib.AFMT_E4M3
        elif pure:
            xa, xs, afmt = x.contiguous(), None, _lib.AFMT_BF16
        else:
            xa, xs, _ = _ops.mxfp4_act_quant(x, rule)
            afmt = _lib.AFMT_E2M1
        # the one-part layer's M-block size (layer_block_m in csrc/capi.cpp)
        bm = 64 if T * K >= 2048 else _lib.GEMM_BLOCK_M
        out = None
        h = None
        for i in range(0, uniq.size, cap):
            part = uniq[i:i + cap]
            table, _ = self.engine.acquire_table(self.layer_idx, part, E)
            inter = self.engine.bank._layout.shapes["w1p"][0]
            if out is None:
                out = torch.empty((T * K, D), dtype=torch.bfloat16, device=x.device)
                h = torch.empty((T * K, inter), dtype=torch.bfloat16, device=x.device)
            keep = torch.isin(ids, torch.from_numpy(part.astype(np.int32)).to(x.device))
            al = _ops.moe_align(torch.where(keep, ids, torch.full_like(ids, -1)), None, E, block_m=bm)
            _ops.gemm_gateup(afmt, xa, xs, K, al, table, D, inter, w, limit, out=h)
            if fp8:
                q = _ops.fp8_act_quant(h, 128, want_codes=True, want_e8m0x4=True)
                ha, has = q["codes"], q["e8m0x4"]
            elif pure:
                ha, has = h, None
            else:
                ha, has, _ = _ops.mxfp4_act_quant(h, rule)
            _ops.gemm_down(afmt, ha, has, al, table, inter, D, out=out)
        y = _ops.moe_combine(out, ids)
        if shared is not None:
            none = torch.full_like(ids, -1)
            ys = _runner(x.device, E, D, h.shape[1]).forward(x, none, weights, table, profile=profile, rule=rule,
                                                               swiglu_limit=limit, shared=shared)
            y = (y.float() + ys.float()).to(torch.bfloat16)
        return y

    def _routed(self, hs: torch.Tensor, input_ids=None, shared=None) -> torch.Tensor:
        """Routed-expert output ``[T, D]`` (``deepseek_v4.py:150-197``); the a4w4
        profile when the module toggle ``_MXFP4_GMM`` is set (``:199-245``).
        ``shared`` (a prepared FP8 shared expert, bf16 profile) adds the shared
        expert's output computed in the same launches."""
        profile = (_lib.PROFILE_A4W4 if _MXFP4_GMM else
                   _lib.PROFILE_BF16 if _FP8_ROUNDTRIP else _lib.PROFILE_BF16_PURE)
        if hs.is_cuda and _FUSED_ROUTE and not _PREFETCH_NEXT:
            y = self._routed_resident(hs, input_ids, profile, shared)
            if y is not None:
                return y
        weights, indices = self._route(hs, input_ids)
        return self._run_experts(hs, weights, indices, profile, input_ids, shared)

    def _routed_resident(self, hs, input_ids, profile, shared):
        """Router and experts in one call (``dsv4_moe_routed_layer_forward``) when the
        engine keeps every expert of this layer resident; None when it cannot."""
        eng = self.engine
        T, D = hs.shape
        if T == 0 or not hasattr(eng, "resident_table"):
            return None
        if self.hash and input_ids is None:
            raise RuntimeError("hash-layer routing needs input_ids (forward_context.input_ids is missing)")
        table = eng.resident_table(self.layer_idx, self.n_routed_experts)
        if table is None:
            return None
        x = hs if (hs.dtype == torch.bfloat16 and hs.is_contiguous()) else hs.to(torch.bfloat16).contiguous()
        inter = eng.bank._layout.shapes["w1p"][0]
        limit = self.swiglu_limit if (self.swiglu_limit and self.swiglu_limit > 0) else 0.0
        y, _, _ = _runner(hs.device, self.n_routed_experts, D, inter).forward_routed(
            x, self.gate.weight, self.topk, table, self.scoring_func,
            bias=None if self.hash else self.gate.e_score_correction_bias, renormalize=bool(self.renormalize),
            scale=float(self.routed_scaling_factor), tid2eid=self.gate.tid2eid if self.hash else None,
            input_ids=input_ids, profile=profile, rule=_RULES[_MX_RULE], swiglu_limit=limit, shared=shared)
        return y.type_as(hs)

    def _fused_shared(self, hs):
        if not (_FUSE_SHARED and not _MXFP4_GMM and _FP8_ROUNDTRIP and hs.is_cuda
                and hasattr(self.engine, "get_shared")):
            return None
        return self.engine.get_shared(self.layer_idx, hs.device)

    def _routed_mxfp4(self, s_w, row, active, group_list, T, hs):
        """a4w4 path from the reference's sorted view (``deepseek_v4.py:199``
        signature): each sorted row is one (token, expert) pair; the grouped
        GEMMs run on the gathered rows and ``moe_unpermute`` sums them back."""
        experts = torch.repeat_interleave(active.to(torch.int64), group_list.to(hs.device))
        xs = _ops.moe_permute(hs.to(torch.bfloat16).contiguous(), row.to(torch.int32))
        out = self._run_experts(xs, s_w.view(-1, 1).float(), experts.view(-1, 1), _lib.PROFILE_A4W4)
        return _ops.moe_unpermute(out.to(torch.bfloat16).contiguous(), row.to(torch.int32), T).type_as(hs)

    def forward(self, hidden_states: torch.Tensor, input_ids=None) -> torch.Tensor:
        num_tokens, hidden_dim = hidden_states.shape
        hs = hidden_states.view(-1, hidden_dim)
        if self.hash and input_ids is None:
            from vllm.forward_context import get_forward_context
            input_ids = getattr(get_forward_context(), "input_ids", None)
        if self.is_sequence_parallel:
            hs = v4.sequence_parallel_chunk(hs)
            if input_ids is not None:
                input_ids = v4.sequence_parallel_chunk(input_ids)
        shared = self._fused_shared(hs)
        if shared is not None:
            out = self._routed(hs, input_ids, shared=shared)
        else:
            out = self._routed(hs, input_ids)
            if self.shared_experts is not None:
                out = out + self.shared_experts(hs)
        if self.is_sequence_parallel:
            out = v4.tensor_model_parallel_all_gather(out, 0)[:num_tokens]
        return out.view(num_tokens, hidden_dim)


def _offload_load_weights(self, weights):
    """Tee of the weight stream: main-model routed experts go to the engine's
    host pool, everything else to the wrapped ``load_weights``
    (``deepseek_v4.py:272-288``)."""
    engine = get_engine()
    it = iter(weights)

    def filtered():
        for name, w in it:
            if is_expert_weight(name):
                engine.capture(name, w)
            else:
                if hasattr(engine, "capture_shared"):
                    engine.capture_shared(name, w)   # a copy; the shared MLP still loads it
                yield name, w

    return _ORIG_LOAD_WEIGHTS(self, filtered())


def _causal_lm_class():
    if v4 is None:
        return None
    for name in ("AscendDeepseekV4ForCausalLM", "DeepseekV4ForCausalLM"):
        cls = getattr(v4, name, None)
        if cls is not None:
            return cls
    return None


_LM_CLASS = _causal_lm_class()
_ORIG_LOAD_WEIGHTS = _LM_CLASS.load_weights if _LM_CLASS is not None else None


def install_patches():
    """Swap in the offload MoE and the load_weights tee (idempotent)."""
    global _PATCHED
    if _PATCHED:
        return
    if v4 is not None and _LM_CLASS is not None and not getattr(v4, "_DSV4_OFFLOAD_PATCHED", False):
        v4.DeepseekV4MoE = OffloadDeepseekV4MoE
        _LM_CLASS.load_weights = _offload_load_weights
        v4._DSV4_OFFLOAD_PATCHED = True
    _PATCHED = True
