"""ctypes binding of ``libdsv4hip.so`` (the C ABI declared in ``include/dsv4_moe.h``).

The library is built in-tree (``make -C csrc``, driven by ``__graft_entry__.build``)
and loaded from this directory. There is no fallback: if the library is
missing or fails to load, every call raises.
"""

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdsv4hip.so")

DSV4_OK = 0
AFMT_E4M3 = 0
AFMT_E2M1 = 1
AFMT_BF16 = 2  # bf16 rows as they are, bf16 MFMA on the dequantised weights; block_m 16 or 64
PROFILE_BF16 = 0
PROFILE_A4W4 = 1
PROFILE_BF16_PURE = 2  # the bf16 profile without the FP8 round trips of x and h
RULE_CEIL_DIV6 = 0
RULE_OCP_FLOOR = 1
SCORING = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}
GEMM_BLOCK_M = 16
MAX_EXPERTS = 512
MAX_TOPK = 32
UNPERMUTE_MAX_ROWS = 64  # rows one token may receive in moe_unpermute
NOALLOC_SCRATCH_BYTES = 64 << 20  # static workspace of dsv4_moe_layer_forward_noalloc
NOALLOC_STREAMS_ORDERED = 1  # its flag: this call is ordered after every earlier one on the device
TILED_WEIGHTS = 1  # pointer tag of an MFMA-tiled packed field in the expert table

_c_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "dsv4_last_error": (ctypes.c_char_p, []),
    "dsv4_abi_version": (_i32, []),
    "dsv4_mxfp4_dequant_bf16": (_i32, [_c_p, _c_p, _c_p, _i64, _i64, _c_p]),
    "dsv4_mxfp4_dequant_bf16_multi": (_i32, [_i32, ctypes.POINTER(_c_p), ctypes.POINTER(_c_p), ctypes.POINTER(_c_p),
                                             ctypes.POINTER(_i64), ctypes.POINTER(_i64), _c_p]),
    "dsv4_mxfp4_gemv_bf16": (_i32, [_c_p, _i32, _c_p, _c_p, _i32, _i32, _c_p, _c_p]),
    "dsv4_mxfp4_tile_weights": (_i32, [_c_p, _c_p, _i64, _i64, _i32, _c_p]),
    "dsv4_mxfp4_tile_host": (_i32, [_c_p, _c_p, _i64, _i64]),
    "dsv4_fp8_act_quant": (_i32, [_c_p, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "dsv4_mxfp4_act_quant": (_i32, [_c_p, _i64, _i64, _i32, _c_p, _c_p, _c_p, _c_p]),
    "dsv4_moe_route_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "dsv4_moe_route": (_i32, [_c_p, _i32, _c_p, _c_p, _c_p, _i32, _i64, _c_p, _i32, _i32, _i32, _i32, _i32, _i32,
                              _i32, _f32, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "dsv4_moe_align_max_blocks": (_i32, [_i32, _i32, _i32]),
    "dsv4_moe_align": (_i32, [_c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32] + [_c_p] * 13 + [_c_p]),
    "dsv4_moe_align_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "dsv4_moe_align_ws": (_i32, [_c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32] + [_c_p] * 13
                          + [_c_p, _i64, _c_p]),
    "dsv4_moe_permute": (_i32, [_c_p, _i64, _c_p, _i64, _i64, _c_p, _c_p]),
    "dsv4_moe_unpermute_workspace_bytes": (_i64, [_i32, _i32]),
    "dsv4_moe_unpermute": (_i32, [_c_p, _c_p, _i32, _i32, _i32, _i32, _c_p, _c_p, _c_p, _c_p]),
    "dsv4_moe_combine": (_i32, [_c_p, _c_p, _i32, _i32, _i32, _i32, _c_p, _c_p]),
    "dsv4_moe_gemm_gateup": (_i32, [_i32, _c_p, _c_p, _i32, _c_p, _c_p, _c_p, _i32, _i32, _i32, _c_p, _i32,
                                    _i32, _c_p, _f32, _c_p, _c_p]),
    "dsv4_moe_gemm_down": (_i32, [_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _c_p, _i32, _i32,
                                  _c_p, _c_p]),
    "dsv4_moe_layer_workspace_bytes": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i64)]),
    "dsv4_moe_layer_forward": (_i32, [_i32, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32, _c_p,
                                      _f32, _c_p, _i64, _c_p, _c_p]),
    "dsv4_moe_layer_forward_noalloc": (_i32, [_i32, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32,
                                              _c_p, _f32, _c_p, _i32, _c_p]),
    "dsv4_moe_layer_shared_workspace_bytes": (_i32, [_i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i64)]),
    "dsv4_moe_layer_forward_shared": (_i32, [_c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32, _c_p] + [_c_p] * 6
                                      + [_f32, _c_p, _i64, _c_p, _c_p]),
    "dsv4_expand_block_scales": (_i32, [_c_p, _i64, _i64, _c_p, _c_p]),
    "dsv4_moe_routed_layer_workspace_bytes": (_i32, [_i32] * 7 + [ctypes.POINTER(_i64)]),
    "dsv4_moe_routed_layer_forward": (_i32, [_i32, _i32, _c_p] + [_i32] * 5 + [_c_p, _c_p, _c_p, _i32, _i64, _c_p, _i32,
                                             _i32, _i32, _f32, _c_p] + [_c_p] * 6
                                      + [_f32, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p]),
    # slot cache
    "dsv4_lru_create": (_i32, [_i32, ctypes.POINTER(_c_p)]),
    "dsv4_lru_destroy": (_i32, [_c_p]),
    "dsv4_lru_access": (_i32, [_c_p, _i64, ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i64)]),
    "dsv4_lru_keys": (_i32, [_c_p, _c_p, _i32, ctypes.POINTER(_i32)]),
    "dsv4_slots_create": (_i32, [_i32, _i64, _i32, _c_p, _i32, ctypes.POINTER(_c_p)]),
    "dsv4_slots_destroy": (_i32, [_c_p]),
    "dsv4_slots_host_record": (_i32, [_c_p, _i32, _i32, _i32, ctypes.POINTER(_c_p), ctypes.POINTER(_i32)]),
    "dsv4_slots_num_registered": (_i32, [_c_p, ctypes.POINTER(_i64)]),
    "dsv4_slots_acquire": (_i32, [_c_p, _i32, _c_p, _i32, _c_p, _c_p, ctypes.POINTER(_i32)]),
    "dsv4_slots_prefetch": (_i32, [_c_p, _i32, _c_p, _i32, ctypes.POINTER(_i32)]),
    "dsv4_slots_release": (_i32, [_c_p, _c_p]),
    "dsv4_slots_copy_record": (_i32, [_c_p, _i32, _i32, _c_p, _c_p]),
    "dsv4_slots_lookup": (_i32, [_c_p, _i32, _i32, ctypes.POINTER(_i32)]),
    "dsv4_slots_keys": (_i32, [_c_p, _c_p, _i32, ctypes.POINTER(_i32)]),
    "dsv4_slots_sync": (_i32, [_c_p]),
    "dsv4_slots_invalidate": (_i32, [_c_p, _c_p]),
    "dsv4_slots_stats": (_i32, [_c_p, _c_p]),
    "dsv4_slots_reset_stats": (_i32, [_c_p]),
    "dsv4_probe_mfma_rate": (_i32, [_i32, _i32, _i32, _i32, _i32, _c_p, _c_p, _c_p]),
}

# DSV4_ABI_VERSION of include/dsv4_moe.h that SIGNATURES above describe
ABI_VERSION = 2

_LIB = None


class Dsv4Error(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def lib():
    """Load (once) and return the HIP library; raises if it is not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (or make -C csrc). "
                "The MoE expert path has no implementation other than this HIP library.")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        got = h.dsv4_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"libdsv4hip.so ABI version {got}, this binding expects {ABI_VERSION}")
        _LIB = h
    return _LIB


_FN = {}
_RAW_STREAM = None


def stream_handle(device):
    """torch's current stream on ``device`` as the raw handle the entry points take
    (read without building a torch Stream object per call)."""
    global _RAW_STREAM
    import torch
    if _RAW_STREAM is None:
        _RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", False)
    if _RAW_STREAM:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


def call(name, *args):
    """Call a status-returning entry point and raise ``Dsv4Error`` on failure."""
    fn = _FN.get(name)
    if fn is None:
        fn = _FN[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != DSV4_OK:
        msg = lib().dsv4_last_error().decode(errors="replace")
        raise Dsv4Error(name, rc, msg)
    return rc
