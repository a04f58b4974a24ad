"""The C-ABI library loads on a CPU-only host, exports every function the header
declares, and rejects bad arguments on the host before touching a GPU."""

import ctypes
import os
import re

import pytest

from dsv4_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsv4_moe.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b(?:int|int64_t|const char\*)\s+(dsv4_\w+)\s*\(", src)
    assert names, "no declarations found"
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    assert set(declared_functions()) <= set(_lib.SIGNATURES), set(declared_functions()) - set(_lib.SIGNATURES)


def test_abi_version():
    m = re.search(r"#define DSV4_ABI_VERSION (\d+)", open(HEADER).read())
    assert m and int(m.group(1)) == _lib.ABI_VERSION == _lib.lib().dsv4_abi_version()


def _err(rc):
    return rc, _lib.lib().dsv4_last_error().decode()


def test_dequant_validation():
    lib = _lib.lib()
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16(None, None, None, 4, 33, None))
    assert rc == -2 and "multiple of 32" in msg
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16(None, None, None, 4, 64, None))
    assert rc == -1 and "null" in msg
    assert lib.dsv4_mxfp4_dequant_bf16(None, None, None, 0, 64, None) == 0  # empty is a no-op


def test_dequant_multi_validation():
    lib = _lib.lib()
    P = ctypes.c_void_p * 2
    L = ctypes.c_int64 * 2
    nul = P(None, None)
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16_multi(0, nul, nul, nul, L(1, 1), L(32, 32), None))
    assert rc == -3 and "tensors" in msg
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16_multi(9, nul, nul, nul, L(1, 1), L(32, 32), None))
    assert rc == -3
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16_multi(2, nul, nul, nul, L(0, 1), L(32, 48), None))
    assert rc == -2 and "multiple of 32" in msg
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16_multi(2, nul, nul, nul, L(1, 1), L(32, 32), None))
    assert rc == -1 and "null" in msg
    # a tiled source (pointer tag 1) needs 16-row tiles and 256-wide K stages
    rc, msg = _err(lib.dsv4_mxfp4_dequant_bf16_multi(1, P(1, None), nul, nul, L(8, 0), L(256, 0), None))
    assert rc == -2 and "tiled" in msg
    # empty tensors are no-ops, null pointers allowed for them
    assert lib.dsv4_mxfp4_dequant_bf16_multi(2, nul, nul, nul, L(0, 4), L(64, 0), None) == 0


def test_quant_validation():
    lib = _lib.lib()
    rc, msg = _err(lib.dsv4_fp8_act_quant(None, 2, 256, 64, None, None, None, None, None))
    assert rc == -3 and "block_size" in msg
    rc, msg = _err(lib.dsv4_fp8_act_quant(None, 2, 200, 128, None, None, None, None, None))
    assert rc == -2
    rc, msg = _err(lib.dsv4_mxfp4_act_quant(None, 2, 64, 7, None, None, None, None))
    assert rc == -3 and "rule" in msg


def test_align_validation_and_bound():
    lib = _lib.lib()
    # the padded-block bound: sum_e ceil(c_e/B) <= R/B + min(E, R) (+1)
    assert lib.dsv4_moe_align_max_blocks(64, 256, 16) == 64 // 16 + 64 + 1
    assert lib.dsv4_moe_align_max_blocks(16384, 256, 64) == 256 + 256 + 1
    args = [None, 1, None, 8, 8, 1024, 16, 100] + [None] * 13 + [None]
    rc, msg = _err(lib.dsv4_moe_align(*args))
    assert rc == -3 and "E=1024" in msg
    args = [None, 1, None, 8, 8, 256, 16, 3] + [None] * 13 + [None]
    rc, msg = _err(lib.dsv4_moe_align(*args))
    assert rc == -2 and "max_blocks" in msg


def test_gemm_and_layer_validation():
    lib = _lib.lib()
    rc, msg = _err(lib.dsv4_moe_gemm_gateup(0, None, None, 8, None, None, None, 64, 32, 10, None, 4096, 2048,
                                            None, ctypes.c_float(10.0), None, None))
    assert rc == -3 and "block_m" in msg
    rc, msg = _err(lib.dsv4_moe_gemm_down(3, None, None, None, None, None, 64, 16, 10, None, 2048, 4096, None,
                                          None))
    assert rc == -3 and "format" in msg
    # bf16 activations (the pure-bf16 variant) only in the 16- and 64-row kernels
    rc, msg = _err(lib.dsv4_moe_gemm_down(2, None, None, None, None, None, 64, 128, 10, None, 2048, 4096, None,
                                          None))
    assert rc == -3 and "bf16 activations" in msg
    rc, msg = _err(lib.dsv4_moe_gemm_down(2, None, None, None, None, None, 64, 64, 10, None, 2048, 4096, None,
                                          None))
    assert rc == -1 and "null" in msg
    n = ctypes.c_int64(0)
    assert lib.dsv4_moe_layer_workspace_bytes(2048, 8, 256, 4096, 2048, 2, ctypes.byref(n)) == 0
    assert lib.dsv4_moe_layer_workspace_bytes(8, 8, 256, 4096, 2048, 3, ctypes.byref(n)) == -3
    rc, msg = _err(lib.dsv4_moe_gemm_gateup(0, None, None, 8, None, None, None, 64, 16, 10, None, 4000, 2048,
                                            None, ctypes.c_float(10.0), None, None))
    assert rc == -3 and "512" in msg
    # K = 8192 is not compiled (its unrolled K loops spill): rejected before any launch
    for kd in (8192, 256):
        rc, msg = _err(lib.dsv4_moe_gemm_gateup(0, None, None, 8, None, None, None, 64, 16, 10, None, kd, 2048,
                                                None, ctypes.c_float(10.0), None, None))
        assert rc == -3 and "unsupported" in msg, kd
    rc, msg = _err(lib.dsv4_moe_gemm_down(0, None, None, None, None, None, 64, 16, 10, None, 8192, 4096, None, None))
    assert rc == -3 and "unsupported" in msg
    # unpermute: at most 64 rows per token (one wave ranks them)
    rc, msg = _err(lib.dsv4_moe_unpermute(None, None, 8, 2, 65, 64, None, None, None, None))
    assert rc == -3 and "Kmax" in msg
    n = ctypes.c_int64(0)
    assert lib.dsv4_moe_layer_workspace_bytes(8, 8, 256, 4096, 2048, 0, ctypes.byref(n)) == 0
    assert n.value > 2 * 64 * 4096  # holds at least the [R, D] bf16 expert outputs
    rc, msg = _err(lib.dsv4_moe_layer_forward(0, 1, None, None, 1, None, 8, 8, 256, 4096, 2048, None,
                                              ctypes.c_float(10.0), None, 0, None, None))
    assert rc == -1


def test_ops_reject_cpu_tensors():
    import torch
    from dsv4_hip import ops
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.dequant_mxfp4(torch.zeros(4, 16, dtype=torch.uint8), torch.zeros(4, 1, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.moe_align(torch.zeros(4, 2, dtype=torch.int64), None, 8)


def test_route_validation():
    lib = _lib.lib()
    args = dict(x=None, x_f32=0, w=None, bias=None, tab=None, tab64=0, vocab=0, ids=None, ids64=0, T=4, D=4096,
                E=256, K=8, scoring=2, renorm=1, scale=1.5, ow=None, oi=None, st=None, ws=None, stream=None)

    def route(**kw):
        a = dict(args, **kw)
        return _err(lib.dsv4_moe_route(*a.values()))

    rc, msg = route(D=4080)
    assert rc == -2 and "multiple of 32" in msg
    rc, msg = route(E=250)
    assert rc == -3 and "experts" in msg
    rc, msg = route(E=1024)
    assert rc == -3
    rc, msg = route(K=0)
    assert rc == -3 and "top-k" in msg
    rc, msg = route(K=65, E=512)
    assert rc == -3
    rc, msg = route(scoring=3)
    assert rc == -3 and "scoring" in msg
    rc, msg = route()
    assert rc == -1 and "null" in msg
    assert route(T=0)[0] == 0  # no tokens is a no-op
    # the partial-logit workspace [S, T, E]: K split 16 ways at decode sizes, 8 ways at 2048 tokens
    assert lib.dsv4_moe_route_workspace_bytes(8, 4096, 256) == 16 * 8 * 256 * 4
    assert lib.dsv4_moe_route_workspace_bytes(2048, 4096, 256) == 8 * 2048 * 256 * 4
    assert lib.dsv4_moe_route_workspace_bytes(0, 4096, 256) == 0
