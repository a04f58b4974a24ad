"""HIP (gfx950) implementation of the routed-MoE expert path.

``_lib`` binds the C ABI of ``libdsv4hip.so``; ``ops`` wraps it for torch
tensors on a ROCm device; ``synth`` generates the seeded synthetic workloads.
"""

from . import _lib  # noqa: F401
from ._lib import (AFMT_BF16, AFMT_E2M1, AFMT_E4M3, PROFILE_A4W4, PROFILE_BF16, PROFILE_BF16_PURE, RULE_CEIL_DIV6,  # noqa: F401
                   RULE_OCP_FLOOR, Dsv4Error, lib)
