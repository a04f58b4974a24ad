"""CPU oracle for the routed-MoE expert path (test infrastructure only).

This package restates, in numpy, the arithmetic of the reference's MoE expert
path so that the HIP kernels can be checked against it. It is the checker,
never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it. The shipped library
(``libdsv4hip.so`` and the Python surface around it) never imports, links or
calls anything here, and raises when its HIP library is missing.

Modules and the reference code each one follows:

* ``mxfp4``   - ``npu_ops.py:20-158`` (FP4 table, E8M0 scale, FP8 act_quant
  round trip, ``_round_fp4``/``fp4_act_quant``, ``dequant_fp4_weight``) plus
  the OCP-MX ``floor(log2 amax) - 2`` activation rule that stands in for the
  closed ``npu_dynamic_mx_quant`` (``deepseek_v4.py:212,240``).
* ``routing`` - ``deepseek_v4.py:150-164`` sort/count/active (moe_align) with
  the stable order, the row gather of ``:171,213-214``, the unweighted
  ``index_add_`` unpermute of ``:195-197`` and the router ``_route`` of
  ``:118-148``.
* ``moe``     - ``deepseek_v4.py:166-245`` (bf16 profile and a4w4 profile of
  ``_routed``), ``model_npu.py:492-533`` (per-expert loop baseline).
* ``lru``     - ``offload.py:86-129`` (OrderedDict LRU and its counters).

How each function is pinned (golden vectors, brute force, library routines,
closed forms) is recorded in the tests that exercise it
(``tests/test_oracle_*.py``). ``mxfp4.dynamic_mx_quant`` with rule
``"ocp_floor"`` has no reference implementation to compare with (the closed
``npu_dynamic_mx_quant`` is not available): it is pinned by the OCP MX v1.0
closed form and brute force only, and its parity with the closed op is
unpinned.
"""
