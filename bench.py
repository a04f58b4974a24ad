"""Benchmark of the MI355X routed-MoE expert path (one GPU).

Headline workload: bf16-profile MoE decode layer - 256 experts, top-8 routing,
8 tokens, hidden 4096, expert intermediate 2048 - with every expert's packed
MXFP4 weights resident in HBM. A step is one pass of the routed layer (align,
FP8 activation quant, gate/up GEMM + SwiGLU, h quant, down GEMM, combine) over
one batch of 8 tokens. Eight independent layers' worth of expert weights are
cycled through so consecutive steps do not re-read the same weights from the
256 MB last-level cache (a decode step visits every layer once).

Prints ONE JSON line. ``value`` = decode tokens/s through the layer.
``roofline`` = the dominant kernel (gate/up GEMM) - algorithmic bytes per
launch over its HIP-event-timed average duration, against 8 TB/s HBM.
``cpu_baseline`` = the same layer on the host cores (min(cores, 16) threads): the
torch CPU restatement of the reference path, with the numpy oracle beside it.
``extra`` = dequant GB/s (config-0 matrices), a4w4 decode (64 tokens),
prefill (2048 tokens) in both profiles, and expert offload (8 layers x 256
experts in pinned host memory, 512 device slots, 512 drifting-Zipf decode
steps: hit rate, H2D traffic and layer tokens/s with exposed copy time).
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepseek-v4-flash-offload_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
MXFP4_PEAK_TFLOPS = 10100.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
D, I, E = 4096, 2048, 256
EXPERT_BYTES = 2 * (I * D // 2 + I * D // 32) + (D * I // 2 + D * I // 32)  # 13,369,344
GATEUP_BYTES = 2 * (I * D // 2 + I * D // 32)                                  # 8,912,896


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8, help="distinct expert-weight sets cycled through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default="",
                    help="profile helper: run only 'decode', 'dequant', 'prefill', 'prefill2048', 'compute', "
                         "'router', 'routed', 'shared', 'offload', 'mfma' (matrix-core issue rates) or 'cpu' "
                         "(CPU baselines of configs 0, 2, 3, 4)")
    ap.add_argument("--offload-steps", type=int, default=512, help="decode steps of the expert-offload leg")
    ap.add_argument("--weight-layout", choices=("tiled", "checkpoint"), default="tiled",
                    help="packed expert weights in HBM: the MFMA-tiled layout (default) or the checkpoint layout")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first copy 1 GiB device-to-device (a plain copy of known size for counter calibration)")
    return ap.parse_args()


WEIGHT_LAYOUT = "tiled"


def progress(msg):
    """One line on stderr per finished leg (the JSON result stays the only stdout line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gen_layer_weights(dev, n_layers, gen):
    """Per layer: one contiguous [E, EXPERT_BYTES] pool + its pointer table. The
    packed fields are random bytes, read in the layout WEIGHT_LAYOUT names (the
    MFMA-tiled one by default: what the slot cache holds)."""
    from dsv4_hip import ops
    pools, tables = [], []
    offs = {}
    o = 0
    for k, n in (("w1p", I * D // 2), ("w1s", I * D // 32), ("w3p", I * D // 2), ("w3s", I * D // 32),
                 ("w2p", D * I // 2), ("w2s", D * I // 32)):
        offs[k] = (o, n)
        o += n
    for _ in range(n_layers):
        pool = torch.randint(0, 256, (E, EXPERT_BYTES), dtype=torch.uint8, device=dev, generator=gen)
        for k in ("w1s", "w3s", "w2s"):  # scale bytes uniform in 117..127
            a, n = offs[k]
            pool[:, a:a + n] = torch.randint(117, 128, (E, n), dtype=torch.uint8, device=dev, generator=gen)
        experts = {e: {k: pool[e, a:a + n] for k, (a, n) in offs.items()} for e in range(E)}
        pools.append(pool)
        tables.append(ops.expert_table(experts, E, dev, tiled=WEIGHT_LAYOUT == "tiled"))
    return pools, tables


def routing_batches(n, T, K, seed):
    from dsv4_hip import synth
    rng = np.random.default_rng(seed)
    perm = synth.rank_permutation(E, 3)
    out = []
    for i in range(n):
        ids = synth.zipf_topk(T, K, E, perm, rng)
        w = synth.routing_weights(T, K, seed + 1000 + i)
        x = synth.bf16_normal(rng, (T, D))
        out.append((x, ids, w))
    return out


def time_layer(runner, batches_dev, tables, steps, warmup, profile, rule, shared=None):
    """Seconds per layer call; ``shared`` (a list of prepared shared experts, one
    per weight set) runs the layer with the shared expert fused in."""
    n = len(batches_dev)
    L = len(tables)
    for i in range(warmup):
        x, ids, w = batches_dev[i % n]
        runner.forward(x, ids, w, tables[i % L], profile=profile, rule=rule,
                       shared=shared[i % L] if shared else None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        x, ids, w = batches_dev[i % n]
        runner.forward(x, ids, w, tables[i % L], profile=profile, rule=rule,
                       shared=shared[i % L] if shared else None)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def measure_gemms(batches_dev, batches_host, tables, steps, profile, rule):
    """Average gate/up and down GEMM durations and their algorithmic bytes.

    The operands of every step (layout, quantised x, quantised h) are prepared
    first; then each GEMM is launched back to back over all steps between two
    HIP events on the stream the kernels run on, so the host never leaves the
    GPU idle inside the timed window."""
    from dsv4_hip import ops, AFMT_E4M3, AFMT_E2M1, PROFILE_BF16
    n, L = len(batches_dev), len(tables)
    fp8 = profile == PROFILE_BF16
    afmt = AFMT_E4M3 if fp8 else AFMT_E2M1
    prep, b_gu, b_dn, flops = [], [], [], []
    for i in range(steps):
        x, ids, w = batches_dev[i % n]
        T, K = ids.shape
        A = len(np.unique(batches_host[i % n][1]))
        al = ops.moe_align(ids, None, E)
        if fp8:
            q = ops.fp8_act_quant(x, 128, want_codes=True, want_e8m0x4=True)
            a, a_s = q["codes"], q["e8m0x4"]
        else:
            a, a_s, _ = ops.mxfp4_act_quant(x, rule)
        h = ops.gemm_gateup(afmt, a, a_s, K, al, tables[i % L], D, I, w.reshape(-1), 10.0)
        if fp8:
            q = ops.fp8_act_quant(h, 128, want_codes=True, want_e8m0x4=True)
            ha, has = q["codes"], q["e8m0x4"]
        else:
            ha, has, _ = ops.mxfp4_act_quant(h, rule)
        prep.append((a, a_s, K, al, tables[i % L], w.reshape(-1), ha, has))
        R = T * K
        a_bytes = T * D * (1 if fp8 else 0.5) + T * D / 32
        b_gu.append(A * GATEUP_BYTES + a_bytes + 2 * R * I)
        b_dn.append(A * (EXPERT_BYTES - GATEUP_BYTES) + R * I * ((1 if fp8 else 0.5) + 1 / 32) + 2 * R * D)
        flops.append(6.0 * R * D * I)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    e0.record(s)
    for a, a_s, K, al, tab, wf, _, _ in prep:
        ops.gemm_gateup(afmt, a, a_s, K, al, tab, D, I, wf, 10.0)
    e1.record(s)
    for _, _, _, al, tab, _, ha, has in prep:
        ops.gemm_down(afmt, ha, has, al, tab, I, D)
    e2.record(s)
    e2.synchronize()
    return {"t_gateup": e0.elapsed_time(e1) * 1e-3 / steps, "t_down": e1.elapsed_time(e2) * 1e-3 / steps,
            "bytes_gateup": float(np.mean(b_gu)), "bytes_down": float(np.mean(b_dn)),
            "flops": float(np.mean(flops))}


def measure_dequant(dev, gen, n_mats=64, reps=5):
    """Config-0 matrices ([2048, 4096] = 2048x2048 packed + 2048x128 scales) dequantised
    back to back over >= 1.36 GB so the 256 MB last-level cache cannot hold them."""
    from dsv4_hip import ops
    N, K = 2048, 4096
    packed = torch.randint(0, 256, (n_mats, N, K // 2), dtype=torch.uint8, device=dev, generator=gen)
    scales = torch.randint(117, 128, (n_mats, N, K // 32), dtype=torch.uint8, device=dev, generator=gen)
    out = torch.empty((n_mats, N, K), dtype=torch.bfloat16, device=dev)
    for m in range(n_mats):
        ops.dequant_mxfp4(packed[m], scales[m], out=out[m])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for m in range(n_mats):
            ops.dequant_mxfp4(packed[m], scales[m], out=out[m])
    e1.record()
    e1.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / (reps * n_mats)
    per = N * K * 2.53125
    # the same 64 matrices as one [64*2048, 4096] launch: kernel throughput without the
    # per-call host overhead of the Python wrapper
    big_p, big_s, big_o = packed.view(n_mats * N, K // 2), scales.view(n_mats * N, K // 32), out.view(n_mats * N, K)
    e0.record()
    for _ in range(reps):
        ops.dequant_mxfp4(big_p, big_s, out=big_o)
    e1.record()
    e1.synchronize()
    tb = e0.elapsed_time(e1) * 1e-3 / reps
    gbs_b = per * n_mats / tb / 1e9
    # config-0 GEMV (bf16 x [1, 4096] @ dequant(W)^T) over the same 64 matrices as one
    # [1, 64*2048] launch: weight bytes (packed + scales) + x + y per launch
    x = torch.randn(1, K, device=dev, generator=gen).to(torch.bfloat16)
    ops.mxfp4_gemv(x, big_p, big_s)
    e0.record()
    for _ in range(reps):
        ops.mxfp4_gemv(x, big_p, big_s)
    e1.record()
    e1.synchronize()
    tg = e0.elapsed_time(e1) * 1e-3 / reps
    gemv_bytes = n_mats * N * (K // 2 + K // 32) + 2 * K + 2 * n_mats * N
    # ExpertBank.get's miss path (offload.py:77-84): one expert's w1 [I, D], w2 [D, I] and w3
    # [I, D], MFMA-tiled as the slot records hold them, dequantised by ONE launch per expert
    # (dsv4_mxfp4_dequant_bf16_multi). 16 distinct experts (1 GB) back to back; the launches
    # are queued behind one batched dequant so that host time between calls is not timed.
    import ctypes
    from dsv4_hip import _lib
    n_ex = 16
    shapes = ((I, D), (D, I), (I, D))
    fn = _lib.lib().dsv4_mxfp4_dequant_bf16_multi
    P3, L3 = ctypes.c_void_p * 3, ctypes.c_int64 * 3
    keep, calls = [], []
    for _ in range(n_ex):
        ts = [(torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen),
               torch.randint(117, 128, (n, k // 32), dtype=torch.uint8, device=dev, generator=gen),
               torch.empty((n, k), dtype=torch.bfloat16, device=dev)) for n, k in shapes]
        keep.append(ts)
        calls.append((3, P3(*[t[0].data_ptr() | _lib.TILED_WEIGHTS for t in ts]), P3(*[t[1].data_ptr() for t in ts]),
                      P3(*[t[2].data_ptr() for t in ts]), L3(*[n for n, _ in shapes]), L3(*[k for _, k in shapes])))
    st = _lib.stream_handle(dev)
    for c in calls:
        assert fn(*c, st) == 0
    torch.cuda.synchronize()
    tm = []
    for _ in range(reps):
        ops.dequant_mxfp4(big_p, big_s, out=big_o)          # keeps the GPU busy while the calls queue
        e0.record()
        for c in calls:
            fn(*c, st)
        e1.record()
        e1.synchronize()
        tm.append(e0.elapsed_time(e1) * 1e-3 / n_ex)
    t_ex = float(np.median(tm))
    ex_bytes = sum(n * k for n, k in shapes) * 2.53125
    t0h = time.perf_counter()
    for _ in range(reps):
        for c in calls:
            fn(*c, st)
    torch.cuda.synchronize()
    host_us = (time.perf_counter() - t0h) / (reps * n_ex) * 1e6
    del keep
    return {"gbs": gbs_b, "frac_hbm": gbs_b / HBM_PEAK_GBS, "batched_us": tb * 1e6,
            "expert_get_one_launch": {"us_per_expert": t_ex * 1e6, "gbs": ex_bytes / t_ex / 1e9,
                                      "frac_hbm": ex_bytes / t_ex / 1e9 / HBM_PEAK_GBS,
                                      "bytes_per_expert": ex_bytes, "experts": n_ex,
                                      "us_per_call_host_inclusive": host_us},
            "per_matrix_call_gbs": per / t / 1e9, "us_per_matrix_call": t * 1e6,
            "bytes_per_matrix": per, "matrices": n_mats,
            "gemv_batched_us": tg * 1e6, "gemv_gbs": gemv_bytes / tg / 1e9,
            "gemv_frac_hbm": gemv_bytes / tg / 1e9 / HBM_PEAK_GBS}


def measure_pcie(dev, record_bytes):
    """Pinned host -> device copy rate: one expert record at a time (16 back to back) and 1 GiB."""
    out = {}
    for name, nbytes, reps in (("record", record_bytes, 16), ("1GiB", 1 << 30, 3)):
        src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        src.fill_(1)
        dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            dst.copy_(src, non_blocking=True)
        e1.record()
        e1.synchronize()
        out[f"h2d_{name}_gbs"] = nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
        del src, dst
    return out


def measure_offload(dev, n_steps=512, n_layers=8, n_slots=512, T=8, K=8, warmup_steps=32, prefetch_steps=128):
    """Expert offload: every layer's 256 experts in a pinned host pool, ``n_slots`` device
    slots shared by all layers (LRU), decode steps of T tokens with per-layer Zipf routing
    whose hot set drifts. A miss is one record copy on the slot cache's copy stream; the
    compute stream waits for it, so exposed copy time is part of the layer time. Host-side
    work (unique ids, slot acquisition, table upload) is inside the timed region, as it is
    for a serving loop.

    A second timed phase (``prefetch_steps`` more steps on the same cache) prefetches, right
    after each layer's acquire, the experts the next layer will route to: the copy stream
    then never waits for a layer's routing to learn its misses. The prefetch is told the
    next layer's true experts, so this phase bounds what next-layer prefetch can give
    (a predictor, such as routing with the next layer's gate, would miss some)."""
    from dsv4_hip import ops, synth, PROFILE_BF16, RULE_OCP_FLOOR
    from dsv4_hip.slots import SlotCache, SlotLayout
    base = [{k: torch.from_numpy(v) for k, v in synth.expert_weights(e, D, I).items()} for e in range(8)]
    layout = SlotLayout(base[0])
    t0 = time.perf_counter()
    cache = SlotCache(dev, n_slots, layout, pin=True)
    pinned = True
    for l in range(n_layers):
        for e in range(E):
            pinned &= cache.register(l, e, base[(l * 7 + e) % len(base)])
    t_reg = time.perf_counter() - t0
    route = synth.DriftingZipf(n_layers, E, K)
    total = warmup_steps + n_steps + prefetch_steps
    ids_all = np.stack([np.stack(route.step(T)) for _ in range(total)])       # [steps, L, T, K]
    w_all = np.stack([synth.routing_weights(T, K, 1000 + s) for s in range(total)])
    ids_dev = torch.from_numpy(ids_all).to(dev)
    w_dev = torch.from_numpy(w_all).to(dev)
    uniq = [[np.unique(ids_all[s, l]).astype(np.int32) for l in range(n_layers)] for s in range(total)]
    x = synth.bf16_normal(np.random.default_rng(6), (T, D)).to(dev)
    runner = ops.LayerRunner(dev, E, D, I)
    ys = [torch.empty((T, D), dtype=torch.bfloat16, device=dev) for _ in range(n_layers)]

    def run(s0, s1, prefetch=False):
        for s in range(s0, s1):
            for l in range(n_layers):
                slots, _ = cache.acquire(l, uniq[s][l])
                if prefetch:
                    ns, nl = (s, l + 1) if l + 1 < n_layers else (s + 1, 0)
                    if ns < s1:
                        cache.prefetch(nl, uniq[ns][nl])
                table = cache.table(uniq[s][l], slots, E)
                runner.forward(x, ids_dev[s, l], w_dev[s], table, profile=PROFILE_BF16, rule=RULE_OCP_FLOOR,
                               out=ys[l])

    run(0, warmup_steps)
    torch.cuda.synchronize()
    cache.reset_stats()
    t0 = time.perf_counter()
    run(warmup_steps, warmup_steps + n_steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    st = cache.stats()
    layer_s = wall / (n_steps * n_layers)
    lookups = st["hits"] + st["misses"]
    res = {"layers": n_layers, "experts_per_layer": E, "slots": n_slots, "steps": n_steps, "tokens_per_step": T,
           "host_pool_gb": n_layers * E * layout.record_bytes / 1e9, "host_pool_pinned": bool(pinned),
           "slot_pool_gb": n_slots * layout.record_bytes / 1e9, "register_s": t_reg,
           "ms_per_layer": layer_s * 1e3, "layer_tokens_per_s": T / layer_s, "step_tokens_per_s": T / (wall / n_steps),
           "hit_rate": st["hits"] / max(lookups, 1), "misses_per_step": st["misses"] / n_steps,
           "h2d_gb": st["bytes_h2d"] / 1e9, "h2d_effective_gbs": st["bytes_h2d"] / wall / 1e9,
           "hits": st["hits"], "misses": st["misses"], "evictions": st["evictions"], "warmup_steps": warmup_steps}
    if prefetch_steps > 0:
        cache.reset_stats()
        t0 = time.perf_counter()
        run(warmup_steps + n_steps, total, prefetch=True)
        torch.cuda.synchronize()
        wall_pf = time.perf_counter() - t0
        sp = cache.stats()
        lp = sp["hits"] + sp["misses"]
        res["prefetch_next_upper_bound"] = {
            "steps": prefetch_steps, "ms_per_layer": wall_pf / (prefetch_steps * n_layers) * 1e3,
            "hit_rate": sp["hits"] / max(lp, 1), "misses_per_step": sp["misses"] / prefetch_steps,
            "prefetched_per_step": sp["prefetched"] / prefetch_steps,
            "h2d_effective_gbs": sp["bytes_h2d"] / wall_pf / 1e9}
    res.update(measure_pcie(dev, layout.record_bytes))
    cache.close()
    del cache, ys, runner
    torch.cuda.empty_cache()
    return res


def measure_shared(dev, gen, steps=200, n_sets=8):
    """The decode layer (8 tokens, top-8 of 256, hidden 4096, inter 2048, bf16
    profile) with the FP8 shared expert (inter 2048, 128x128 block scales) fused
    into its launches, against the routed-only layer on the same inputs. Each of
    the n_sets weight sets has its own shared expert (25 MB of E4M3 weights)."""
    from dsv4_hip import ops, PROFILE_BF16, RULE_OCP_FLOOR, synth
    pools, tables = gen_layer_weights(dev, n_sets, gen)
    shared = []
    for i in range(n_sets):
        sh = synth.shared_expert_weights(900 + i, D, I)
        d = {k: torch.from_numpy(v).to(dev) for k, v in sh.items()}
        shared.append(ops.prepare_shared_expert(d["w1"], d["w1s"], d["w3"], d["w3s"], d["w2"], d["w2s"]))
    host = routing_batches(64, 8, 8, 11)
    dev_b = [(x.to(dev), torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)) for x, ids, w in host]
    runner = ops.LayerRunner(dev, E, D, I)
    t_r = time_layer(runner, dev_b, tables, steps, 20, PROFILE_BF16, RULE_OCP_FLOOR)
    t_s = time_layer(runner, dev_b, tables, steps, 20, PROFILE_BF16, RULE_OCP_FLOOR, shared=shared)
    shared_bytes = 3 * D * I + 3 * D * I // 32
    del pools, tables, shared
    torch.cuda.empty_cache()
    return {"ms_per_layer_routed": t_r * 1e3, "ms_per_layer_routed_plus_shared": t_s * 1e3,
            "tokens_per_s_with_shared": 8 / t_s, "shared_extra_us": (t_s - t_r) * 1e6,
            "shared_weight_bytes": shared_bytes,
            "shared_extra_gbs": shared_bytes / max(t_s - t_r, 1e-9) / 1e9}


def measure_routed_layer(dev, gen, steps=200, n_sets=8):
    """The decode layer with its router (8 tokens, hidden 4096, fp32 gate [256, 4096],
    sqrt(softplus) scores with a correction bias, top-8, bf16 profile): dsv4_moe_route
    followed by dsv4_moe_layer_forward, against dsv4_moe_routed_layer_forward, which
    runs the top-k, the expert layout and the quantisation of x in one launch. Every
    expert is resident (the whole layer in HBM); each weight set has its own gate.
    The C entry points are called directly on preallocated buffers, so the host
    enqueues faster than the GPU runs and the time is the GPU's."""
    import ctypes
    from dsv4_hip import _lib, PROFILE_BF16, RULE_OCP_FLOOR
    lib = _lib.lib()
    pools, tables = gen_layer_weights(dev, n_sets, gen)
    rng = np.random.default_rng(41)
    gates = [torch.from_numpy((rng.standard_normal((E, D)) * 0.03).astype(np.float32)).to(dev) for _ in range(n_sets)]
    biases = [torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(dev) for _ in range(n_sets)]
    xs = [x.to(dev) for x, _, _ in routing_batches(n_sets, 8, 8, 12)]
    T, K = 8, 8
    n_ws = ctypes.c_int64(0)
    lib.dsv4_moe_routed_layer_workspace_bytes(T, K, E, D, I, PROFILE_BF16, 0, ctypes.byref(n_ws))
    ws = torch.empty(n_ws.value, dtype=torch.uint8, device=dev)
    n_l = ctypes.c_int64(0)
    lib.dsv4_moe_layer_workspace_bytes(T, K, E, D, I, PROFILE_BF16, ctypes.byref(n_l))
    ws_l = torch.empty(n_l.value, dtype=torch.uint8, device=dev)
    ws_r = torch.empty(max(int(lib.dsv4_moe_route_workspace_bytes(T, D, E)), 4), dtype=torch.uint8, device=dev)
    out_w = torch.empty(T, K, dtype=torch.float32, device=dev)
    out_ids = torch.empty(T, K, dtype=torch.int32, device=dev)
    y = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sq = _lib.SCORING["sqrtsoftplus"]
    route_args, layer_args, fused_args = [], [], []
    for i in range(n_sets):
        x, g, b, tab = xs[i], gates[i], biases[i], tables[i]
        route_args.append((P(x), 0, P(g), P(b), None, 0, 0, None, 0, T, D, E, K, sq, 1, 1.5, P(out_w), P(out_ids),
                           None, P(ws_r), st))
        layer_args.append((PROFILE_BF16, RULE_OCP_FLOOR, P(x), P(out_ids), 0, P(out_w), T, K, E, D, I, P(tab), 10.0,
                           P(ws_l), ws_l.numel(), P(y), st))
        fused_args.append((PROFILE_BF16, RULE_OCP_FLOOR, P(x), T, K, E, D, I, P(g), P(b), None, 0, 0, None, 0, sq, 1,
                           1.5, P(tab), None, None, None, None, None, None, 10.0, P(out_w), P(out_ids), None, P(ws),
                           ws.numel(), P(y), st))
    f_route, f_layer, f_fused = lib.dsv4_moe_route, lib.dsv4_moe_layer_forward, lib.dsv4_moe_routed_layer_forward

    def two_calls(i):
        if f_route(*route_args[i % n_sets]) or f_layer(*layer_args[i % n_sets]):
            raise RuntimeError(lib.dsv4_last_error().decode())

    def one_call(i):
        if f_fused(*fused_args[i % n_sets]):
            raise RuntimeError(lib.dsv4_last_error().decode())

    res = {}
    for name, fn in (("route_then_layer", two_calls), ("routed_layer", one_call)):
        for i in range(20):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            fn(i)
        e1.record()
        e1.synchronize()
        res[f"ms_per_layer_{name}"] = e0.elapsed_time(e1) / steps
    res["tokens_per_s_routed_layer"] = T / (res["ms_per_layer_routed_layer"] * 1e-3)
    res["saved_us"] = (res["ms_per_layer_route_then_layer"] - res["ms_per_layer_routed_layer"]) * 1e3
    del pools, tables
    torch.cuda.empty_cache()
    return res


def measure_mfma_rate(dev, n_wg=2048, iters=20000):
    """What the matrix cores sustain per scaled-MFMA shape and operand pair (the
    ceiling the grouped GEMMs are judged against besides the published peaks):
    one launch of dsv4_probe_mfma_rate per variant, 8 workgroups of 4 waves per CU,
    timed with events on the launch's stream after an untimed short launch."""
    import ctypes
    from dsv4_hip import _lib
    out = torch.empty(n_wg * 256, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev)
    flop = ctypes.c_double(0.0)
    res = {}
    for shape, sname in ((0, "16x16x128"), (1, "32x32x64")):
        for fa, fb, fname in ((4, 4, "fp4xfp4"), (0, 4, "fp8xfp4"), (0, 0, "fp8xfp8")):
            _lib.call("dsv4_probe_mfma_rate", shape, fa, fb, n_wg, 16, out.data_ptr(), None, st.cuda_stream)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            _lib.call("dsv4_probe_mfma_rate", shape, fa, fb, n_wg, iters, out.data_ptr(), ctypes.addressof(flop),
                      st.cuda_stream)
            e1.record(st)
            e1.synchronize()
            s = e0.elapsed_time(e1) * 1e-3
            peak = MXFP4_PEAK_TFLOPS if fname == "fp4xfp4" else FP8_PEAK_TFLOPS
            res[f"{sname}_{fname}"] = {"tflops": flop.value / s / 1e12, "frac_published_peak": flop.value / s / 1e12 / peak,
                                       "ms": s * 1e3}
    return res


def measure_router(dev, iters=200):
    """dsv4_moe_route (gate logits + score + top-8 + weights) at decode and prefill
    token counts: 256 experts, hidden 4096, fp32 gate weight, sqrt(softplus) scores
    with a correction bias."""
    from dsv4_hip import ops
    rng = np.random.default_rng(31)
    w = torch.from_numpy((rng.standard_normal((E, D)) * 0.03).astype(np.float32)).to(dev)
    b = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(dev)
    res = {}
    for Tn in (8, 2048):
        x = torch.from_numpy(rng.standard_normal((Tn, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
        for _ in range(5):
            ops.route(x, w, 8, "sqrtsoftplus", bias=b)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            ops.route(x, w, 8, "sqrtsoftplus", bias=b)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        byts = E * D * 4 + Tn * D * 2 + Tn * 8 * 8
        flops = 2.0 * Tn * E * D
        res[f"tokens_{Tn}"] = {"us": us, "gbs": byts / us / 1e3, "tflops_fp32": flops / us / 1e6,
                               "frac_fp32_mfma_peak": flops / us / 1e6 / FP32_PEAK_TFLOPS}
    return res


def cpu_baseline(sample_steps=2, threads=None, min_seconds=10.0):
    """The same bf16 decode layer (8 tokens, top-8 of 256, hidden 4096, inter 2048, every
    active expert dequantised from MXFP4 per step, as the GPU reads packed weights) on the
    host cores, two ways:
    * ``value``: the torch CPU restatement of the reference path (oracle/torch_cpu.py:
      per-group fp32 ``torch.matmul``), ``torch.set_num_threads(min(host cores, 16))``;
    * ``numpy_oracle``: the numpy oracle, experts spread over that many threads with
      single-threaded BLAS inside each."""
    from threadpoolctl import threadpool_limits
    from oracle import moe as M
    from oracle import torch_cpu as TC
    from dsv4_hip import synth
    threads = threads or min(os.cpu_count() or 1, 16)
    x, ids, w = synth.layer_inputs(8, 8, E, D)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    experts = {int(e): synth.expert_weights(int(e), D, I) for e in np.unique(ids)}
    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        dt_t, n_t = _timed(lambda: TC.routed_bf16(xb, ids, w, experts), min_seconds, min_runs=sample_steps)
    finally:
        torch.set_num_threads(saved)
    with threadpool_limits(limits=1):
        dt, n = _timed(lambda: M.routed_bf16(xb, ids, w, experts, n_experts=E, workers=threads), min_seconds,
                       min_runs=sample_steps)
    return {"value": 8.0 / dt_t, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n_t} decode steps of the torch CPU restatement after one warm-up (8 tokens, top-8, "
                      f"{len(experts)} active experts, bf16 profile, experts dequantised per step, per-group "
                      f"fp32 torch.matmul), torch on {threads} threads; {dt_t:.2f} s/step",
            "numpy_oracle": {"value": 8.0 / dt, "unit": "tokens/s", "cores": threads,
                             "sample": f"{n} decode steps of the numpy float64 oracle after one warm-up, experts "
                                       f"on {threads} threads; {dt:.2f} s/step"}}


def _timed(fn, min_seconds, min_runs=1, warmup=True):
    """Calls fn until min_runs calls and min_seconds have passed; (seconds per call, calls)."""
    if warmup:
        fn()
    t0 = time.perf_counter()
    n = 0
    while n < min_runs or time.perf_counter() - t0 < min_seconds:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def offload_lru_replay(res, n_layers=8, n_slots=512, T=8, K=8):
    """The offload leg's acquisitions (its warm-up steps, then the timed steps) replayed
    through the textbook LRU the reference's ExpertBank implements (offload.py:103-129);
    the slot cache's hit, miss and eviction counts over the timed steps must equal it."""
    from oracle.lru import LRUOracle
    from dsv4_hip import synth
    route = synth.DriftingZipf(n_layers, E, K)
    lru = LRUOracle(n_slots)
    for s in range(res["warmup_steps"] + res["steps"]):
        if s == res["warmup_steps"]:
            lru.hits = lru.misses = lru.evictions = 0
        for l, ids in enumerate(route.step(T)):
            for e in np.unique(ids):
                lru.access((l, int(e)))
    got = (res["hits"], res["misses"], res["evictions"])
    want = (lru.hits, lru.misses, lru.evictions)
    assert got == want, f"offload slot cache (hits, misses, evictions) {got} != LRU replay {want}"
    return {"hits": lru.hits, "misses": lru.misses, "evictions": lru.evictions, "matches_slot_cache": True}


def cpu_baselines(threads=None, seconds=8.0):
    """The numpy oracle of configs 0, 2, 3 and 4 on the host cores (reported baselines;
    config 1 is ``cpu_baseline``). Each is a bounded sample: a few calls after one
    warm-up, experts spread over ``threads`` threads with single-threaded BLAS inside."""
    import platform
    from threadpoolctl import threadpool_limits
    from oracle import moe as M
    from oracle import mxfp4 as Q
    from oracle.lru import LRUOracle
    from oracle import torch_cpu as TC
    from dsv4_hip import synth
    threads = threads or min(os.cpu_count() or 1, 16)
    cpu_model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), cpu_model)
    except OSError:
        pass
    out = {"threads": threads, "host_cores": os.cpu_count(), "cpu_model": cpu_model,
           "torch": torch.__version__, "numpy": np.__version__, "kind": "port"}
    with threadpool_limits(limits=1):
        # config 0: one [2048, 4096] MXFP4 matrix -> bf16, and the bf16 GEMV x [1, 4096] @ W^T
        packed, scales, x = synth.dequant_config0()
        xb = x.view(torch.int16).numpy().view(np.uint16)
        t_dq, n_dq = _timed(lambda: Q.dequant_fp4_weight(packed, scales), seconds / 2)
        t_gv, n_gv = _timed(lambda: M.dequant_gemv(xb, packed, scales), seconds / 2)
        out["config0_dequant_gemv"] = {"dequant_gbs": 2048 * 4096 * 2.53125 / t_dq / 1e9, "dequant_ms": t_dq * 1e3,
                                       "gemv_with_dequant_ms": t_gv * 1e3, "sample": f"{n_dq} dequants, {n_gv} GEMVs"}
        # config 2: a4w4 layer, 64 tokens
        x2, ids2, w2 = synth.layer_inputs(64, 8, E, D)
        xb2 = x2.view(torch.int16).numpy().view(np.uint16)
        ex2 = {int(e): synth.expert_weights(int(e), D, I) for e in np.unique(ids2)}
        t2, n2 = _timed(lambda: M.routed_a4w4(xb2, ids2, w2, ex2, n_experts=E, workers=threads), seconds,
                        warmup=False)
        out["config2_a4w4_64"] = {"tokens_per_s": 64 / t2, "ms_per_layer": t2 * 1e3,
                                  "sample": f"{n2} layer calls, {len(ex2)} active experts"}
        # config 3: prefill, 2048 tokens, both profiles (one call each, ~15-30 s of CPU work)
        x3, ids3, w3 = synth.layer_inputs(2048, 8, E, D)
        xb3 = x3.view(torch.int16).numpy().view(np.uint16)
        ex3 = {int(e): synth.expert_weights(int(e), D, I) for e in np.unique(ids3)}
        flops3 = 6.0 * 2048 * 8 * D * I
        for name, fn in (("config3_bf16_2048", lambda: M.routed_bf16(xb3, ids3, w3, ex3, n_experts=E, workers=threads)),
                         ("config3_a4w4_2048", lambda: M.routed_a4w4(xb3, ids3, w3, ex3, n_experts=E,
                                                                    workers=threads))):
            t3, n3 = _timed(fn, 0.0, warmup=False)
            out[name] = {"tokens_per_s": 2048 / t3, "ms_per_layer": t3 * 1e3, "tflops": flops3 / t3 / 1e12,
                         "sample": f"{n3} layer call(s), {len(ex3)} active experts"}
        saved = torch.get_num_threads()
        torch.set_num_threads(threads)
        try:
            with threadpool_limits(limits=threads):  # the torch restatement runs on every thread
                for name, fn in (("config3_bf16_2048_torch", lambda: TC.routed_bf16(xb3, ids3, w3, ex3)),
                                 ("config3_a4w4_2048_torch", lambda: TC.routed_a4w4(xb3, ids3, w3, ex3))):
                    t3, n3 = _timed(fn, 0.0, warmup=False)
                    out[name] = {"tokens_per_s": 2048 / t3, "ms_per_layer": t3 * 1e3,
                                 "tflops": flops3 / t3 / 1e12,
                                 "sample": f"{n3} layer call(s) of the torch CPU restatement, torch on "
                                           f"{threads} threads"}
        finally:
            torch.set_num_threads(saved)
        del ex3
        # config 4: the offload workload's routing (8 layers, drifting Zipf, 512 slots) through
        # an LRU of packed experts; on the host every layer dequantises its active experts
        route = synth.DriftingZipf(8, E, 8)
        lru = LRUOracle(512)
        bases = [synth.expert_weights(e, D, I) for e in range(8)]
        wts = synth.routing_weights(8, 8, 1000)
        xb4 = synth.bf16_normal(np.random.default_rng(6), (8, D)).view(torch.int16).numpy().view(np.uint16)
        for _ in range(64):                  # warm the LRU with the bench's own warm-up steps
            for l, ids in enumerate(route.step(8)):
                for e in np.unique(ids):
                    lru.access((l, int(e)))
        lru.hits = lru.misses = lru.evictions = 0
        n_layers, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds or n_layers < 8:
            for l, ids in enumerate(route.step(8)):
                for e in np.unique(ids):
                    lru.access((l, int(e)))
                ex = {int(e): bases[(l * 7 + int(e)) % 8] for e in np.unique(ids)}
                M.routed_bf16(xb4, ids, wts, ex, n_experts=E, workers=threads)
                n_layers += 1
        t4 = (time.perf_counter() - t0) / n_layers
        out["config4_offload"] = {"layer_tokens_per_s": 8 / t4, "ms_per_layer": t4 * 1e3,
                                  "hit_rate": lru.stats()["hit_rate"],
                                  "sample": f"{n_layers} layer calls (8 tokens each) of the drifting-Zipf routing "
                                            "after 64 warm-up steps; every active expert dequantised per call"}
    return out


def main():
    global WEIGHT_LAYOUT
    args = parse()
    WEIGHT_LAYOUT = args.weight_layout
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(across GPUs the expert path would shard by expert, with an all-to-all of routed rows per layer)", file=sys.stderr)
        sys.exit(2)
    from dsv4_hip import ops, PROFILE_A4W4, PROFILE_BF16, PROFILE_BF16_PURE, RULE_OCP_FLOOR
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    T, K = 8, 8
    if args.calib_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"calib-copy: {src.numel()} bytes read, {dst.numel()} bytes written", file=sys.stderr)
        del src, dst
        torch.cuda.empty_cache()
    pure_decode = None
    if args.only in ("", "decode"):
        pools, tables = gen_layer_weights(dev, args.layers, gen)
        host = routing_batches(64, T, K, 11)
        dev_b = [(x.to(dev), torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)) for x, ids, w in host]
        runner = ops.LayerRunner(dev, E, D, I)
        torch.cuda.synchronize()
        s = time_layer(runner, dev_b, tables, args.steps, args.warmup, PROFILE_BF16, RULE_OCP_FLOOR)
        gm = measure_gemms(dev_b, host, tables, min(args.steps, 100), PROFILE_BF16, RULE_OCP_FLOOR)
        if not args.no_extra and args.only == "":  # the same layer without the FP8 round trips of x and h
            sp = time_layer(runner, dev_b, tables, args.steps, args.warmup, PROFILE_BF16_PURE, RULE_OCP_FLOOR)
            pure_decode = {"ms_per_layer": sp * 1e3, "tokens_per_s": T / sp,
                           "vs_fp8_roundtrip_layer": s / sp}
        ach = gm["bytes_gateup"] / gm["t_gateup"] / 1e9
        # HBM bytes per launch from the committed counter profile (FETCH_SIZE/WRITE_SIZE
        # scaled by a 1 GiB copy): measured traffic / algorithmic bytes, applied to this run
        traffic = None
        tpath = os.path.join(ROOT, "profiles", "moe_gemm_decode_bf16_traffic.json")
        if os.path.exists(tpath):
            with open(tpath) as f:
                tr = json.load(f)
            traffic = tr["gateup_traffic_over_algorithmic"] * gm["bytes_gateup"]
        line = {
            "metric": "MoE decode tok/s (bf16 profile, 256 experts top-8, hidden 4096, inter 2048)",
            "value": T / s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": s * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp8e4m3 x mxfp4 (scaled MFMA: exact products, fp32 sums that drop products >10-13 binades "
                     "below their group's largest)", "data": "synthetic",
            "config": {"workload": "bf16-profile MoE decode layer: 8 tokens, 256 experts, top-8 Zipf(1.1), "
                                   "hidden 4096, inter 2048, MXFP4 experts resident in HBM",
                       "tokens": T, "topk": K, "experts": E, "hidden": D, "inter": I,
                       "weight_sets_cycled": args.layers, "weight_layout": WEIGHT_LAYOUT},
            "roofline": {"bound": "hbm", "kernel": "moe_gemm_kernel<E4M3, gate/up>", "achieved": ach,
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach / HBM_PEAK_GBS, "traffic": traffic,
                         "traffic_source": "profiles/moe_gemm_decode_bf16_traffic.json" if traffic else None,
                         "algorithmic_bytes_per_launch": gm["bytes_gateup"],
                         "avg_launch_us": gm["t_gateup"] * 1e6},
            "gemm": {"gateup_us": gm["t_gateup"] * 1e6, "down_us": gm["t_down"] * 1e6,
                     "down_gbs": gm["bytes_down"] / gm["t_down"] / 1e9,
                     "layer_tflops": gm["flops"] / s / 1e12},
        }
        del pools, tables
        torch.cuda.empty_cache()
        progress(f"decode: {s * 1e6:.1f} us per layer")
    else:
        line = {"metric": "profile helper", "value": None}
    extra = {}
    if pure_decode is not None:
        extra["bf16_pure_decode_8"] = pure_decode
    if not args.no_extra and args.only in ("", "dequant"):
        extra["dequant_config0"] = measure_dequant(dev, gen)
        progress("dequant done")
        torch.cuda.empty_cache()
    if not args.no_extra and args.only in ("", "prefill", "prefill2048", "compute"):
        pools, tables = gen_layer_weights(dev, 2, gen)
        runner = ops.LayerRunner(dev, E, D, I)
        legs = []
        if args.only in ("", "prefill", "prefill2048"):
            legs += [("a4w4_decode_64", 64, PROFILE_A4W4), ("bf16_prefill_2048", 2048, PROFILE_BF16),
                     ("a4w4_prefill_2048", 2048, PROFILE_A4W4), ("bf16_pure_prefill_2048", 2048, PROFILE_BF16_PURE)]
        if args.only in ("", "prefill", "compute"):
            # the compute-bound point: 16384 tokens x top-8 = 131072 routed rows, every expert
            # with hundreds of rows, arithmetic intensity ~1.9 kFLOP/B (MXFP4 ridge ~1.26 kFLOP/B)
            legs += [("bf16_prefill_16384", 16384, PROFILE_BF16), ("a4w4_prefill_16384", 16384, PROFILE_A4W4),
                     ("bf16_pure_prefill_16384", 16384, PROFILE_BF16_PURE)]
        for name, Tn, prof in legs:
            host = routing_batches(2 if Tn > 2048 else 4, Tn, K, 21 + Tn)
            dev_b = [(x.to(dev), torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev))
                     for x, ids, w in host]
            st = 20 if Tn <= 64 else 5
            s2 = time_layer(runner, dev_b, tables, st, 3, prof, RULE_OCP_FLOOR)
            A = float(np.mean([len(np.unique(b[1])) for b in host]))
            flops = 6.0 * Tn * K * D * I
            byts = A * EXPERT_BYTES + 4 * Tn * D
            peak = {PROFILE_A4W4: MXFP4_PEAK_TFLOPS, PROFILE_BF16: FP8_PEAK_TFLOPS,
                    PROFILE_BF16_PURE: BF16_PEAK_TFLOPS}[prof]
            extra[name] = {"ms_per_layer": s2 * 1e3, "tokens_per_s": Tn / s2, "tflops": flops / s2 / 1e12,
                           "frac_mfma_peak": flops / s2 / 1e12 / peak, "mfma_peak_tflops": peak,
                           "hbm_gbs": byts / s2 / 1e9, "frac_hbm": byts / s2 / 1e9 / HBM_PEAK_GBS,
                           "active_experts": A}
            progress(f"{name}: {s2 * 1e3:.3f} ms per layer")
            del host, dev_b
        del pools, tables, runner
        torch.cuda.empty_cache()
    if not args.no_extra and args.only in ("", "mfma"):
        extra["mfma_rate"] = measure_mfma_rate(dev)
        progress("mfma probe done")
    if not args.no_extra and args.only in ("", "router"):
        extra["router"] = measure_router(dev)
        progress("router done")
    if not args.no_extra and args.only in ("", "routed"):
        extra["decode_routed_layer"] = measure_routed_layer(dev, gen)
        progress("routed layer done")
    if not args.no_extra and args.only in ("", "shared"):
        extra["decode_with_shared_expert"] = measure_shared(dev, gen)
        progress("shared expert done")
    if not args.no_extra and args.only in ("", "offload") and args.offload_steps > 0:
        extra["offload_config4"] = measure_offload(dev, n_steps=args.offload_steps)
        progress("offload done")
    if extra:
        line["extra"] = extra
    if not args.no_cpu_baseline and args.only == "":
        line["cpu_baseline"] = cpu_baseline()
        progress("cpu baseline done")
        line["cpu_baseline"]["host_threads_available"] = os.cpu_count()
    if not args.no_cpu_baseline and args.only in ("", "cpu"):
        extra["cpu_baselines"] = cpu_baselines()
        progress("cpu baselines of configs 0, 2, 3, 4 done")
        if "offload_config4" in extra:  # the CPU leg checks the offload leg's policy too
            extra["offload_config4"]["lru_replay"] = offload_lru_replay(extra["offload_config4"])
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
