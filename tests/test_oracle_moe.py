"""Pins the oracle's routing, combine, grouped GEMM, routed-layer and LRU
restatements (CPU only) against library routines, brute force and the
reference's own known-answer tests."""

import numpy as np
import pytest
import torch

from oracle import moe as M
from oracle import mxfp4 as Q
from oracle import routing as RT
from oracle.lru import LRUOracle
from dsv4_hip import synth


def test_align_vs_torch_stable_sort_and_bincount():
    ids = synth.zipf_topk(64, 8, 256)
    w = synth.routing_weights(64, 8)
    al = RT.moe_align(ids, w, 256, 16)
    flat = torch.from_numpy(ids).reshape(-1)
    order = torch.argsort(flat, stable=True)
    assert np.array_equal(al["order"], order.numpy())
    assert np.array_equal(al["s_e"], flat[order].numpy())
    assert np.array_equal(al["s_w"], torch.from_numpy(w).reshape(-1)[order].numpy())
    assert np.array_equal(al["row"], (order // 8).numpy())
    counts = torch.bincount(flat, minlength=256)
    assert np.array_equal(al["counts"], counts.numpy())
    assert np.array_equal(al["active"], torch.nonzero(counts > 0).squeeze(-1).numpy())
    assert np.array_equal(al["group_list"], counts[counts > 0].numpy())


def test_align_invariants_and_padding():
    T, K, E, B = 300, 6, 64, 32
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E), np.random.default_rng(1))
    al = RT.moe_align(ids, np.ones((T, K), np.float32), E, B)
    R = T * K
    assert al["counts"].sum() == R
    assert np.all(np.diff(al["s_e"]) >= 0)
    for e in al["active"]:  # within a group, token ids strictly increase (distinct picks per token)
        rows = al["row"][al["s_e"] == e]
        assert np.all(np.diff(rows) > 0)
    assert sorted(al["order"].tolist()) == list(range(R))  # bijection
    P = al["num_post_padded"]
    assert P % B == 0 and P == sum(-(-c // B) * B for c in al["counts"])
    real = al["sorted_ids"][al["sorted_ids"] < R]
    assert np.array_equal(real, al["order"])
    for b, e in enumerate(al["block_expert"]):
        blk = al["sorted_ids"][b * B:(b + 1) * B]
        blk = blk[blk < R]
        assert np.all(ids.reshape(-1)[blk] == e)


def test_align_bruteforce_tiny():
    ids = np.array([[3, 1], [1, 0], [3, 2], [0, 1]], np.int64)
    al = RT.moe_align(ids, np.arange(8, dtype=np.float32).reshape(4, 2), 4, 2)
    # stable by (expert, flat index): expert 0: flat 3, 6; expert 1: 1, 2, 7; expert 2: 5; expert 3: 0, 4
    assert al["order"].tolist() == [3, 6, 1, 2, 7, 5, 0, 4]
    assert al["row"].tolist() == [1, 3, 0, 1, 3, 2, 0, 2]
    assert al["sorted_ids"].tolist() == [3, 6, 1, 2, 7, 8, 5, 8, 0, 4]
    assert al["block_expert"].tolist() == [0, 1, 1, 2, 3]


def test_unpermute_vs_bruteforce_and_index_add():
    T, K, D = 5, 3, 16
    ids = np.array([[0, 2, 1], [1, 3, 0], [2, 0, 3], [3, 1, 2], [0, 1, 2]], np.int64)
    al = RT.moe_align(ids, np.ones((T, K), np.float32), 4, 1)
    rng = np.random.default_rng(0)
    out = Q.f32_to_bf16_bits(rng.standard_normal((T * K, D)).astype(np.float32) * 100)
    got = RT.unpermute(out, al["row"], T)
    of = Q.bf16_bits_to_f32(out)
    want = np.zeros((T, D), np.float32)
    for u in range(T * K):  # sorted order, one addition at a time, fp32
        want[al["row"][u]] = (want[al["row"][u]] + of[u]).astype(np.float32)
    assert np.array_equal(got, Q.f32_to_bf16_bits(want))
    ref = torch.zeros(T, D).index_add_(0, torch.from_numpy(al["row"]), torch.from_numpy(of)).to(torch.bfloat16)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


def test_grouped_gemm_groups_with_empty_group():
    # _bench_gmm.py:8-22: OUT=8, IN=4, counts [2, 0, 3]
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 4)).astype(np.float32)
    ws = [rng.standard_normal((8, 4)).astype(np.float32) for _ in range(3)]
    out = M.grouped_gemm(x, ws, [2, 0, 3])
    ref = torch.cat([torch.from_numpy(x[:2]).double() @ torch.from_numpy(ws[0]).double().T,
                     torch.from_numpy(x[2:]).double() @ torch.from_numpy(ws[2]).double().T]).float()
    assert np.array_equal(out, ref.numpy())


def test_swiglu_vs_torch():
    rng = np.random.default_rng(3)
    g = (rng.standard_normal((64, 128)) * 8).astype(np.float32)
    u = (rng.standard_normal((64, 128)) * 8).astype(np.float32)
    w = rng.random(64).astype(np.float32)
    ours = M.swiglu(g, u, w, 10.0)
    tg, tu = torch.from_numpy(g), torch.from_numpy(u)
    tu = tu.clamp(min=-10.0, max=10.0)
    tg = tg.clamp(max=10.0)
    ref = torch.nn.functional.silu(tg) * tu * torch.from_numpy(w)[:, None]
    np.testing.assert_allclose(ours, ref.numpy(), rtol=2e-6, atol=1e-6)


def _tiny_experts(E, D, I):
    return {e: synth.expert_weights(e, D, I) for e in range(E)}


def test_routed_bf16_equals_per_expert_baseline_loop():
    # test_moe_align.py:171-177: the grouped path equals model_npu.MoE's loop bit for bit
    T, K, E, D, I = 12, 4, 8, 256, 128
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E), np.random.default_rng(2))
    w = synth.routing_weights(T, K, 3)
    x = synth.bf16_normal(np.random.default_rng(4), (T, D)).view(torch.int16).numpy().view(np.uint16)
    ex = _tiny_experts(E, D, I)
    r = M.routed_bf16(x, ids, w, ex, n_experts=E)
    base = M.baseline_loop_bf16(x, ids, w, ex, n_experts=E)
    assert np.array_equal(r["y"], base)
    # spreading the experts over threads (the CPU baseline does) changes nothing
    rt = M.routed_bf16(x, ids, w, ex, n_experts=E, workers=4)
    for k in ("gate", "up", "h_bf16", "out", "y"):
        assert np.array_equal(rt[k], r[k]), k


def test_routed_bf16_exactness_of_fp8_and_fp4_operands():
    # the FP8 round trip is exactly e4m3(code) * 2^k and the dequantised weight
    # is exactly e2m1 * 2^(s-127): products of these are what the GEMM sums
    T, D = 4, 512
    x = synth.bf16_normal(np.random.default_rng(5), (T, D)).view(torch.int16).numpy().view(np.uint16)
    rt, codes, s, k = Q.act_quant(x, 128)
    vals = Q.e4m3fn_code_to_f32(codes).reshape(T, 4, 128) * np.ldexp(np.float32(1), k)[..., None]
    assert np.array_equal(Q.f32_to_bf16_bits(vals.reshape(T, D)), rt)
    wp, ws = synth.packed_weight(np.random.default_rng(6), 16, D)
    wf = Q.dequant_fp4_weight_f32(wp, ws)
    assert np.array_equal(Q.f32_to_bf16_f32(wf), wf)


def test_a4w4_close_to_bf16_profile():
    # test_moe_align.py:46-56 dual threshold (max < 0.35, mean < 0.08) with x scaled like the
    # reference test (0.5 * N(0,1)) on synthetic weights scaled to a comparable output range
    T, K, E, D, I = 8, 4, 8, 512, 256
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E), np.random.default_rng(7))
    w = synth.routing_weights(T, K, 8)
    x = (synth.bf16_normal(np.random.default_rng(9), (T, D)).float() * 0.5).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    ex = _tiny_experts(E, D, I)
    for d in ex.values():      # scale weights down (E8M0 exponent - 7) for realistic magnitudes
        for k in ("w1s", "w2s", "w3s"):
            d[k] = (d[k] - 7).astype(np.uint8)
    b = Q.bf16_bits_to_f32(M.routed_bf16(xb, ids, w, ex, n_experts=E)["y"])
    for rule in ("ocp_floor", "ceil_div6"):
        a = Q.bf16_bits_to_f32(M.routed_a4w4(xb, ids, w, ex, n_experts=E, rule=rule)["y"])
        diff = np.abs(a - b)
        assert diff.max() < 0.35 * max(1.0, np.abs(b).max()) and diff.mean() < 0.08 * max(1.0, np.abs(b).mean())


def test_lru_known_answer_sequence():
    # test_offload.py:67-86
    lru = LRUOracle(4)
    for eid in range(4):
        lru.access((0, eid))
    assert len(lru.cache) == 4
    lru.access((0, 0))
    hit, ev = lru.access((1, 0))
    assert not hit and ev == (0, 1)
    assert (0, 1) not in lru.cache and (0, 0) in lru.cache and (1, 0) in lru.cache
    assert lru.evictions == 1
    s = lru.stats()
    assert s["misses"] == 5 and s["hits"] == 1 and s["hit_rate"] == 1 / 6
    zero = LRUOracle(0)
    zero.access((0, 0))
    zero.access((0, 0))
    assert len(zero.cache) == 0 and zero.stats()["misses"] == 2


def test_fp8_weight_dequant_matches_torch_float8():
    # npu_ops.py:161-167: E4M3 code value (torch's own float8_e4m3fn decode) x 2^(s-127)
    # per 128x128 block, exact in bf16
    rng = np.random.default_rng(3)
    codes, sc = synth.fp8_weight(rng, 200, 384)
    got = Q.dequant_fp8_weight_f32(codes, sc)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    s = torch.pow(2.0, torch.from_numpy(sc.astype(np.float32)) - 127.0)
    s = s.repeat_interleave(128, 0)[:200].repeat_interleave(128, 1)[:, :384]
    want = (vals * s).numpy()
    assert np.array_equal(got, want)
    assert np.array_equal(Q.f32_to_bf16_f32(got), got)            # bf16-exact
    assert not np.isnan(got).any() and 0x7F not in codes and 0xFF not in codes
    # each block's largest magnitude sits in the top binade of E4M3 (256..448)
    a = np.abs(vals.numpy())
    top = np.array([[a[i:i + 128, j:j + 128].max() for j in range(0, 384, 128)] for i in range(0, 200, 128)])
    assert np.all((top >= 224) & (top <= 448))


def _e2m1_as_fp8(mx, n, k):
    """An MXFP4 weight whose per-32 scales are constant over 128x128 blocks, as
    E4M3 codes + block scales holding exactly the same values."""
    vals = Q.dequant_fp4_weight_f32(mx[0], np.full((n, k // 32), 127, np.uint8))  # E2M1 values, scale 1
    code = {v: c for c in range(256) if c not in (0x7F, 0xFF)
            for v in [float(Q.e4m3fn_code_to_f32(np.array([c], np.uint8))[0])]}
    codes = np.vectorize(lambda v: code[float(v)])(vals).astype(np.uint8)
    return codes, mx[1][::128, ::4].copy()


def test_shared_expert_equals_a_routed_expert_with_weight_one():
    # model_npu.Expert (FP8 weights, no routing weight) and the routed path are the
    # same computation: for weights both formats hold exactly, the shared expert's
    # output equals the routed path with K = 1 and weight 1.0 bit for bit
    T, D, I = 6, 256, 256
    rng = np.random.default_rng(8)
    ex, sh = {}, {}
    for w, (n, k) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
        p = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
        blk = rng.integers(117, 124, size=(n // 128, k // 128), dtype=np.uint8)
        s32 = np.repeat(np.repeat(blk, 128, 0), 4, 1)
        ex[w + "p"], ex[w + "s"] = p, s32
        sh[w], sh[w + "s"] = _e2m1_as_fp8((p, s32), n, k)
        assert np.array_equal(Q.dequant_fp8_weight_f32(sh[w], sh[w + "s"]), Q.dequant_fp4_weight_f32(p, s32))
    x = synth.bf16_normal(np.random.default_rng(9), (T, D)).view(torch.int16).numpy().view(np.uint16)
    ys = M.shared_expert_bf16(x, sh)
    yr = M.routed_bf16(x, np.zeros((T, 1), np.int64), np.ones((T, 1), np.float32), {0: ex}, n_experts=1)["y"]
    assert np.array_equal(ys, yr)
    # the layer output adds the two bf16 tensors (deepseek_v4.py:262-264)
    ids = synth.zipf_topk(T, 2, 4, synth.rank_permutation(4), np.random.default_rng(1))
    w = synth.routing_weights(T, 2, 2)
    exs = {e: synth.expert_weights(e, D, I) for e in range(4)}
    y, y_r, y_s = M.routed_plus_shared_bf16(x, ids, w, exs, sh, n_experts=4)
    assert np.array_equal(y_s, ys)
    want = (torch.from_numpy(y_r.view(np.int16)).view(torch.bfloat16)
            + torch.from_numpy(y_s.view(np.int16)).view(torch.bfloat16))
    assert np.array_equal(y, want.view(torch.int16).numpy().view(np.uint16))
