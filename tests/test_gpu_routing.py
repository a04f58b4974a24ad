"""GPU parity: moe_align (stable sort + padded layout), permute, unpermute, combine.

Index outputs are bit-exact against the oracle and against torch's stable
argsort/bincount; the combine is bit-exact against the oracle's index_add_
restatement."""

import numpy as np
import pytest
import torch

from oracle import routing as RT
from oracle import mxfp4 as Q
from dsv4_hip import ops, synth

pytestmark = pytest.mark.gpu


def _check_align(res, al, T, K):
    R = T * K
    assert np.array_equal(res.order.cpu().numpy(), al["order"])
    assert np.array_equal(res.s_e.cpu().numpy(), al["s_e"])
    assert np.array_equal(res.row.cpu().numpy(), al["row"])
    assert np.array_equal(res.s_w.cpu().numpy(), al["s_w"])
    assert np.array_equal(res.counts.cpu().numpy(), al["counts"])
    assert np.array_equal(res.expert_start.cpu().numpy(), al["expert_start"])
    na = int(res.num_active.item())
    assert na == len(al["active"])
    assert np.array_equal(res.active.cpu().numpy()[:na], al["active"])
    assert np.all(res.active.cpu().numpy()[na:] == -1)
    P = int(res.num_post_padded.item())
    assert P == al["num_post_padded"]
    assert np.array_equal(res.sorted_ids.cpu().numpy()[:P], al["sorted_ids"])
    assert np.array_equal(res.block_expert.cpu().numpy()[:P // res.block_m], al["block_expert"])
    pp = res.padded_pos.cpu().numpy()
    assert np.array_equal(al["sorted_ids"][pp], np.arange(R))
    assert int(res.status.item()) == 0


@pytest.mark.parametrize("T,K,E,bm", [(8, 8, 256, 16), (64, 8, 256, 16), (2048, 8, 256, 16), (2048, 8, 256, 64),
                                      (8, 6, 256, 16), (1, 8, 256, 16), (3000, 6, 160, 32), (512, 4, 512, 16)])
def test_moe_align_matches_oracle(gpu, T, K, E, bm):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(4 + T))
    w = synth.routing_weights(T, K, 5)
    al = RT.moe_align(ids, w, E, bm)
    for dt in (torch.int64, torch.int32):
        res = ops.moe_align(torch.from_numpy(ids).to(dt).to(gpu), torch.from_numpy(w).to(gpu), E, bm)
        torch.cuda.synchronize()
        _check_align(res, al, T, K)
    # library cross-check: torch's stable argsort and bincount
    flat = torch.from_numpy(ids).reshape(-1)
    assert np.array_equal(al["order"], torch.argsort(flat, stable=True).numpy())
    assert np.array_equal(al["counts"], torch.bincount(flat, minlength=E).numpy())


def test_moe_align_all_to_one_expert_and_out_of_range(gpu):
    ids = np.full((100, 4), 7, dtype=np.int64)
    ids[:, 1] = 3
    ids[:, 2] = 250
    ids[:, 3] = 9
    al = RT.moe_align(ids, np.ones((100, 4), np.float32), 256, 16)
    res = ops.moe_align(torch.from_numpy(ids).to(gpu), torch.ones(100, 4, device=gpu), 256, 16)
    torch.cuda.synchronize()
    _check_align(res, al, 100, 4)
    bad = ids.copy()
    bad[5, 2] = 256
    bad[7, 0] = -1
    res = ops.moe_align(torch.from_numpy(bad).to(gpu), None, 256, 16)
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="2 expert id"):
        res.check()


def test_moe_align_empty(gpu):
    res = ops.moe_align(torch.zeros((0, 8), dtype=torch.int64, device=gpu), None, 256, 16)
    torch.cuda.synchronize()
    assert int(res.num_post_padded.item()) == 0 and int(res.num_active.item()) == 0


def test_permute_rows(gpu):
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.integers(0, 256, (64, 2048 + 128), dtype=np.uint8)).to(gpu)
    row = torch.from_numpy(rng.integers(0, 64, 300).astype(np.int32)).to(gpu)
    out = ops.moe_permute(x, row)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), x.cpu()[row.cpu().long()])


@pytest.mark.parametrize("T,K,D", [(8, 8, 4096), (64, 8, 4096), (37, 6, 512)])
def test_unpermute_and_combine_bitexact(gpu, T, K, D):
    E = 256
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(T))
    al = RT.moe_align(ids, np.ones((T, K), np.float32), E, 16)
    rng = np.random.default_rng(9)
    out_sorted = Q.f32_to_bf16_bits((rng.standard_normal((T * K, D)) * 3).astype(np.float32))
    want = RT.unpermute(out_sorted, al["row"], T)
    # library cross-check of the oracle: torch index_add_ on CPU
    ref = torch.zeros(T, D).index_add_(0, torch.from_numpy(al["row"]),
                                       torch.from_numpy(Q.bf16_bits_to_f32(out_sorted))).to(torch.bfloat16)
    assert np.array_equal(ref.view(torch.int16).numpy().view(np.uint16), want)
    dev_out = torch.from_numpy(out_sorted.view(np.int16)).view(torch.bfloat16).to(gpu)
    y = ops.moe_unpermute(dev_out, torch.from_numpy(al["row"]).to(gpu), T)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), want)
    # flat-order combine: row t*K+k holds the sorted row of flat index t*K+k
    out_flat = np.empty_like(out_sorted)
    out_flat[al["order"]] = out_sorted
    yf = ops.moe_combine(torch.from_numpy(out_flat.view(np.int16)).view(torch.bfloat16).to(gpu),
                         torch.from_numpy(ids).to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(yf.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("R,T,seed", [(3, 2, 0), (200, 10, 1), (64, 1, 2), (513, 40, 3)])
def test_unpermute_uneven_rows_per_token(gpu, R, T, seed):
    # index_add_ semantics for any row -> token map (not only K rows per token): uneven
    # counts, a token with no rows, all rows on one token (64 = the per-token bound)
    rng = np.random.default_rng(seed)
    row = np.zeros(R, np.int32) if R == 3 or T == 1 else rng.integers(0, T, R).astype(np.int32)
    if T > 2:
        row[row == T - 1] = 0          # token T-1 receives nothing
    D = 512
    out = Q.f32_to_bf16_bits((rng.standard_normal((R, D)) * 3).astype(np.float32))
    ref = torch.zeros(T, D).index_add_(0, torch.from_numpy(row.astype(np.int64)),
                                       torch.from_numpy(Q.bf16_bits_to_f32(out))).to(torch.bfloat16)
    want = ref.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(RT.unpermute(out, row, T), want)
    y = ops.moe_unpermute(torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).to(gpu),
                          torch.from_numpy(row).to(gpu), T)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), want)


def test_unpermute_rejects_what_it_would_drop(gpu):
    D = 64
    out = torch.zeros(70, D, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="beyond 64 rows"):
        ops.moe_unpermute(out, torch.zeros(70, dtype=torch.int32, device=gpu), 2)   # 70 rows on one token
    bad = torch.tensor([0, 1, 2, 5], dtype=torch.int32, device=gpu)
    with pytest.raises(IndexError):
        ops.moe_unpermute(out[:4], bad, 3)
    with pytest.raises(IndexError):
        ops.moe_unpermute(out[:4], torch.tensor([0, -1, 1, 1], dtype=torch.int32, device=gpu), 3)
