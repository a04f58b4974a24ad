"""The router restatement (``deepseek_v4.py:118-148``) pinned against torch's own
routines (``F.linear`` / ``softmax`` / ``sigmoid`` / ``softplus`` / ``topk`` in
float64) and against brute force over every K-subset on tiny inputs."""

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mxfp4 as Q
from oracle import routing as RT
from dsv4_hip import synth


def _inputs(T, D, E, seed):
    rng = np.random.default_rng(seed)
    x = synth.bf16_normal(rng, (T, D)).view(torch.int16).numpy().view(np.uint16)
    w = (rng.standard_normal((E, D)) * 0.03).astype(np.float32)
    b = (rng.standard_normal(E) * 0.1).astype(np.float32)
    return x, w, b


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid", "sqrtsoftplus"])
@pytest.mark.parametrize("renorm", [True, False])
def test_route_matches_torch_float64(scoring, renorm):
    T, D, E, K = 16, 256, 64, 6
    x, w, b = _inputs(T, D, E, 1)
    ow, oi, sc = RT.route(x, w, K, scoring, bias=b, renormalize=renorm, scale=1.5)
    xt = torch.from_numpy(Q.bf16_bits_to_f32(x)).double()
    g = F.linear(xt, torch.from_numpy(w).double())
    s = {"softmax": lambda v: v.softmax(-1), "sigmoid": torch.sigmoid,
         "sqrtsoftplus": lambda v: F.softplus(v).sqrt()}[scoring](g)
    np.testing.assert_allclose(sc, s.numpy(), rtol=1e-12, atol=1e-15)
    idx = torch.topk(s + torch.from_numpy(b).double(), K, dim=-1, sorted=True)[1]
    assert np.array_equal(oi, idx.numpy())
    ref = s.gather(1, idx)
    if renorm:
        ref = ref / ref.sum(-1, keepdim=True)
    np.testing.assert_allclose(ow, (ref * 1.5).numpy(), rtol=1e-12)


def test_softplus_threshold_follows_torch():
    v = np.array([-30.0, -1.0, 0.0, 19.5, 20.0, 20.5, 60.0, 100.0])
    np.testing.assert_allclose(RT._softplus(v), F.softplus(torch.from_numpy(v)).numpy(), rtol=1e-15)


def test_topk_is_the_best_subset_by_brute_force():
    T, D, E, K = 6, 64, 8, 3
    x, w, b = _inputs(T, D, E, 3)
    _, oi, sc = RT.route(x, w, K, "sigmoid", bias=b)
    c = sc + b.astype(np.float64)
    for t in range(T):
        best = max(itertools.combinations(range(E), K), key=lambda s: sum(c[t, list(s)]))
        assert sorted(best) == sorted(oi[t].tolist())
        assert all(c[t, oi[t, i]] >= c[t, oi[t, i + 1]] for i in range(K - 1))  # descending


def test_ties_go_to_the_lower_id_and_bias_only_chooses():
    D, E, K = 32, 16, 4
    x = np.zeros((1, D), np.uint16)                    # all logits 0 -> all scores equal
    w = np.zeros((E, D), np.float32)
    ow, oi, _ = RT.route(x, w, K, "sqrtsoftplus")
    assert oi[0].tolist() == [0, 1, 2, 3]
    np.testing.assert_allclose(ow, 1.5 / K)
    b = np.zeros(E, np.float32)
    b[[9, 3, 12, 5]] = [4.0, 3.0, 2.0, 1.0]            # bias picks; the weights stay unbiased
    ow, oi, _ = RT.route(x, w, K, "sqrtsoftplus", bias=b)
    assert oi[0].tolist() == [9, 3, 12, 5]
    np.testing.assert_allclose(ow, 1.5 / K)


def test_hash_layer_uses_the_table_row_of_each_token():
    T, D, E, K, V = 5, 64, 32, 4, 50
    x, w, _ = _inputs(T, D, E, 4)
    rng = np.random.default_rng(9)
    tab = np.stack([rng.permutation(E)[:K] for _ in range(V)]).astype(np.int32)
    ids = rng.integers(0, V, T)
    ow, oi, sc = RT.route(x, w, K, "sqrtsoftplus", tid2eid=tab, input_ids=ids, renormalize=False, scale=2.0)
    assert np.array_equal(oi, tab[ids])
    np.testing.assert_allclose(ow, 2.0 * np.take_along_axis(sc, tab[ids].astype(np.int64), 1))
    with pytest.raises(RuntimeError, match="input_ids"):
        RT.route(x, w, K, tid2eid=tab)
