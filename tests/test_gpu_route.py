"""GPU parity: the router (``dsv4_moe_route``, ``deepseek_v4.py:118-148``) against
the float64 oracle.

The logits are fp32 sums on the GPU and float64 in the oracle, so the weights
are compared with a tolerance (rtol 2e-5) and the chosen ids are compared where
the oracle's biased scores leave no doubt: a pick whose neighbours in the sorted
order lie within 1e-5 of it may legitimately swap places (the reference's
``topk(sorted=False)`` leaves the order open anyway), and a token whose K-th and
(K+1)-th scores lie within 1e-5 may pick either. Such tokens are counted and
must stay rare."""

import numpy as np
import pytest
import torch

from oracle import routing as RT
from dsv4_hip import ops, synth

pytestmark = pytest.mark.gpu

GAP = 1e-5


def _inputs(T, D, E, seed, xdtype):
    rng = np.random.default_rng(seed)
    xb = synth.bf16_normal(rng, (T, D))                    # bf16 torch tensor
    w = (rng.standard_normal((E, D)) * 0.03).astype(np.float32)
    b = (rng.standard_normal(E) * 0.1).astype(np.float32)
    if xdtype == "fp32":  # fp32 hidden states with more than bf16 precision
        xf = xb.float() + torch.from_numpy((rng.standard_normal((T, D)) * 1e-3).astype(np.float32))
        return xf, w, b
    return xb, w, b


def _oracle(x, w, K, scoring, bias, renorm, scale, **kw):
    if x.dtype == torch.float32:
        # the oracle takes bf16 bits; fp32 hidden states go through the same float64 steps here
        xf = x.double().numpy()
        logits = xf @ w.astype(np.float64).T
        return _finish(logits, K, scoring, bias, renorm, scale)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    return RT.route(bits, w, K, scoring, bias=bias, renormalize=renorm, scale=scale, **kw)


def _finish(logits, K, scoring, bias, renorm, scale):
    if scoring == "softmax":
        e = np.exp(logits - logits.max(-1, keepdims=True))
        s = e / e.sum(-1, keepdims=True)
    elif scoring == "sigmoid":
        s = 1.0 / (1.0 + np.exp(-logits))
    else:
        s = np.sqrt(RT._softplus(logits))
    c = s if bias is None else s + bias.astype(np.float64)
    ids = np.argsort(-c, axis=-1, kind="stable")[:, :K]
    wts = np.take_along_axis(s, ids, 1)
    if renorm:
        wts = wts / wts.sum(-1, keepdims=True)
    return wts * scale, ids, s


def _check(out_w, out_ids, ref_w, ref_ids, scores, bias, K):
    T = ref_ids.shape[0]
    c = scores if bias is None else scores + bias.astype(np.float64)
    cs = -np.sort(-c, axis=-1)
    ambiguous = 0
    for t in range(T):
        if K < c.shape[1] and cs[t, K - 1] - cs[t, K] <= GAP:
            ambiguous += 1
            continue
        assert sorted(out_ids[t].tolist()) == sorted(ref_ids[t].tolist()), t
        for k in range(K):
            lo = cs[t, k] - cs[t, k + 1] if k + 1 < c.shape[1] else np.inf
            hi = cs[t, k - 1] - cs[t, k] if k > 0 else np.inf
            if min(lo, hi) > GAP:
                assert out_ids[t, k] == ref_ids[t, k], (t, k)
        # weights follow the ids the kernel chose
        order = np.argsort(out_ids[t])
        ref_order = np.argsort(ref_ids[t])
        np.testing.assert_allclose(out_w[t, order], ref_w[t, ref_order], rtol=2e-5, atol=1e-7)
    assert ambiguous <= max(2, T // 100), ambiguous


@pytest.mark.parametrize("T,D,E,K,scoring,use_bias,renorm,xdtype", [
    (8, 4096, 256, 8, "sqrtsoftplus", True, True, "bf16"),     # decode
    (64, 4096, 256, 8, "softmax", True, True, "bf16"),
    (2048, 4096, 256, 8, "sigmoid", False, True, "bf16"),      # prefill: 8-wave groups over 256 experts, x in LDS
    (512, 2048, 256, 8, "softmax", True, True, "fp32"),        # the same with fp32 x
    (256, 1024, 96, 6, "sqrtsoftplus", True, True, "bf16"),    # 64x32 tiles per wave, 512-k chunks, loads 3 steps ahead
    (256, 768, 64, 4, "sigmoid", False, True, "fp32"),         # 64x32 tiles, a 768-k chunk: one step ahead
    (1, 4096, 256, 6, "sqrtsoftplus", True, True, "fp32"),
    (37, 1024, 48, 5, "softmax", False, True, "fp32"),         # E not a multiple of 64, ragged T
    (300, 2048, 512, 8, "sqrtsoftplus", True, False, "bf16"),
    (5, 512, 16, 16, "sigmoid", True, True, "bf16"),           # K = E
    (129, 4096, 256, 1, "softmax", True, True, "bf16"),        # K = 1
])
def test_route_matches_oracle(gpu, T, D, E, K, scoring, use_bias, renorm, xdtype):
    x, w, b = _inputs(T, D, E, T + E + K, xdtype)
    bias = b if use_bias else None
    ref_w, ref_ids, sc = _oracle(x, w, K, scoring, bias, renorm, 1.5)
    out_w, out_ids = ops.route(x.to(gpu), torch.from_numpy(w).to(gpu), K, scoring,
                               bias=None if bias is None else torch.from_numpy(bias).to(gpu),
                               renormalize=renorm, scale=1.5)
    torch.cuda.synchronize()
    assert out_ids.dtype == torch.int32 and out_ids.shape == (T, K) and out_w.shape == (T, K)
    _check(out_w.cpu().numpy(), out_ids.cpu().numpy(), ref_w, ref_ids, sc, bias, K)


@pytest.mark.parametrize("tab_dtype", [torch.int32, torch.int64])
def test_route_hash_layer_and_bad_ids(gpu, tab_dtype):
    T, D, E, K, V = 12, 4096, 256, 6, 1000
    x, w, _ = _inputs(T, D, E, 7, "bf16")
    rng = np.random.default_rng(8)
    tab = np.stack([rng.permutation(E)[:K] for _ in range(V)]).astype(np.int64)
    ids = rng.integers(0, V, T)
    ref_w, ref_ids, _ = RT.route(x.view(torch.int16).numpy().view(np.uint16), w, K, "sqrtsoftplus",
                                 tid2eid=tab, input_ids=ids)
    tab_d = torch.from_numpy(tab).to(tab_dtype).to(gpu)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    out_w, out_ids = ops.route(x.to(gpu), torch.from_numpy(w).to(gpu), K, "sqrtsoftplus", tid2eid=tab_d,
                               input_ids=torch.from_numpy(ids).to(gpu), status=status)
    torch.cuda.synchronize()
    assert np.array_equal(out_ids.cpu().numpy(), ref_ids)   # table order, bit-exact ids
    np.testing.assert_allclose(out_w.cpu().numpy(), ref_w, rtol=2e-5)
    assert int(status.item()) == 0
    # an input id outside the vocabulary and a table entry outside [0, E)
    bad_ids = ids.copy()
    bad_ids[3] = V + 5
    tab[ids[5], 2] = E + 7
    tab_d = torch.from_numpy(tab).to(tab_dtype).to(gpu)
    out_w, out_ids = ops.route(x.to(gpu), torch.from_numpy(w).to(gpu), K, "sqrtsoftplus", tid2eid=tab_d,
                               input_ids=torch.from_numpy(bad_ids).to(gpu), status=status)
    torch.cuda.synchronize()
    oi, ow = out_ids.cpu().numpy(), out_w.cpu().numpy()
    assert np.all(oi[3] == -1) and np.all(ow[3] == 0)
    assert oi[5, 2] == -1 and ow[5, 2] == 0
    assert int(status.item()) == 2
    good = [t for t in range(T) if t not in (3, 5)]
    assert np.array_equal(oi[good], ref_ids[good])
