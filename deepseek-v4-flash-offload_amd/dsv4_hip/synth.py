"""Seeded synthetic workloads for the routed-MoE layer (numpy on the host).

Distributions (same for every config):
  * packed E2M1 bytes uniform over 0..255 (both nibbles uniform over 0..15);
  * E8M0 scale bytes uniform over 117..127;
  * activations N(0, 1) rounded to bf16;
  * expert ids: Zipf(s=1.1) over expert ranks, a seeded rank -> expert
    permutation, K distinct experts per token drawn by Gumbel-top-k
    (Plackett-Luce sampling without replacement);
  * routing weights: softmax of N(0, 1) logits over the K picks (fp32);
  * shared expert: N(0, 2^-6) weights block-quantised to E4M3 with 128x128
    E8M0 scales 2^ceil(log2(amax / 448)) (the checkpoint's FP8 form).

Seeds: config-0 matrix rng(0) bytes / rng(1) scales / rng(2) x; experts
rng(100 + e); rank permutation rng(3); Gumbel noise rng(4); routing logits
rng(5); activations rng(6); offload drift rng(7 + layer).
"""

import numpy as np
import torch

ZIPF_S = 1.1


def packed_weight(rng, n, k):
    """([n, k/2] uint8 bytes, [n, k/32] uint8 E8M0 in 117..127)."""
    return (rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8),
            rng.integers(117, 128, size=(n, k // 32), dtype=np.uint8))


def expert_weights(e, hidden, inter):
    """Checkpoint-layout tensors of expert ``e`` (numpy): w1/w3 [I, D/2]+[I, D/32], w2 [D, I/2]+[D, I/32]."""
    rng = np.random.default_rng(100 + e)
    w1p, w1s = packed_weight(rng, inter, hidden)
    w3p, w3s = packed_weight(rng, inter, hidden)
    w2p, w2s = packed_weight(rng, hidden, inter)
    return {"w1p": w1p, "w1s": w1s, "w2p": w2p, "w2s": w2s, "w3p": w3p, "w3s": w3s}


def fp8_weight(rng, n, k, std=2.0 ** -6):
    """A block-quantised FP8 weight as checkpoints hold it: N(0, std) values, each
    128x128 block scaled by 2^ceil(log2(amax / 448)) and rounded to E4M3 (RNE).
    Returns ([n, k] uint8 E4M3 codes, [ceil(n/128), ceil(k/128)] uint8 E8M0)."""
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    nb, kb = (n + 127) // 128, (k + 127) // 128
    pad = np.zeros((nb * 128, kb * 128), np.float32)
    pad[:n, :k] = np.abs(w)
    amax = pad.reshape(nb, 128, kb, 128).max(axis=(1, 3))
    e = np.ceil(np.log2(np.maximum(amax, 1e-30) / 448.0)).astype(np.int32)
    s = np.repeat(np.repeat(np.ldexp(np.float32(1), e), 128, 0)[:n], 128, 1)[:, :k].astype(np.float32)
    codes = torch.from_numpy(w / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, (e + 127).astype(np.uint8)


def shared_expert_weights(seed, hidden, inter):
    """Shared expert in the checkpoint's FP8 form (numpy): w1/w3 [I, D] + [I/128, D/128],
    w2 [D, I] + [D/128, I/128] (E4M3 codes, E8M0 128x128 block scales)."""
    rng = np.random.default_rng(seed)
    w1, w1s = fp8_weight(rng, inter, hidden)
    w3, w3s = fp8_weight(rng, inter, hidden)
    w2, w2s = fp8_weight(rng, hidden, inter)
    return {"w1": w1, "w1s": w1s, "w2": w2, "w2s": w2s, "w3": w3, "w3s": w3s}


def bf16_normal(rng, shape):
    """N(0,1) as a bf16 torch tensor (RNE from fp32) on the host."""
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(torch.bfloat16)


def zipf_probs(n_experts, s=ZIPF_S):
    p = 1.0 / np.arange(1, n_experts + 1, dtype=np.float64) ** s
    return p / p.sum()


def rank_permutation(n_experts, seed=3):
    return np.random.default_rng(seed).permutation(n_experts)


def zipf_topk(T, K, n_experts, perm=None, rng=None, s=ZIPF_S):
    """[T, K] int64 expert ids, K distinct per token, Zipf over ranks."""
    if perm is None:
        perm = rank_permutation(n_experts)
    if rng is None:
        rng = np.random.default_rng(4)
    logp = np.log(zipf_probs(n_experts, s))
    g = rng.gumbel(size=(T, n_experts))
    ranks = np.argsort(-(logp[None, :] + g), axis=1, kind="stable")[:, :K]
    return perm[ranks].astype(np.int64)


def routing_weights(T, K, seed=5):
    z = np.random.default_rng(seed).standard_normal((T, K)).astype(np.float64)
    z = np.exp(z - z.max(axis=1, keepdims=True))
    return (z / z.sum(axis=1, keepdims=True)).astype(np.float32)


def layer_inputs(T, K=8, n_experts=256, hidden=4096):
    """(x bf16 [T, D] torch, topk_ids int64 [T, K] numpy, topk_w fp32 [T, K] numpy)."""
    ids = zipf_topk(T, K, n_experts, rank_permutation(n_experts, 3), np.random.default_rng(4))
    w = routing_weights(T, K, 5)
    x = bf16_normal(np.random.default_rng(6), (T, hidden))
    return x, ids, w


def dequant_config0():
    """Config-0 inputs: packed [2048, 2048], scales [2048, 128], x bf16 [1, 4096]."""
    packed = np.random.default_rng(0).integers(0, 256, size=(2048, 2048), dtype=np.uint8)
    scales = np.random.default_rng(1).integers(117, 128, size=(2048, 128), dtype=np.uint8)
    x = bf16_normal(np.random.default_rng(2), (1, 4096))
    return packed, scales, x


class DriftingZipf:
    """Per-layer Zipf routing whose hot set drifts slowly: every ``every`` steps,
    ``swaps`` random adjacent-rank swaps among ranks 0..127 (rng(7 + layer))."""

    def __init__(self, n_layers, n_experts=256, K=8, every=8, swaps=4, hot=128, seed_base=7):
        self.L, self.E, self.K = n_layers, n_experts, K
        self.every, self.swaps, self.hot = every, swaps, hot
        self.perms = [rank_permutation(n_experts, 3 + 1000 * l) for l in range(n_layers)]
        self.rngs = [np.random.default_rng(seed_base + l) for l in range(n_layers)]
        self.noise = [np.random.default_rng(10_000 + l) for l in range(n_layers)]
        self.logp = np.log(zipf_probs(n_experts))
        self.step_no = 0

    def step(self, T):
        """Routing of one decode step: list over layers of [T, K] int64 ids."""
        if self.step_no and self.step_no % self.every == 0:
            for l in range(self.L):
                for _ in range(self.swaps):
                    r = int(self.rngs[l].integers(0, self.hot - 1))
                    p = self.perms[l]
                    p[r], p[r + 1] = p[r + 1], p[r]
        out = []
        for l in range(self.L):
            g = self.noise[l].gumbel(size=(T, self.E))
            ranks = np.argsort(-(self.logp[None, :] + g), axis=1, kind="stable")[:, :self.K]
            out.append(self.perms[l][ranks].astype(np.int64))
        self.step_no += 1
        return out
