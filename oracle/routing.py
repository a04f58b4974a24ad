"""numpy restatement of the routed-MoE sort / gather / combine steps (test oracle only).

Follows ``dsv4_plugin/models/deepseek_v4.py`` of the reference:

* ``moe_align``  - flatten / argsort / bincount / nonzero, ``:155-164``. The
  reference's ``torch.argsort(flat_e)`` is not stable; the canonical order used
  here is the stable one (expert ascending, flat index ascending), which is
  what ``torch.argsort(stable=True)`` gives. On top of it the padded layout
  (each expert's rows padded up to a multiple of ``block_m``) used by the
  grouped GEMM is derived.
* ``permute``    - ``x_sorted = xq[row]``, ``:171`` / ``:213-214``.
* ``unpermute``  - ``y = zeros(fp32); y.index_add_(0, row, out.float());
  y.to(bf16)``, ``:195-197`` / ``:243-245`` (unweighted, fp32, in sorted order).
* ``route``      - ``OffloadDeepseekV4MoE._route``, ``:118-148``: fp32 gate
  logits, softmax / sigmoid / sqrt(softplus) scores, top-k of the biased scores
  (or the ``tid2eid`` row of each token on hash layers), the unbiased scores of
  the chosen experts as weights, renormalised and scaled. Computed in float64;
  ties in the top-k go to the lower expert id (``topk(sorted=False)`` leaves
  both the tie rule and the output order open).
"""

import numpy as np

from .mxfp4 import bf16_bits_to_f32, f32_to_bf16_bits


def moe_align(topk_ids, topk_weights, n_experts, block_m=64):
    """Returns a dict with the reference's views and the padded block layout.

    Reference views (deepseek_v4.py:155-164):
      order [R]      stable argsort of the flattened expert ids
      s_e, s_w [R]   sorted expert ids / routing weights
      row [R]        order // K (token of each sorted slot)
      counts [E]     bincount
      active [A]     experts with counts > 0 (ascending)
      group_list [A] counts[active]
    Padded layout (the grouped GEMM's M blocks):
      sorted_ids [P]     flat index t*K+k per padded slot, R for padding
      block_expert [P/block_m]
      num_post_padded    P
      expert_start [E]   first padded slot of each expert
    """
    ids = np.asarray(topk_ids).astype(np.int64)
    T, K = ids.shape
    R = T * K
    flat_e = ids.reshape(-1)
    flat_w = np.asarray(topk_weights, dtype=np.float32).reshape(-1)
    if R and (flat_e.min() < 0 or flat_e.max() >= n_experts):
        raise ValueError("expert id out of range")
    order = np.argsort(flat_e, kind="stable")
    s_e = flat_e[order]
    s_w = flat_w[order]
    row = order // K
    counts = np.bincount(flat_e, minlength=n_experts).astype(np.int64)
    active = np.nonzero(counts > 0)[0]
    group_list = counts[active]

    padded = ((counts + block_m - 1) // block_m) * block_m
    expert_start = np.concatenate([[0], np.cumsum(padded)[:-1]]).astype(np.int64)
    P = int(padded.sum())
    sorted_ids = np.full(P, R, dtype=np.int64)
    unpadded_start = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int64)
    for e in active:
        c = counts[e]
        sorted_ids[expert_start[e]:expert_start[e] + c] = order[unpadded_start[e]:unpadded_start[e] + c]
    block_expert = np.repeat(np.arange(n_experts), padded // block_m)
    return {
        "order": order, "s_e": s_e, "s_w": s_w, "row": row,
        "counts": counts, "active": active, "group_list": group_list,
        "sorted_ids": sorted_ids, "block_expert": block_expert,
        "num_post_padded": P, "expert_start": expert_start,
    }


def permute(x, row):
    """``x[row]`` (rows of any dtype)."""
    return np.asarray(x)[np.asarray(row)]


def unpermute(out_sorted_bf16, row, T):
    """``deepseek_v4.py:195-197``: fp32 zeros, ``index_add_`` in sorted order, bf16 cast.

    ``np.add.at`` applies the additions one index at a time in order, which is
    the order ``index_add_`` accumulates in."""
    out = bf16_bits_to_f32(out_sorted_bf16)
    D = out.shape[-1]
    y = np.zeros((T, D), dtype=np.float32)
    np.add.at(y, np.asarray(row), out)
    return f32_to_bf16_bits(y)


def _softplus(l):
    """``F.softplus`` (beta 1, threshold 20): ``l`` above the threshold, else
    ``log1p(exp(l))``."""
    with np.errstate(over="ignore"):
        return np.where(l > 20.0, l, np.log1p(np.exp(np.minimum(l, 20.0))))


def route(x_bf16, gate_w, topk, scoring="sqrtsoftplus", bias=None, renormalize=True,
          scale=1.5, tid2eid=None, input_ids=None):
    """``deepseek_v4.py:118-148`` in float64.

    ``x_bf16`` [T, D] bf16 bit patterns, ``gate_w`` [E, D] fp32. Returns
    ``(weights [T, K] float64, ids [T, K] int64, scores [T, E] float64)`` with the
    ids of a token in descending order of the biased score."""
    x = bf16_bits_to_f32(np.asarray(x_bf16, np.uint16)).astype(np.float64)
    logits = x @ np.asarray(gate_w, np.float32).astype(np.float64).T          # :125
    if scoring == "softmax":                                                  # :126-131
        e = np.exp(logits - logits.max(axis=-1, keepdims=True))
        scores = e / e.sum(axis=-1, keepdims=True)
    elif scoring == "sigmoid":
        scores = 1.0 / (1.0 + np.exp(-logits))
    elif scoring == "sqrtsoftplus":
        scores = np.sqrt(_softplus(logits))
    else:
        raise ValueError(f"unknown scoring function {scoring!r}")
    if tid2eid is not None:                                                   # :133-138
        if input_ids is None:
            raise RuntimeError("hash-layer routing needs input_ids")
        ids = np.asarray(tid2eid)[np.asarray(input_ids).astype(np.int64).reshape(-1)].astype(np.int64)
    else:                                                                     # :139-142
        choice = scores if bias is None else scores + np.asarray(bias, np.float32).astype(np.float64)
        ids = np.argsort(-choice, axis=-1, kind="stable")[:, :topk].astype(np.int64)
    w = np.take_along_axis(scores, ids, axis=1)                               # :144
    if renormalize:                                                           # :145-146
        w = w / w.sum(axis=-1, keepdims=True)
    return w * scale, ids, scores                                             # :147
