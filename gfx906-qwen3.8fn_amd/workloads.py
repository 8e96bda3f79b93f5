"""Seeded synthetic workloads for the routed-MoE expert FFN.

Weights: Q4_0 blocks (18 bytes: half d, 16 code bytes), d = half(|N(0, 0.02)|),
codes uniform 0..15 (low nibble = element j, high nibble = element j+16).
Q4_1 down blocks (20 bytes: half d, half m, 16 code bytes) take the same d and
codes with m = half(-8 d (0.75 + 0.5 u)), u uniform [0, 1), so values stay
centred about zero.
Activations: fp32 N(0, 1), token-major [N][H].
Routing: top-k distinct experts per token, weights = softmax of N(0,1) logits.
  uniform  - every expert equally likely
  zipf(s)  - expert popularity p(rank) ~ 1/rank^s over a seeded permutation of
             the experts, k distinct experts drawn per token without
             replacement by Gumbel-top-k
Ranks are ordered by the sampling key (rank 0 = strongest), as the reference's
select_routes orders them by probability (src/session.hip:666-687).
"""
from __future__ import annotations

import numpy as np

H, I, E, TOP_K = 2048, 512, 512, 10
Q4_BLOCK = 18
Q4_1_BLOCK = 20


def expert_bytes(hidden=H, intermediate=I, down_type=0):
    """Canonical bytes of one expert (down_type 1: Q4_1 down blocks)."""
    return hidden // 32 * intermediate * (2 * Q4_BLOCK + (Q4_1_BLOCK if down_type == 1 else Q4_BLOCK))


def q4_blocks(nblocks, rng):
    """nblocks canonical Q4_0 blocks as uint8 [nblocks, 18]."""
    out = np.empty((nblocks, Q4_BLOCK), np.uint8)
    d = np.abs(rng.standard_normal(nblocks, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    out[:, :2] = d.view(np.uint8).reshape(nblocks, 2)
    out[:, 2:] = rng.integers(0, 256, (nblocks, 16), dtype=np.uint8)
    return out


def q4_1_blocks(nblocks, rng):
    """nblocks canonical Q4_1 blocks as uint8 [nblocks, 20]."""
    q4 = q4_blocks(nblocks, rng)
    d = q4[:, :2].copy().view(np.float16).astype(np.float32).reshape(nblocks)
    m = (-8.0 * d * (0.75 + 0.5 * rng.random(nblocks, dtype=np.float32))).astype(np.float16)
    out = np.empty((nblocks, Q4_1_BLOCK), np.uint8)
    out[:, :2] = q4[:, :2]
    out[:, 2:4] = m.view(np.uint8).reshape(nblocks, 2)
    out[:, 4:] = q4[:, 2:]
    return out


def q4_bank(n_experts, hidden=H, intermediate=I, seed=0, down_type=0):
    """n_experts experts, each [gate I x H/32 | up I x H/32 | down H x I/32]
    blocks; down_type 1 makes the down blocks Q4_1."""
    rng = np.random.default_rng(seed)
    mb = (hidden // 32) * intermediate
    if down_type != 1:
        return q4_blocks(n_experts * 3 * mb, rng).reshape(-1)
    gu = q4_blocks(n_experts * 2 * mb, rng).reshape(n_experts, -1)
    dn = q4_1_blocks(n_experts * mb, rng).reshape(n_experts, -1)
    return np.ascontiguousarray(np.concatenate([gu, dn], axis=1)).reshape(-1)


def activations(tokens, hidden=H, seed=0):
    return np.random.default_rng(seed).standard_normal((tokens, hidden), dtype=np.float32)


def _softmax_weights(rng, tokens, k):
    logits = rng.standard_normal((tokens, k), dtype=np.float32)
    z = np.exp(logits - logits.max(axis=1, keepdims=True))
    return (z / z.sum(axis=1, keepdims=True)).astype(np.float32)


def routes_uniform(tokens, experts=E, k=TOP_K, seed=0):
    rng = np.random.default_rng(seed)
    keys = rng.random((tokens, experts), dtype=np.float32)
    ids = np.argpartition(keys, -k, axis=1)[:, -k:]
    order = np.argsort(-np.take_along_axis(keys, ids, axis=1), axis=1, kind="stable")
    ids = np.take_along_axis(ids, order, axis=1).astype(np.int32)
    return np.ascontiguousarray(ids), _softmax_weights(rng, tokens, k)


def routes_zipf(tokens, s, experts=E, k=TOP_K, seed=0):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(experts)
    logp = np.empty(experts, np.float64)
    logp[perm] = -s * np.log(np.arange(1, experts + 1, dtype=np.float64))
    ids = np.empty((tokens, k), np.int32)
    chunk = 2048
    for t0 in range(0, tokens, chunk):
        n = min(chunk, tokens - t0)
        g = rng.gumbel(size=(n, experts))
        keys = logp[None, :] + g
        sel = np.argpartition(keys, -k, axis=1)[:, -k:]
        order = np.argsort(-np.take_along_axis(keys, sel, axis=1), axis=1, kind="stable")
        ids[t0:t0 + n] = np.take_along_axis(sel, order, axis=1)
    return ids, _softmax_weights(rng, tokens, k)


def group_histogram(ids, experts=E):
    counts = np.bincount(ids.reshape(-1), minlength=experts)
    nz = counts[counts > 0]
    return dict(touched=int((counts > 0).sum()), min=int(nz.min()), median=float(np.median(nz)),
                max=int(nz.max()), ge16=int((counts >= 16).sum()), ge128=int((counts >= 128).sum()))


# name -> (tokens, routing, kwargs).  Config numbers follow BASELINE.json configs[].
CONFIGS = {
    "single_expert_n8": dict(tokens=8, experts=1, routing=None),                 # configs[0]
    "b8_decode": dict(tokens=8, experts=E, routing=("uniform", {})),             # configs[1]
    "prefill_4k_zipf1.1": dict(tokens=4096, experts=E, routing=("zipf", {"s": 1.1})),   # configs[2]
    "prefill_16k_uniform": dict(tokens=16384, experts=E, routing=("uniform", {})),      # configs[3]
    "stack48_mixed_zipf1.3": dict(tokens=8 + 1024, experts=E, routing=("zipf", {"s": 1.3}), layers=48),  # configs[4]
}


def routes_for(name, seed=0, tokens=None):
    cfg = CONFIGS[name]
    n = tokens or cfg["tokens"]
    kind, kw = cfg["routing"]
    if kind == "uniform":
        return routes_uniform(n, seed=seed)
    return routes_zipf(n, kw["s"], seed=seed)


def algorithmic_bytes(tokens, touched, shared=True, hidden=H, intermediate=I, k=TOP_K, down_type=0):
    """Bytes a layer must move at minimum: touched experts' weights (+shared),
    fp32 x in and y out, int32 ids + fp32 weights."""
    return (touched + (1 if shared else 0)) * expert_bytes(hidden, intermediate, down_type) + \
        tokens * hidden * 4 * 2 + tokens * k * 8


def int8_ops(tokens, shared=True, hidden=H, intermediate=I, k=TOP_K):
    """2 ops per multiply-add over the three projections of every routed pair."""
    return 2 * 3 * hidden * intermediate * tokens * (k + (1 if shared else 0))
