"""Expert-parallel decomposition on one GPU: the layer split into shards of
experts gives the same bits as the whole layer.

Under G-way expert parallelism each GPU owns E/G experts.  It receives the
(token, rank) pairs routed to its experts as rows with one local route of
weight 1, and returns their unweighted contribution rows.  Each token's home
GPU then folds the ranks in order and adds the gated shared expert.  Here the
G shards run as separate layers on the one GPU.  The fold runs in the oracle
(the reference's rank-order fold with separately rounded products), and the
result must equal the whole layer's output bit for bit.  A contribution row
depends only on its pair's data, whatever tile or item the pair lands in.
Both grouped paths are checked: all groups on the int8-MFMA kernels, and all
groups streamed.
"""
import os

import numpy as np
import pytest

import moe_ffn
import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def layer_env(env, *args, **kw):
    """A layer created with the given MOE_FFN_* settings (read at creation)."""
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return moe_ffn.MoeLayer(*args, **kw)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.mark.parametrize("path", ["mfma", "stream"])
def test_expert_parallel_shares_compose_to_the_layer(path):
    H, I, E, K, N, G = 2048, 512, 64, 8, 192, 8
    env = {"MOE_FFN_DECODE": 0, "MOE_FFN_MFMA_MIN": 1 if path == "mfma" else 0}
    bank = W.q4_bank(E, seed=801)
    shared = W.q4_bank(1, seed=802)
    eb = bank.size // E
    x = W.activations(N, seed=803)
    ids, w = W.routes_zipf(N, 1.1, experts=E, k=K, seed=804)
    gate = np.random.default_rng(805).standard_normal(N).astype(np.float32)

    full = layer_env(env, H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
    y_full, err = full.forward(dev(x), dev(ids), dev(w), shared_gate=dev(gate))
    y_full, err = host(y_full), int(host(err)[0])
    full.close()
    assert err == 0

    contrib = np.full((N, K, H), np.nan, np.float32)
    for g in range(G):
        lo, hi = g * E // G, (g + 1) * E // G
        t, r = np.nonzero((ids >= lo) & (ids < hi))
        M = t.size
        assert M > 0
        share = layer_env(env, H, I, hi - lo, 1, False, M, experts_q4=bank[lo * eb:hi * eb])
        local = (ids[t, r] - lo).reshape(M, 1).astype(np.int32)
        rows, err_s = share.forward(dev(x[t]), dev(local), dev(np.ones((M, 1), np.float32)))
        assert int(host(err_s)[0]) == 0, g
        contrib[t, r] = host(rows)
        share.close()
    assert not np.isnan(contrib).any()   # every (token, rank) came back once

    sh_layer = layer_env(env, H, I, 1, 1, False, N, experts_q4=shared)
    sh, err_h = sh_layer.forward(dev(x), dev(np.zeros((N, 1), np.int32)), dev(np.ones((N, 1), np.float32)))
    sh = host(sh)
    sh_layer.close()
    assert int(host(err_h)[0]) == 0

    y_home, flags = O.combine_flags(contrib, w, shared=sh, shared_gate=gate)
    assert flags == 0
    assert np.array_equal(y_full.view(np.uint32), y_home.view(np.uint32))
