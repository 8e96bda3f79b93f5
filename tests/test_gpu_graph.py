"""The stack harness (moe_ffn.MoeStack): resident layers with their non-expert
Q4_0 projection and a Q4_0 router matrix, run back to back on one stream and
replayed from one captured HIP graph.

Checks:
  * the eager pipeline is wired right: each layer's projection output is
    bit-identical to the oracle's MMVQ-order matrix product of its input,
    its routes are the oracle router's on its logits, and sampled tokens of
    its output match the oracle layer on that projection output and those
    routes (1e-5 rms: grouped layers sum the down projection in the MFMA
    kernel's order);
  * every replay of the graph reproduces the eager outputs bit for bit, with
    eager launches on the same handles and synchronisations between replays
    (graph nodes must not depend on state the eager work changes);
  * the three layers take the decode path, the grouped path with both item
    kinds on two streams (fork / join inside the capture), and the grouped
    streaming path.
"""
import numpy as np
import pytest

import moe_ffn
import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
H, I, E, K = 2048, 512, 512, 10
TOKENS = (8, 8 + 1024, 300)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def stack():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    layers = [moe_ffn.MoeLayer(H, I, E, K, True, n, synthetic_seed=1100 + l) for l, n in enumerate(TOKENS)]
    rng = np.random.default_rng(1110)
    proj_w, router_w = [], []
    for l, n in enumerate(TOKENS):
        proj_w.append(W.q4_blocks(H * H // 32, rng).reshape(-1))
        router_w.append(W.q4_blocks(E * H // 32, rng).reshape(-1))
    projections = [moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, H, H, w, max_columns=n) for w, n in zip(proj_w, TOKENS)]
    routers = [moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, H, E, w, max_columns=n) for w, n in zip(router_w, TOKENS)]
    xs = [W.activations(n, seed=1120 + l) for l, n in enumerate(TOKENS)]
    S = moe_ffn.MoeStack(layers, projections=projections, routers=routers)
    S.bind([torch.from_numpy(x).cuda() for x in xs])
    yield dict(S=S, layers=layers, xs=xs, proj_w=proj_w, router_w=router_w)
    S.graph = None
    for m in layers + projections + routers:
        m.close()


def test_stack_eager_pipeline_vs_oracle(stack):
    S = stack["S"]
    S.run()
    assert int(host(S.error)[0]) == 0
    rng = np.random.default_rng(1130)
    for l, (L, st) in enumerate(zip(stack["layers"], S.steps)):
        x = stack["xs"][l]
        n = x.shape[0]
        h = host(st["h"])
        assert np.array_equal(bits(h), bits(O.matrix_gpu_order(stack["proj_w"][l], H, H, O.quantize_q8(x)))), l
        logits = host(st["logits"])
        assert np.array_equal(bits(logits), bits(O.matrix_gpu_order(stack["router_w"][l], H, E, O.quantize_q8(h))))
        prob, flags = O.router_softmax(logits)
        ids, w, flags2 = O.select_routes(prob, top_k=K)
        assert flags == 0 and flags2 == 0
        assert np.array_equal(host(st["ids"]), ids) and np.array_equal(bits(host(st["w"])), bits(w)), l
        sample = np.arange(n) if n <= 8 else rng.choice(n, 8, replace=False)
        mask = np.zeros(n, np.uint8)
        mask[sample] = 1
        used = sorted(set(int(e) for e in ids[sample].reshape(-1)))
        eb = moe_ffn.expert_bytes(H, I)
        bank = np.zeros(E * eb, np.uint8)
        for e in used:
            bank[e * eb:(e + 1) * eb] = L.export_expert(e)
        ref = O.moe_layer(h, H, I, E, bank, ids, w, shared_q4=L.export_expert(E), token_mask=mask)["y"]
        y = host(st["y"])
        err = float(np.max(np.abs(y[sample].astype(np.float64) - ref[sample])))
        scale = float(np.sqrt(np.mean(np.square(ref[sample].astype(np.float64)))))
        assert err <= 1e-5 * scale, (l, err, scale)


def test_stack_graph_replays_match_eager(stack):
    S = stack["S"]
    S.run()
    eager = [host(y).copy() for y in S.outputs()]
    assert int(host(S.error)[0]) == 0
    stats = [L.last_stats() for L in stack["layers"]]
    assert stats[1]["mfma_items"] > 0 and stats[1]["stream_items"] > 0   # both chains, two streams
    S.capture()
    for rep in range(3):
        for y in S.outputs():
            y.fill_(float("nan"))
        S.replay()
        torch.cuda.synchronize()
        for l, y in enumerate(S.outputs()):
            assert np.array_equal(bits(host(y)), bits(eager[l])), (rep, l)
        # eager work on the same handle between replays: a forward of a
        # different batch through layer 0 (its workspace and stats change)
        L0 = stack["layers"][0]
        xo = torch.from_numpy(W.activations(5, seed=1140 + rep)).cuda()
        io, wo = W.routes_uniform(5, seed=1150 + rep)
        L0.forward(xo, torch.from_numpy(io).cuda(), torch.from_numpy(wo).cuda())
        torch.cuda.synchronize()
    S.run()
    for l, y in enumerate(S.outputs()):
        assert np.array_equal(bits(host(y)), bits(eager[l])), ("eager after replays", l)
    assert int(host(S.error)[0]) == 0
