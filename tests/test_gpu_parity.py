"""GPU parity of the HIP path (libmoe_ffn.so, called through the C ABI) against
the CPU oracle and the reference-produced golden fixtures.

Bars:
  * Q8_1 activation / middle codes and headers: bit-exact;
  * per-block int32 Q4 x Q8 dot sums: bit-exact;
  * route grouping and the rank-order fold: bit-exact;
  * fp32 FFN outputs: max |gpu - ref| <= 1e-3 * rms(ref).
"""
import os

import numpy as np
import pytest

import moe_ffn
import oracle as O
import workloads as W
from golden_inputs import expert_weights, route_cases

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
DEV = "cuda:0"
TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def rms(a):
    return float(np.sqrt(np.mean(np.square(np.asarray(a, np.float64)))))


def assert_close(got, ref, tol=TOL, what=""):
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))
    assert err <= tol * rms(ref), f"{what}: max abs err {err:.3e} > {tol} * rms {rms(ref):.3e}"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_bytes(q):
    return np.ascontiguousarray(q).view(np.uint8).reshape(-1)


def layer_parity(L, x, ids, w, bank, shared, y_gpu, sample, what, H=2048, I=512):
    """Parity of a whole-layer forward on the tokens `sample`:
      1. x Q8 bytes equal to the reference quantizer's;
      2. every middle Q8 row (grouped order, from debug_last) equal byte for
         byte to the oracle's cpu_expert middle of that (token, expert) --
         the gate/up kernels follow the reference's fp32 order and expf, so
         this is exact, not a tolerance;
      3. the output within 1e-5 rms of the oracle's whole layer (the down
         projection sums its blocks in the kernel's own order; the north_star
         bar is 1e-3 rms)."""
    N, E = x.shape[0], L.E
    nbi = I // 32
    dbg = L.debug_last(N)
    mid = host(dbg["middle_q8"]).reshape(-1, nbi, 36)
    mask = np.zeros(N, np.uint8)
    mask[sample] = 1
    ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, token_mask=mask)
    assert np.array_equal(host(dbg["x_q8"]).reshape(N, -1)[sample], q8_bytes(ref["x_q8"]).reshape(N, -1)[sample])
    groups = O.route_groups(ids, w, E)
    P = int(groups["offsets"][-1])
    eb = len(bank) // E
    mb = eb // 3
    xq = O.quantize_q8(x[sample])
    pos = {int(t): i for i, t in enumerate(sample)}

    def oracle_middle(e_bytes, t):
        ro = O.expert_forward(e_bytes[:mb], e_bytes[mb:2 * mb], e_bytes[2 * mb:], H, I, xq[pos[t]:pos[t] + 1])
        return q8_bytes(ro["middle_q8"]).reshape(nbi, 36)

    for p in range(P):
        t = int(groups["token"][p])
        if t in pos:
            e = int(groups["expert"][p])
            assert np.array_equal(mid[p], oracle_middle(bank[e * eb:(e + 1) * eb], t)), f"{what}: middle of pair {p}"
    for t in sample:
        assert np.array_equal(mid[P + int(t)], oracle_middle(shared, int(t))), f"{what}: shared middle of {t}"
    assert_close(y_gpu[sample], ref["y"][sample], tol=1e-5, what=what)


@pytest.fixture(scope="module", autouse=True)
def gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"\n[gpu] {torch.cuda.get_device_name(0)}", flush=True)
    yield
    torch.cuda.synchronize()


# ------------------------------------------------------------- quantizer ---
def test_quantize_reference_fixture_and_flags():
    f = np.load(os.path.join(GOLDEN, "quant_q8.npz"), allow_pickle=False)
    blocks = f["inputs"]
    q8, err = moe_ffn.quantize_q8_1(dev(blocks.reshape(1, -1)))
    got = host(q8).reshape(len(blocks), 36)
    ok = f["status"] == 0
    assert np.array_equal(got[ok], f["q8"][ok])
    assert np.all(got[~ok] == 0)
    assert int(host(err)[0]) != 0


def test_quantize_random_bit_exact():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((64, 2048)) * np.exp2(rng.integers(-20, 12, (64, 1)))).astype(np.float32)
    q8, err = moe_ffn.quantize_q8_1(dev(x))
    assert np.array_equal(host(q8).reshape(-1), q8_bytes(O.quantize_q8(x)))
    assert int(host(err)[0]) == 0


# ------------------------------------------------------ single expert -----
def _single_expert(H, I, weights, columns):
    bank = np.concatenate(weights)
    return moe_ffn.MoeLayer(H, I, 1, 1, False, columns, experts_q4=bank)


@pytest.fixture(scope="module")
def cfg0():
    """one expert, H 2048, I 512, 8 tokens."""
    bank = W.q4_bank(1, seed=11)
    mb = len(bank) // 3
    g, u, d = bank[:mb], bank[mb:2 * mb], bank[2 * mb:]
    layer = moe_ffn.MoeLayer(2048, 512, 1, 1, False, 8, experts_q4=bank)
    x = W.activations(8, seed=12)
    xq = O.quantize_q8(x)
    ref = O.expert_forward(g, u, d, 2048, 512, xq, avx2=True)
    return dict(layer=layer, g=g, u=u, d=d, x=x, xq=xq, ref=ref)


def test_cfg0_gate_up_block_dots_bit_exact(cfg0):
    r = cfg0["layer"].expert_gate_up(0, dev(q8_bytes(cfg0["xq"]).reshape(8, -1)), 8, path=moe_ffn.PATH_STREAM,
                                     dots=True)
    assert np.array_equal(host(r["gate_dots"]), O.block_dots(cfg0["g"], 2048, 512, cfg0["xq"]))
    assert np.array_equal(host(r["up_dots"]), O.block_dots(cfg0["u"], 2048, 512, cfg0["xq"]))
    assert int(host(r["error"])[0]) == 0


def test_cfg0_middle_and_middle_q8(cfg0):
    """Streaming path (H <= 2048): gate/up in the reference's fp32 order and
    expf, so the middle and its Q8 are bit-identical to the CPU reference's."""
    r = cfg0["layer"].expert_gate_up(0, dev(q8_bytes(cfg0["xq"]).reshape(8, -1)), 8, path=moe_ffn.PATH_STREAM)
    middle = host(r["middle"])
    assert np.array_equal(middle.view(np.uint32), cfg0["ref"]["middle"].view(np.uint32))
    assert np.array_equal(host(r["middle_q8"]).reshape(-1), q8_bytes(cfg0["ref"]["middle_q8"]))


def test_cfg0_down_block_dots_and_projection(cfg0):
    mq = cfg0["ref"]["middle_q8"]
    r = cfg0["layer"].expert_down(0, dev(q8_bytes(mq).reshape(8, -1)), 8, path=moe_ffn.PATH_STREAM, dots=True)
    assert np.array_equal(host(r["down_dots"]), O.block_dots(cfg0["d"], 512, 2048, mq))
    ref = O.matrix_gpu_order(cfg0["d"], 512, 2048, mq)
    assert_close(host(r["y"]), ref, tol=1e-5, what="down projection")


def test_cfg0_expert_pipeline(cfg0):
    L = cfg0["layer"]
    r = L.expert_gate_up(0, dev(q8_bytes(cfg0["xq"]).reshape(8, -1)), 8)
    y = L.expert_down(0, r["middle_q8"], 8)["y"]
    assert_close(host(y), cfg0["ref"]["y"], what="expert output")


def test_reference_shape_expert_vs_golden():
    """The reference's own CPU expert output at its fixed 2560/640 shape."""
    f = np.load(os.path.join(GOLDEN, "cpu_expert_2560x640.npz"), allow_pickle=False)
    g, u, d = expert_weights(2560, 640)
    layer = _single_expert(2560, 640, (g, u, d), 3)
    xq = f["x_q8"].reshape(3, -1)
    # H = 2560 > 2048: the wide streaming kernel (lanes holding two blocks),
    # in the reference's fp32 order: the middle is the reference's, bit for bit.
    r = layer.expert_gate_up(0, dev(xq), 3, path=moe_ffn.PATH_STREAM, dots=True)
    assert np.array_equal(host(r["gate_dots"]), O.block_dots(g, 2560, 640, xq))
    assert np.array_equal(host(r["middle"]).view(np.uint32), f["middle"].view(np.uint32))
    assert np.array_equal(host(r["middle_q8"]).reshape(-1), f["middle_q8"].reshape(-1))
    # I = 640: the lean down kernel with two blocks per lane, also in the
    # reference's order: the output is the reference's, bit for bit.
    y = layer.expert_down(0, r["middle_q8"], 3, path=moe_ffn.PATH_STREAM)["y"]
    assert np.array_equal(host(y).view(np.uint32), f["y"].view(np.uint32))
    layer.close()


# ---------------------------------------------------------- grouping -------
@pytest.fixture(scope="module")
def router_layer():
    return moe_ffn.MoeLayer(2048, 512, 512, 10, True, 2048, synthetic_seed=3)


def _check_groups(got, ref):
    assert np.array_equal(host(got["counts"]), ref["counts"])
    assert np.array_equal(host(got["offsets"]), np.concatenate([[0], np.cumsum(ref["counts"])]))
    assert np.array_equal(host(got["token"]), ref["token"])
    assert np.array_equal(host(got["rank"]), ref["rank"])


@pytest.mark.parametrize("name", ["pattern_n1", "pattern_n7", "pattern_n64", "pattern_n1024", "random_n300"])
def test_group_routes_reference_fixture(router_layer, name):
    f = np.load(os.path.join(GOLDEN, "routes.npz"), allow_pickle=False)
    ids, w = route_cases()[name]
    got = router_layer.group_routes(dev(ids), dev(w))
    ref = {k: f[f"{name}_{k}"] for k in ("token", "rank", "counts")}
    _check_groups(got, ref)
    assert int(host(got["error"])[0]) == 0


@pytest.mark.parametrize("tokens,kind", [(8, "uniform"), (256, "zipf"), (257, "zipf"), (2048, "zipf")])
def test_group_routes_vs_oracle(router_layer, tokens, kind):
    ids, w = W.routes_uniform(tokens, seed=tokens) if kind == "uniform" else W.routes_zipf(tokens, 1.1, seed=tokens)
    got = router_layer.group_routes(dev(ids), dev(w))
    _check_groups(got, O.route_groups(ids, w, 512))


@pytest.mark.parametrize("name", ["duplicate", "bad_id", "negative_weight"])
def test_group_routes_invalid_inputs_flag(router_layer, name):
    ids, w = route_cases()[name]
    got = router_layer.group_routes(dev(ids), dev(w))
    assert int(host(got["error"])[0]) & 1


# ------------------------------------------------------------- fold --------
def test_combine_bit_exact():
    rng = np.random.default_rng(4)
    c = rng.standard_normal((33, 10, 2048), dtype=np.float32)
    w = rng.random((33, 10), dtype=np.float32)
    y, err = moe_ffn.combine(dev(c), dev(w))
    assert np.array_equal(host(y).view(np.uint32), O.routed_fold(c, w).view(np.uint32))
    s = rng.standard_normal((33, 2048), dtype=np.float32)
    y2, _ = moe_ffn.combine(dev(c), dev(w), shared=dev(s))
    assert np.array_equal(host(y2), (O.routed_fold(c, w) + s).astype(np.float32))
    g = rng.standard_normal(33, dtype=np.float32)
    y3, _ = moe_ffn.combine(dev(c), dev(w), shared=dev(s), shared_gate=dev(g))
    sig = (1.0 / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32)
    assert_close(host(y3), O.routed_fold(c, w) + sig[:, None] * s, tol=1e-6, what="sigmoid shared add")
    assert int(host(err)[0]) == 0


@pytest.mark.parametrize("gated", [False, True])
def test_combine_flags_match_two_kernel_sequence(gated):
    """Nonfinite operands and overflowing products in the fold: the routed
    value is zeroed where the routed fold flags, the shared add starts from
    it with flags of its own (the reference's routed_fold, then
    shared_sigmoid_add).  Output bits and the error word equal the oracle's."""
    rng = np.random.default_rng(44)
    T, K, H = 6, 10, 256
    c = rng.standard_normal((T, K, H), dtype=np.float32)
    w = rng.random((T, K), dtype=np.float32)
    s = rng.standard_normal((T, H), dtype=np.float32)
    c[1, 3, 7] = np.nan
    c[2, 0, 9] = np.inf
    c[3, 5, 11] = np.float32(3e38)
    w[3, 5] = 8.0
    s[4, 13] = np.nan
    s[1, 7] = -np.inf
    g = rng.standard_normal(T).astype(np.float32) if gated else None
    if gated:
        g[5] = np.nan
    y, err = moe_ffn.combine(dev(c), dev(w), shared=dev(s), shared_gate=None if g is None else dev(g))
    ref, flags = O.combine_flags(c, w, shared=s, shared_gate=g)
    assert np.array_equal(host(y).view(np.uint32), ref.view(np.uint32))
    assert int(host(err)[0]) == flags == 3
    y2, err2 = moe_ffn.combine(dev(c), dev(w))
    ref2, flags2 = O.combine_flags(c, w)
    assert np.array_equal(host(y2).view(np.uint32), ref2.view(np.uint32))
    assert int(host(err2)[0]) == flags2


# -------------------------------------------------------- whole layer ------
@pytest.fixture(scope="module")
def moe512():
    bank = W.q4_bank(512, seed=21)
    shared = W.q4_bank(1, seed=22)
    layer = moe_ffn.MoeLayer(2048, 512, 512, 10, True, 4096, experts_q4=bank, shared_q4=shared)
    return dict(layer=layer, bank=bank, shared=shared)


def test_b8_decode_forward(moe512):
    """8 tokens, uniform top-10 of 512, + shared expert."""
    x = W.activations(8, seed=31)
    ids, w = W.routes_uniform(8, seed=32)
    L = moe512["layer"]
    y, err = L.forward(dev(x), dev(ids), dev(w))
    ref = O.moe_layer(x, 2048, 512, 512, moe512["bank"], ids, w, shared_q4=moe512["shared"])
    # The decode path follows the reference's fp32 order in every projection
    # and its fold: the layer output is bit-identical to the CPU reference's.
    assert np.array_equal(host(y).view(np.uint32), ref["y"].view(np.uint32))
    assert int(host(err)[0]) == 0
    dbg = L.debug_last(8)
    assert np.array_equal(host(dbg["x_q8"]).reshape(-1), q8_bytes(ref["x_q8"]))
    groups = O.route_groups(ids, w, 512)
    assert np.array_equal(host(dbg["route_token"]), groups["token"])
    assert np.array_equal(host(dbg["route_rank"]), groups["rank"])


def test_b8_decode_forward_shared_gate(moe512):
    x = W.activations(8, seed=41)
    ids, w = W.routes_uniform(8, seed=42)
    g = np.random.default_rng(43).standard_normal(8).astype(np.float32)
    y, err = moe512["layer"].forward(dev(x), dev(ids), dev(w), shared_gate=dev(g))
    ref = O.moe_layer(x, 2048, 512, 512, moe512["bank"], ids, w, shared_q4=moe512["shared"], shared_gate=g)
    assert np.array_equal(host(y).view(np.uint32), ref["y"].view(np.uint32))
    assert int(host(err)[0]) == 0


def test_prefill_4k_zipf_sampled_tokens(moe512):
    """4096 tokens, Zipf(1.1) top-10.  The whole layer runs
    on the GPU; the oracle checks a seeded sample of 24 tokens (each token's
    output depends only on its own routes), plus size-independent properties."""
    x = W.activations(4096, seed=51)
    ids, w = W.routes_zipf(4096, 1.1, seed=52)
    L = moe512["layer"]
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    sample = np.random.default_rng(53).choice(4096, 24, replace=False)
    layer_parity(L, x, ids, w, moe512["bank"], moe512["shared"], yh, sample, "4K prefill")


def test_prefill_16k_uniform_sampled_tokens(moe512):
    """16384 tokens, uniform top-10 (every group ~320
    wide, all on the MFMA path).  Sampled tokens against the oracle, plus
    determinism of the whole output."""
    L = moe_ffn.MoeLayer(2048, 512, 512, 10, True, 16384, experts_q4=moe512["bank"], shared_q4=moe512["shared"])
    x = W.activations(16384, seed=56)
    ids, w = W.routes_uniform(16384, seed=57)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    st = L.last_stats()
    assert st["stream_items"] == 0 and st["mfma_items"] > 0 and st["active_experts"] == 513
    sample = np.random.default_rng(58).choice(16384, 16, replace=False)
    layer_parity(L, x, ids, w, moe512["bank"], moe512["shared"], yh, sample, "16K prefill")
    y2, _ = L.forward(dev(x), dev(ids), dev(w))
    assert np.array_equal(host(y2), yh)
    L.close()


def test_max_tokens_layer(moe512):
    """The largest batch a layer takes (max_tokens = 65536, Zipf(1.1) top-10):
    its contribution buffer (65536 x 11 x 2048 fp32, 5.9 GB) is past 2^32
    bytes, so 32-bit offsets anywhere in the grouped path would show here.
    The first, last and sampled tokens against the oracle (middle Q8 rows
    byte-equal, outputs within 1e-5 rms), then determinism of the whole
    output."""
    N = 65536
    L = moe_ffn.MoeLayer(2048, 512, 512, 10, True, N, experts_q4=moe512["bank"], shared_q4=moe512["shared"])
    x = W.activations(N, seed=59)
    ids, w = W.routes_zipf(N, 1.1, seed=60)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    st = L.last_stats()
    assert st["mfma_items"] > 0 and st["active_experts"] == 513
    sample = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(61).choice(N, 6, replace=False)]))
    layer_parity(L, x, ids, w, moe512["bank"], moe512["shared"], yh, sample, "65536-token layer")
    y2, _ = L.forward(dev(x), dev(ids), dev(w))
    assert np.array_equal(host(y2), yh)
    L.close()


@pytest.mark.parametrize("path", ["mfma", "stream"])
def test_top_k_32_layer(path):
    """The largest top-k a layer takes (32, half of 64 experts per token, +
    shared): 33 routes per token are more than the decode kernels fold (16),
    so the grouped path runs, and the fold takes its ranks in four chunks of
    eight.  Sampled tokens against the oracle (middle Q8 rows byte-equal,
    outputs within 1e-5 rms; bit-identical on the streaming path)."""
    H, I, E, K, N = 2048, 512, 64, 32, 96
    env = {"MOE_FFN_MFMA_MIN": 1 if path == "mfma" else 0}
    bank = W.q4_bank(E, seed=901)
    shared = W.q4_bank(1, seed=902)
    L = _layer_env(env, H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
    x = W.activations(N, seed=903)
    ids, w = W.routes_zipf(N, 1.1, experts=E, k=K, seed=904)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    st = L.last_stats()
    assert (st["mfma_items"] > 0) == (path == "mfma")
    sample = np.random.default_rng(905).choice(N, 12, replace=False)
    layer_parity(L, x, ids, w, bank, shared, yh, sample, f"top-32 layer, {path} path")
    if path == "stream":
        mask = np.zeros(N, np.uint8)
        mask[sample] = 1
        ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, token_mask=mask)
        assert np.array_equal(yh[sample].view(np.uint32), ref["y"][sample].view(np.uint32))
    L.close()


def _sparse_bank(L, experts):
    """Canonical bank of layer L with only `experts` exported (others zero)."""
    eb = moe_ffn.expert_bytes(L.H, L.I)
    bank = np.zeros(L.E * eb, np.uint8)
    for e in sorted(set(int(e) for e in experts)):
        bank[e * eb:(e + 1) * eb] = L.export_expert(e)
    return bank


def test_stack_layers_mixed_batch():
    """BASELINE configs[4] in miniature: three resident layers with their own
    seeded weights, each run on a mixed batch of 8 decode + 1024 prefill
    tokens with Zipf(1.3) routing, back to back on one stream; then every
    layer's output is checked against the oracle on its 8 decode tokens and 8
    sampled prefill tokens (weights exported from the device bank)."""
    NS = 8 + 1024
    layers = [moe_ffn.MoeLayer(2048, 512, 512, 10, True, NS, synthetic_seed=900 + l) for l in range(3)]
    runs = []
    for l, L in enumerate(layers):
        x = W.activations(NS, seed=910 + l)
        ids, w = W.routes_zipf(NS, 1.3, seed=920 + l)
        runs.append((x, ids, w, L.forward(dev(x), dev(ids), dev(w))))
    rng = np.random.default_rng(930)
    for l, (L, (x, ids, w, (y, err))) in enumerate(zip(layers, runs)):
        yh = host(y)
        assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
        sample = np.concatenate([np.arange(8), 8 + rng.choice(1024, 8, replace=False)])
        bank = _sparse_bank(L, ids[sample].reshape(-1))
        shared = L.export_expert(L.E)
        # debug_last holds the most recent forward of this handle, which is
        # this layer's own (each layer has its own workspace).
        layer_parity(L, x, ids, w, bank, shared, yh, sample, f"stack layer {l}")
    for L in layers:
        L.close()


@pytest.mark.parametrize("tokens", [8, 300, 4096])
def test_forward_q8_matches_forward(moe512, tokens):
    """moe_ffn_forward_q8 on the reference quantizer's Q8 rows of x gives
    forward(x)'s bits on every path (decode at 8 tokens, grouped streaming
    and MFMA at 300 and 4096), and leaves the same x Q8 for debug_last."""
    L = moe512["layer"]
    x = W.activations(tokens, seed=61 + tokens)
    ids, w = (W.routes_uniform(tokens, seed=62) if tokens == 8 else W.routes_zipf(tokens, 1.1, seed=62 + tokens))
    g = np.random.default_rng(63).standard_normal(tokens).astype(np.float32)
    y1, e1 = L.forward(dev(x), dev(ids), dev(w), shared_gate=dev(g))
    xq1 = host(L.debug_last(tokens)["x_q8"]).copy()
    y1h = host(y1).copy()
    xq = q8_bytes(O.quantize_q8(x)).reshape(tokens, -1)
    assert np.array_equal(xq1.reshape(tokens, -1), xq)
    y2, e2 = L.forward_q8(dev(xq), dev(ids), dev(w), shared_gate=dev(g))
    assert np.array_equal(host(y2).view(np.uint32), y1h.view(np.uint32))
    assert np.array_equal(host(L.debug_last(tokens)["x_q8"]), xq1)
    assert int(host(e1)[0]) == 0 and int(host(e2)[0]) == 0


def test_read_probe_leaves_sink():
    """The measurement hook streams a buffer and never writes its sink for
    non-matching data; bad sizes are rejected before any launch."""
    buf = torch.ones(1 << 20, dtype=torch.int32, device=DEV)
    sink = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    moe_ffn.read_probe(buf, sink)
    assert int(host(sink)[0]) == 7
    with pytest.raises(moe_ffn.MoeError):
        moe_ffn.read_probe(buf, sink, nbytes=20)


def test_forward_reuse_smaller_batch_and_determinism(moe512):
    L = moe512["layer"]
    x = W.activations(37, seed=61)
    ids, w = W.routes_zipf(37, 1.3, seed=62)
    y1, _ = L.forward(dev(x), dev(ids), dev(w))
    y1 = host(y1)
    x5 = x[:5].copy()
    y5, _ = L.forward(dev(x5), dev(ids[:5]), dev(w[:5]))
    y2, _ = L.forward(dev(x), dev(ids), dev(w))
    assert np.array_equal(host(y2), y1)                   # deterministic
    # 5 tokens take the decode path (reference order throughout), 37 the
    # grouped MFMA path (its down projection sums blocks in its own order).
    ref = O.moe_layer(x, 2048, 512, 512, moe512["bank"], ids, w, shared_q4=moe512["shared"])
    assert np.array_equal(host(y5).view(np.uint32), ref["y"][:5].view(np.uint32))
    assert_close(y1, ref["y"], tol=1e-5, what="37-token layer")


def test_forward_flags_bad_inputs(moe512):
    L = moe512["layer"]
    x = W.activations(8, seed=71)
    ids, w = W.routes_uniform(8, seed=72)
    xb = x.copy()
    xb[3, 100] = np.nan
    y, err = L.forward(dev(xb), dev(ids), dev(w))
    assert int(host(err)[0]) & 1
    ib = ids.copy()
    ib[2, 4] = 600
    _, err = L.forward(dev(x), dev(ib), dev(w))
    assert int(host(err)[0]) & 1
    ib = ids.copy()
    ib[2, 4] = ib[2, 0]
    _, err = L.forward(dev(x), dev(ib), dev(w))
    assert int(host(err)[0]) & 1
    # A valid call afterwards is clean (nothing sticky inside the layer).
    y, err = L.forward(dev(x), dev(ids), dev(w))
    assert int(host(err)[0]) == 0


def test_synthetic_bank_export_roundtrip():
    L = moe_ffn.MoeLayer(2048, 512, 4, 2, True, 8, synthetic_seed=99)
    e2 = L.export_expert(2)
    sh = L.export_expert(4)
    d = e2[:18 * 64 * 512].reshape(-1, 18)[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.isfinite(d)) and np.all(d >= 0) and 0.01 < float(np.mean(d)) < 0.025   # |N(0, .02)|
    x = W.activations(8, seed=81)
    ids = np.array([[2, 1]] * 8, np.int32)
    w = np.full((8, 2), 0.5, np.float32)
    bank = np.concatenate([L.export_expert(e) for e in range(4)])
    y, err = L.forward(dev(x), dev(ids), dev(w))
    ref = O.moe_layer(x, 2048, 512, 4, bank, ids, w, shared_q4=sh)
    assert_close(host(y), ref["y"], what="synthetic bank")
    L.close()


def _split_tensors(bank, E, H, I):
    """Canonical per-expert bank [E][gate|up|down] -> the reference's three
    routed-expert tensors [E][rows][blocks] (src/session.hip:700-716)."""
    mb = H // 32 * I * 18
    per = bank.reshape(E, 3, mb)
    return [np.ascontiguousarray(per[:, m, :]).reshape(-1) for m in range(3)]


def test_create_from_reference_tensors(moe512):
    """moe_ffn_create_tensors at the bench shape: 512 experts + shared span two
    staging chunks (455 expert matrices each); every expert on either side of
    the boundary and the shared one export to the canonical bytes, and the
    forward matches the canonical-upload layer bit for bit."""
    bank, shared = moe512["bank"], moe512["shared"]
    ts = _split_tensors(bank, 512, 2048, 512)
    ss = _split_tensors(shared, 1, 2048, 512)
    L = moe_ffn.MoeLayer(2048, 512, 512, 10, True, 64, tensors=ts, shared_tensors=ss)
    eb = len(bank) // 512
    for e in (0, 1, 454, 455, 456, 511):
        assert np.array_equal(L.export_expert(e), bank[e * eb:(e + 1) * eb]), e
    assert np.array_equal(L.export_expert(512), shared)
    x = W.activations(8, seed=91)
    ids, w = W.routes_uniform(8, seed=92)
    y1, e1 = L.forward(dev(x), dev(ids), dev(w))
    y2, e2 = moe512["layer"].forward(dev(x), dev(ids), dev(w))
    assert np.array_equal(host(y1), host(y2))
    assert int(host(e1)[0]) == 0 and int(host(e2)[0]) == 0
    L.close()


def _layer_with_path(decode, *args, **kw):
    """A layer whose forward path is forced: MOE_FFN_DECODE is read at creation."""
    old = os.environ.get("MOE_FFN_DECODE")
    os.environ["MOE_FFN_DECODE"] = "1" if decode else "0"
    try:
        return moe_ffn.MoeLayer(*args, **kw)
    finally:
        if old is None:
            del os.environ["MOE_FFN_DECODE"]
        else:
            os.environ["MOE_FFN_DECODE"] = old


@pytest.mark.parametrize("gate", [False, True])
def test_decode_and_grouped_paths_agree(gate):
    """The ungrouped decode path (work per (token, rank), fold inside the down
    kernel) and the grouped streaming path both follow the reference's fp32
    order, so they give the same bits as each other and as the oracle,
    including for an invalid id and a duplicate id (both contribute nothing
    and set bit 1; the oracle sees a weight-0 route to an unused expert).
    The grouped MFMA path (the default for grouped batches) has the same
    middle and sums its down blocks in its own order: within 1e-5 rms."""
    H, I, E, K, N = 2048, 512, 24, 6, 5
    bank = W.q4_bank(E, seed=301)
    shared = W.q4_bank(1, seed=302)
    x = W.activations(N, seed=303)
    ids, w = W.routes_uniform(N, experts=E, k=K, seed=304)
    g = np.random.default_rng(305).standard_normal(N).astype(np.float32) if gate else None
    ids_bad = ids.copy()
    ids_bad[0, 0] = E + 5           # bad id (rank 0: the token's reporting workgroup)
    ids_bad[3, 2] = ids_bad[3, 1]   # duplicate
    outs = {}
    paths = {"decode": {"MOE_FFN_DECODE": 1}, "stream": {"MOE_FFN_DECODE": 0, "MOE_FFN_MFMA_MIN": 0},
             "mfma": {"MOE_FFN_DECODE": 0, "MOE_FFN_MFMA_MIN": 1}}
    for path, env in paths.items():
        L = _layer_env(env, H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
        for name, i_ in (("ok", ids), ("bad", ids_bad)):
            y, err = L.forward(dev(x), dev(i_), dev(w), shared_gate=None if g is None else dev(g))
            outs[(path, name)] = (host(y), int(host(err)[0]))
        dbg = L.debug_last(N)
        assert np.array_equal(host(dbg["x_q8"]).reshape(-1), q8_bytes(O.quantize_q8(x)))
        L.close()
    rid, rw = ids_bad.copy(), w.copy()
    for t, r in ((0, 0), (3, 2)):
        rid[t, r] = next(e for e in range(E) if e not in ids_bad[t])
        rw[t, r] = 0.0
    refs = {"ok": O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, shared_gate=g)["y"],
            "bad": O.moe_layer(x, H, I, E, bank, rid, rw, shared_q4=shared, shared_gate=g)["y"]}
    for name in ("ok", "bad"):
        (yd, ed), (ys, es), (ym, em) = outs[("decode", name)], outs[("stream", name)], outs[("mfma", name)]
        assert ed == es == em == (0 if name == "ok" else 1), (name, ed, es, em)
        assert np.array_equal(yd.view(np.uint32), refs[name].view(np.uint32)), name
        assert np.array_equal(ys.view(np.uint32), refs[name].view(np.uint32)), name
        assert_close(ym, refs[name], tol=1e-5, what=f"MFMA path, {name} routes")


def test_decode_path_middle_debug_view(moe512):
    """debug_last on a decode-path forward returns the middle Q8 rows in
    grouped order, bit-identical to the single-expert gate/up stage of the
    same expert on the same token (same per-row arithmetic)."""
    L = moe512["layer"]
    x = W.activations(8, seed=311)
    ids, w = W.routes_uniform(8, seed=312)
    L.forward(dev(x), dev(ids), dev(w))
    dbg = L.debug_last(8)
    groups = O.route_groups(ids, w, 512)
    mid = host(dbg["middle_q8"]).reshape(8 * 11, -1)
    xq = dev(q8_bytes(O.quantize_q8(x)).reshape(8, -1))
    for pos in (0, 17, 45, 79):
        t, e = int(groups["token"][pos]), int(groups["expert"][pos])
        r = L.expert_gate_up(e, xq[t:t + 1].contiguous(), 1)
        assert np.array_equal(mid[pos], host(r["middle_q8"]).reshape(-1)), pos
    # shared expert rows follow the routed ones, one per token
    r = L.expert_gate_up(512, xq, 8)
    assert np.array_equal(mid[80:], host(r["middle_q8"]).reshape(8, -1))


def test_decode_quantizer_reference_fixture():
    """The decode path quantizes x inside its gate/up kernel (4 lanes per
    block); the x Q8 it writes must equal the reference quantizer's bytes on
    the reference fixture's blocks (ties, tiny and huge scales, zero blocks),
    with failing blocks zeroed and flagged, like the standalone quantizer."""
    f = np.load(os.path.join(GOLDEN, "quant_q8.npz"), allow_pickle=False)
    blocks = f["inputs"]
    rows = -(-len(blocks) // 64)
    x = np.zeros((rows * 64, 32), np.float32)
    x[:len(blocks)] = blocks
    x = x.reshape(rows, 2048)
    bank = W.q4_bank(4, seed=321)
    L = _layer_with_path(True, 2048, 512, 4, 1, False, rows, experts_q4=bank)
    ids = np.zeros((rows, 1), np.int32)
    w = np.ones((rows, 1), np.float32)
    _, err = L.forward(dev(x), dev(ids), dev(w))
    got = host(L.debug_last(rows)["x_q8"]).reshape(-1, 36)[:len(blocks)]
    ok = f["status"] == 0
    assert np.array_equal(got[ok], f["q8"][ok])
    assert np.all(got[~ok] == 0)
    assert int(host(err)[0]) != 0
    L.close()


# ------------------------------------------------------- int8-MFMA path ----
def _layer_env(env, *args, **kw):
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


@pytest.fixture(scope="module")
def mfma_expert():
    bank = W.q4_bank(1, seed=401)
    mb = len(bank) // 3
    layer = moe_ffn.MoeLayer(2048, 512, 1, 1, False, 200, experts_q4=bank)
    return dict(layer=layer, g=bank[:mb], u=bank[mb:2 * mb], d=bank[2 * mb:])


@pytest.mark.parametrize("columns", [1, 8, 33, 128, 200])
def test_mfma_expert_stages_bit_exact_dots(mfma_expert, columns):
    """Single-expert stages on the int8-MFMA path: per-block int32 dots of
    gate, up and down bit-exact (partial token tiles, one and two 128-pair
    items), middle within 1e-3 rms of the oracle and its Q8 bytes equal to
    the reference quantizer of the GPU middle, down within 1e-5 rms of the
    reference cpu_expert order on a shared middle."""
    L, g, u, d = mfma_expert["layer"], mfma_expert["g"], mfma_expert["u"], mfma_expert["d"]
    x = W.activations(columns, seed=410 + columns)
    xq = O.quantize_q8(x)
    r = L.expert_gate_up(0, dev(q8_bytes(xq).reshape(columns, -1)), columns, path=moe_ffn.PATH_MFMA, dots=True)
    assert np.array_equal(host(r["gate_dots"]), O.block_dots(g, 2048, 512, xq))
    assert np.array_equal(host(r["up_dots"]), O.block_dots(u, 2048, 512, xq))
    ref = O.expert_forward(g, u, d, 2048, 512, xq, avx2=True)
    middle = host(r["middle"])
    # The MFMA gate/up follows the reference's fp32 order and expf: the
    # middle and its Q8 are bit-identical to the CPU reference's.
    assert np.array_equal(middle.view(np.uint32), ref["middle"].view(np.uint32))
    assert np.array_equal(host(r["middle_q8"]).reshape(-1), q8_bytes(ref["middle_q8"]))
    assert int(host(r["error"])[0]) == 0
    mq = ref["middle_q8"]
    rd = L.expert_down(0, dev(q8_bytes(mq).reshape(columns, -1)), columns, path=moe_ffn.PATH_MFMA, dots=True)
    assert np.array_equal(host(rd["down_dots"]), O.block_dots(d, 512, 2048, mq))
    assert_close(host(rd["y"]), O.matrix_gpu_order(d, 512, 2048, mq), tol=1e-5, what="MFMA down projection")
    # The non-debug kernels give the same bits as the debug ones.
    r2 = L.expert_gate_up(0, dev(q8_bytes(xq).reshape(columns, -1)), columns, path=moe_ffn.PATH_MFMA)
    assert np.array_equal(host(r2["middle_q8"]), host(r["middle_q8"]))
    rd2 = L.expert_down(0, dev(q8_bytes(mq).reshape(columns, -1)), columns, path=moe_ffn.PATH_MFMA)
    assert np.array_equal(host(rd2["y"]), host(rd["y"]))


def test_mfma_reference_shape_expert_vs_golden():
    """The reference's own CPU expert output at 2560/640 on the MFMA path
    (80 and 20 blocks per row: partial 16-block chunks of the s8 term)."""
    f = np.load(os.path.join(GOLDEN, "cpu_expert_2560x640.npz"), allow_pickle=False)
    g, u, d = expert_weights(2560, 640)
    layer = _single_expert(2560, 640, (g, u, d), 3)
    xq = f["x_q8"].reshape(3, -1)
    r = layer.expert_gate_up(0, dev(xq), 3, path=moe_ffn.PATH_MFMA, dots=True)
    assert np.array_equal(host(r["gate_dots"]), O.block_dots(g, 2560, 640, xq))
    assert np.array_equal(host(r["up_dots"]), O.block_dots(u, 2560, 640, xq))
    # bit-identical to the compiled reference cpu_expert's middle (80 blocks:
    # reference lanes holding two blocks each)
    assert np.array_equal(host(r["middle"]).view(np.uint32), f["middle"].view(np.uint32))
    rd = layer.expert_down(0, r["middle_q8"], 3, path=moe_ffn.PATH_MFMA, dots=True)
    mq = host(r["middle_q8"]).reshape(3, -1)
    assert np.array_equal(host(rd["down_dots"]), O.block_dots(d, 640, 2560, mq))
    assert_close(host(rd["y"]), f["y"], what="MFMA expert vs reference cpu_expert")
    layer.close()


def test_mfma_layer_4k_zipf(moe512):
    """BASELINE configs[2] with every group on the MFMA path: sampled tokens
    against the oracle, and every token against the streaming path."""
    x = W.activations(4096, seed=501)
    ids, w = W.routes_zipf(4096, 1.1, seed=502)
    L = _layer_env({"MOE_FFN_MFMA_MIN": 1}, 2048, 512, 512, 10, True, 4096, experts_q4=moe512["bank"],
                   shared_q4=moe512["shared"])
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    st = L.last_stats()
    assert st["stream_items"] == 0 and st["mfma_items"] > 0
    sample = np.random.default_rng(503).choice(4096, 24, replace=False)
    layer_parity(L, x, ids, w, moe512["bank"], moe512["shared"], yh, sample, "MFMA 4K prefill")
    # Every token against the streaming kernels (k_gate_up_lean / k_down_lean):
    # both gate/up paths follow the reference's fp32 order, so the middles
    # are identical; the two down kernels sum their blocks in different
    # orders.
    S = _layer_env({"MOE_FFN_MFMA_MIN": 0}, 2048, 512, 512, 10, True, 4096, experts_q4=moe512["bank"],
                   shared_q4=moe512["shared"])
    ys, es = S.forward(dev(x), dev(ids), dev(w))
    assert int(host(es)[0]) == 0 and S.last_stats()["mfma_items"] == 0
    assert np.array_equal(host(S.debug_last(4096)["middle_q8"]), host(L.debug_last(4096)["middle_q8"]))
    assert_close(yh, host(ys), tol=1e-5, what="MFMA vs streaming path, all 4096 tokens")
    S.close()
    y2, _ = L.forward(dev(x), dev(ids), dev(w))
    assert np.array_equal(host(y2), yh)   # deterministic
    L.close()


@pytest.mark.parametrize("mfma_min", [1, 16, 0])
def test_mfma_layer_small_batches(moe512, mfma_min):
    """Grouped path (decode path off) with MFMA for groups >= mfma_min (0:
    streaming kernels only): 37 and 300 Zipf tokens fully against the oracle;
    per-token independence (bit-exact on a single path; with mixed paths the
    down projection of a group depends on the path its size selects)."""
    L = _layer_env({"MOE_FFN_MFMA_MIN": mfma_min, "MOE_FFN_DECODE": 0}, 2048, 512, 512, 10, True, 300,
                   experts_q4=moe512["bank"], shared_q4=moe512["shared"])
    for n, seed in ((37, 511), (300, 512)):
        x = W.activations(n, seed=seed)
        ids, w = W.routes_zipf(n, 1.3, seed=seed + 100)
        y, err = L.forward(dev(x), dev(ids), dev(w))
        yh = host(y)
        assert int(host(err)[0]) == 0
        layer_parity(L, x, ids, w, moe512["bank"], moe512["shared"], yh, np.arange(n),
                     f"{n}-token layer, mfma_min {mfma_min}")
        y5, _ = L.forward(dev(x[:5].copy()), dev(ids[:5]), dev(w[:5]))
        if mfma_min in (0, 1):
            assert np.array_equal(host(y5), yh[:5])
        else:
            assert_close(host(y5), yh[:5], tol=1e-5, what="mixed paths, 5-token batch")
    L.close()


def test_mfma_layer_invalid_routes_flag():
    """A bad id and a duplicate id on the MFMA path contribute nothing and set
    bit 1; the rest matches the oracle with those routes at weight 0."""
    H, I, E, K, N = 2048, 512, 24, 6, 40
    bank = W.q4_bank(E, seed=601)
    shared = W.q4_bank(1, seed=602)
    x = W.activations(N, seed=603)
    ids, w = W.routes_uniform(N, experts=E, k=K, seed=604)
    ids[0, 0] = E + 5
    ids[3, 2] = ids[3, 1]
    L = _layer_env({"MOE_FFN_MFMA_MIN": 1, "MOE_FFN_DECODE": 0}, H, I, E, K, True, N, experts_q4=bank,
                   shared_q4=shared)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    assert int(host(err)[0]) == 1
    rid, rw = ids.copy(), w.copy()
    for t, r in ((0, 0), (3, 2)):
        rid[t, r] = next(e for e in range(E) if e not in ids[t])
        rw[t, r] = 0.0
    ref = O.moe_layer(x, H, I, E, bank, rid, rw, shared_q4=shared)["y"]
    assert_close(host(y), ref, what="MFMA path, invalid routes")
    L.close()


def test_expf_device_matches_libm():
    """The kernels' expf on the GPU equals the C library's expf bit for bit
    (the function the reference's CPU SiLU calls, src/cpu_expert.cpp:251)."""
    from test_abi import _expf_sample
    # Regimes interleaved lane by lane (normal, overflow, underflow, +-inf,
    # nan, the |x| >= 88 band): the table lookup must not depend on which
    # lanes of a wave take a special-case exit.
    special = np.array([0.5, 100.0, -200.0, np.inf, -np.inf, np.nan, 88.5, -95.0, -103.0, 88.7, -104.0, 1e-30],
                       np.float32)
    mixed = np.tile(special, 64) * np.repeat(np.float32([1, -1]), special.size * 32)
    x = np.concatenate([mixed, _expf_sample()])
    got = host(moe_ffn.expf_device(dev(x)))
    ref = O.expf_libm(x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ------------------------------------------------------------------ router ---
def _router_check(logits, k, what):
    x = dev(logits)
    ids, w, p, err = moe_ffn.router_select(x, top_k=k, probabilities=True)
    p_ref, f_ref = O.router_softmax(logits)
    i_ref, w_ref, g_ref = O.select_routes(p_ref, k)
    assert np.array_equal(host(p).view(np.uint32), p_ref.view(np.uint32)), what
    assert np.array_equal(host(ids), i_ref), what
    assert np.array_equal(host(w).view(np.uint32), w_ref.view(np.uint32)), what
    assert int(host(err)[0]) == (f_ref | g_ref), what


def test_router_select_bit_exact():
    """Device router (softmax in router_softmax's order + select_routes) against
    the oracle restatement: probabilities, ids and weights bit for bit."""
    rng = np.random.default_rng(700)
    _router_check((rng.standard_normal((4096, 512)) * 3).astype(np.float32), 10, "random 4096 x 512")
    _router_check((rng.standard_normal((64, 64)) * 0.1).astype(np.float32), 4, "64 experts, top-4")
    _router_check(np.zeros((8, 512), np.float32), 10, "uniform: ties to the lower ids")
    tie = rng.standard_normal((16, 512)).astype(np.float32)
    tie[:, 100:140] = 5.0                           # forty equal leaders
    _router_check(tie, 10, "equal leaders")
    spread = np.zeros((4, 512), np.float32)
    spread[:, :] = -60.0
    spread[:, 0] = 60.0                             # one winner, the rest underflow to 0
    _router_check(spread, 10, "one winner")
    order = np.full((2, 512), -300.0, np.float32)   # the oracle's hand-derived lane-order case
    order[:, 31] = 0.0
    order[:, 0:512:32] = -16.7
    order[1] = np.roll(order[1], 7)
    _router_check(order, 10, "lane-order rounding")
    _router_check((rng.standard_normal((16, 1024)) * 2).astype(np.float32), 32, "1024 experts, top-32")
    wide = rng.standard_normal((8, 1024)).astype(np.float32)
    wide[:, 500:560] = 4.0                          # sixty equal leaders across the two halves
    _router_check(wide, 32, "1024 experts, equal leaders")
    _router_check(rng.standard_normal((16, 32)).astype(np.float32), 32, "32 experts, all selected")
    _router_check(rng.standard_normal((16, 96)).astype(np.float32), 7, "96 experts, top-7")
    # More than 512 rows: one wave per row (batches up to 512 rows spread a
    # row's exponentials over several waves); same bits either way.
    _router_check((rng.standard_normal((600, 1024)) * 2).astype(np.float32), 32, "600 x 1024, top-32, one wave per row")
    _router_check(rng.standard_normal((700, 96)).astype(np.float32), 7, "700 x 96, top-7, one wave per row")
    _router_check(rng.standard_normal((513, 64)).astype(np.float32), 32, "513 x 64, top-32 (the pair bound at its limit)")
    _router_check(rng.standard_normal((520, 32)).astype(np.float32), 32, "520 x 32, all selected, one wave per row")
    big_tie = rng.standard_normal((600, 512)).astype(np.float32)
    big_tie[:, 100:140] = 5.0
    _router_check(big_tie, 10, "600 rows, equal leaders, one wave per row")
    # The same shapes at 300 rows take the spread form.
    _router_check((rng.standard_normal((300, 1024)) * 2).astype(np.float32), 32, "300 x 1024, top-32, spread")
    _router_check(rng.standard_normal((400, 96)).astype(np.float32), 7, "400 x 96, top-7, spread")


def test_router_select_flags_bad_rows():
    x = np.random.default_rng(701).standard_normal((6, 512)).astype(np.float32)
    x[1, 3] = np.nan
    x[4, 9] = np.inf
    x[2, 5], x[2, 6] = 3e38, -3e38   # x - max overflows to -inf: the arithmetic bit
    ids, w, p, err = moe_ffn.router_select(dev(x), top_k=10, probabilities=True)
    assert int(host(err)[0]) == 3
    ph, ih, wh = host(p), host(ids), host(w)
    for t in (1, 2, 4):   # zero row: ids 0..9, zero weights
        assert np.all(ph[t] == 0) and list(ih[t]) == list(range(10)) and np.all(wh[t] == 0)
    _router_check(x, 10, "rows with nonfinite logits")
    for rows in (300, 600):   # spread, then one wave per row
        big = np.random.default_rng(704 + rows).standard_normal((rows, 512)).astype(np.float32)
        big[7, 11] = np.nan
        big[250, 3], big[250, 4] = 3e38, -3e38
        _router_check(big, 10, f"{rows} rows with bad rows")


def test_router_then_forward_matches_oracle(moe512):
    """Logits -> device router -> forward, without a host round trip: B8 output
    bit-identical to the oracle layer on the oracle's own routes."""
    rng = np.random.default_rng(702)
    logits = rng.standard_normal((8, 512)).astype(np.float32)
    x = W.activations(8, seed=703)
    ids, w, _, err = moe_ffn.router_select(dev(logits))
    y, err2 = moe512["layer"].forward(dev(x), ids, w)
    p_ref, _ = O.router_softmax(logits)
    i_ref, w_ref, _ = O.select_routes(p_ref, 10)
    ref = O.moe_layer(x, 2048, 512, 512, moe512["bank"], i_ref, w_ref, shared_q4=moe512["shared"])
    assert int(host(err)[0]) == 0 and int(host(err2)[0]) == 0
    assert np.array_equal(host(y).view(np.uint32), ref["y"].view(np.uint32))
