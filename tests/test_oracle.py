"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the checker.

Sources of truth, in order:
  * golden fixtures written by the reference's own compiled CPU code
    (tests/golden/make_golden.py, oracle/_ref): bitwise equality;
  * literal known answers from the reference's tests
    (tests/quant_test.cpp:218-300, 338-405, 438-480, 572-603);
  * closed forms / brute force: IEEE binary16 via numpy, wide-integer dots,
    one-hot folds.
"""
import hashlib
import os

import numpy as np
import pytest

import oracle as O
from golden_inputs import expert_input, expert_weights, matmul_case, q4_1_matrix, route_cases

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def q8_bytes(q):
    return np.ascontiguousarray(q).view(np.uint8).reshape(-1)


# ----------------------------------------------------------------- half ----
def test_half_to_float_exhaustive_vs_ieee():
    h = np.arange(65536, dtype=np.uint16)
    mine = np.array([O.lib().mo_half_to_float(int(v)) for v in h], np.float32)
    ieee = h.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ieee)
    assert np.array_equal(mine[finite].view(np.uint32), ieee[finite].view(np.uint32))
    # NaNs keep sign and payload and are quieted (quant.cpp:224-227).
    nan = h[~finite]
    bits = mine[~finite].view(np.uint32)
    expect = ((nan.astype(np.uint32) & 0x8000) << 16) | 0x7f800000 | ((nan.astype(np.uint32) & 0x3ff) << 13) | 0x400000
    assert np.array_equal(bits, expect)


def test_float_to_half_rne_vs_numpy():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # Concentrate on the half range, subnormal range and rounding boundaries.
    mags = (rng.standard_normal(200000) * np.exp2(rng.integers(-30, 18, 200000))).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, 2.0**-24, 2.0**-25, np.nextafter(2.0**-25, 1), 2.0**-26,
                      6.1035156e-05, 5.9604645e-08, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11], np.float32)
    vals = np.concatenate([bits.view(np.float32), mags, edges, -edges])
    vals = vals[~np.isnan(vals)]
    mine = np.array([O.lib().mo_float_to_half(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, ref)


# ------------------------------------------------------------- quantize ----
def test_quantize_matches_reference_fixture():
    f = load("quant_q8.npz")
    for i, block in enumerate(f["inputs"]):
        if f["status"][i] != 0:
            with pytest.raises(O.OracleError):
                O.quantize_q8(block.reshape(1, 32))
            continue
        assert np.array_equal(q8_bytes(O.quantize_q8(block.reshape(1, 32))), f["q8"][i]), i


def _q(values):
    return O.quantize_q8(np.asarray(values, np.float32).reshape(1, 32)).reshape(-1)[0]


def test_quantize_literal_known_answers():
    # Ties round away from zero (quant_test.cpp:227-235).
    v = np.zeros(32, np.float32)
    v[0] = 127.0
    v[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    assert list(_q(v)["qs"][1:9]) == [1, -1, 2, -2, 3, -3, 127, -127]
    # Raw input sum, not the code reconstruction (quant_test.cpp:244-252).
    v = np.full(32, 0.4, np.float32)
    v[0] = 127.0
    assert _q(v)["s"] == np.float16(np.float32(139.4)).view(np.uint16)
    # Codes use the original FP32 scale (quant_test.cpp:254-261).
    v = np.zeros(32, np.float32)
    v[0] = 1.0
    v[1] = np.nextafter(np.float32(1.0 / 127.0) * np.float32(0.5), np.float32(0))
    assert _q(v)["qs"][1] == 0
    # Ascending XOR butterfly: cancellation gives s = 0 (quant_test.cpp:263-272).
    v = np.zeros(32, np.float32)
    v[:4] = [1048576.0, 0.03125, -1048576.0, 0.03125]
    assert _q(v)["s"] == 0
    # Minimum surviving half scale keeps codes (quant_test.cpp:274-279).
    v = np.zeros(32, np.float32)
    v[0] = np.float32(127.0) * np.nextafter(np.float32(2.0**-25), np.float32(1))
    v[1] = -v[0]
    q = _q(v)
    assert q["d"] == 1 and q["qs"][0] == 127 and q["qs"][1] == -127
    # Tiny constant: stored half d = 0, codes and raw sum kept (quant_test.cpp:343-353).
    for sign in (1.0, -1.0):
        q = _q(np.full(32, sign * 3.4e-6, np.float32))
        assert q["d"] == 0 and (q["s"] & 0x7fff) != 0 and all(c == int(sign) * 127 for c in q["qs"])
    # Zero and negative-zero blocks are the exact zero block.
    v = np.zeros(32, np.float32)
    v[::2] = -0.0
    assert q8_bytes(_q(v)).sum() == 0


def test_quantize_rejections():
    for bad in (np.inf, -np.inf, np.nan):
        v = np.ones(32, np.float32)
        v[7] = bad
        with pytest.raises(O.OracleError):
            _q(v)
    v = np.zeros(32, np.float32)
    v[0] = np.float32(1.4e-45)        # FP32 scale underflows to zero
    with pytest.raises(O.OracleError):
        _q(v)
    with pytest.raises(O.OracleError):
        _q(np.full(32, 3000.0, np.float32))   # raw sum overflows half


# ------------------------------------------------------------------ dots ---
def test_block_dot_full_range_closed_form():
    L = O.lib()
    for code in range(16):
        qs = np.full(16, code * 17, np.uint8)
        for value in (-128, -127, -1, 0, 1, 126, 127):
            c = np.full(32, value, np.int8)
            assert L.mo_block_dot(qs.ctypes.data, c.ctypes.data) == 32 * code * value


def test_block_dot_brute_force():
    rng = np.random.default_rng(3)
    L = O.lib()
    for _ in range(500):
        qs = rng.integers(0, 256, 16, dtype=np.uint8)
        c = rng.integers(-128, 128, 32, dtype=np.int8)
        nib = np.concatenate([qs & 15, qs >> 4]).astype(np.int64)
        assert L.mo_block_dot(qs.ctypes.data, c.ctypes.data) == int((nib * c.astype(np.int64)).sum())


def test_scaled_dot_literal():
    # quant_test.cpp:460-467: d4 = -1, d8 = 0.5, s8 = 3, codes -128, nibbles 0 -> 24.
    x = np.zeros(1, O.Q8_DTYPE)
    x["d"], x["s"], x["qs"] = 0x3800, 0x4200, -128
    assert O.lib().mo_scaled_dot_q4_0(0, 0xbc00, x.ctypes.data) == 24.0


def test_matmul_literal_fixture():
    # quant_test.cpp:572-603: two one-block rows x two columns, column-major out.
    x = np.zeros(2, O.Q8_DTYPE)
    x["d"] = 0x3c00
    x["s"][0], x["s"][1] = 0x4000, 0xc200
    x["qs"][0, :16], x["qs"][0, 16:], x["qs"][1] = 3, -4, -128
    w = np.zeros((2, 18), np.uint8)
    w[:, :2] = np.array([0x3c00], np.uint16).view(np.uint8)
    w[0, 2:], w[1, 2:] = 0x21, 0x75
    out = O.matmul_full(w.reshape(-1), 32, 2, x)
    assert out.reshape(-1).tolist() == [-96.0, -224.0, -6120.0, -24552.0]


def test_matmul_matches_reference_fixture():
    f = load("matmul.npz")
    for name, (w, K, M, xq) in matmul_case().items():
        mine = O.matmul_full(w, K, M, xq)
        for tag in ("scalar", "avx2", "q8ref"):
            key = f"{name}_{tag}"
            if key in f:
                assert np.array_equal(mine.view(np.uint32), f[key].view(np.uint32)), key


# ----------------------------------------------------------- cpu_expert ----
@pytest.fixture(scope="module")
def expert_fixture():
    f = load("cpu_expert_2560x640.npz")
    gate, up, down = expert_weights(2560, 640)
    assert hashlib.sha256(gate.tobytes() + up.tobytes() + down.tobytes()).hexdigest() == str(f["weights_sha256"])
    return f, gate, up, down


def test_expert_input_quantization_matches_reference(expert_fixture):
    f, *_ = expert_fixture
    x = expert_input(3, 2560)
    assert np.array_equal(x, f["x"])
    assert np.array_equal(q8_bytes(O.quantize_q8(x)), f["x_q8"].reshape(-1))


@pytest.mark.parametrize("avx2", [False, True])
def test_expert_forward_bitwise_vs_reference(expert_fixture, avx2):
    f, gate, up, down = expert_fixture
    out = O.expert_forward(gate, up, down, 2560, 640, f["x_q8"], avx2=avx2)
    for key in ("gate", "up", "middle", "y"):
        assert np.array_equal(out[key].view(np.uint32), f[key].view(np.uint32)), key
    assert np.array_equal(q8_bytes(out["middle_q8"]), f["middle_q8"].reshape(-1))


def test_expert_q41_down_bitwise_vs_reference(expert_fixture):
    """Q4_1 down (the checkpoint's layers 0-5): the oracle's expert equals the
    compiled reference's cpu_expert bit for bit; dropping the half rounding of
    d4*d8 and m4*s8 changes the output (so the rounding is really tested)."""
    f0, gate, up, _ = expert_fixture
    f = load("cpu_expert_2560x640_q41.npz")
    down = q4_1_matrix(404, 640, 2560)
    assert hashlib.sha256(gate.tobytes() + up.tobytes() + down.tobytes()).hexdigest() == str(f["weights_sha256"])
    out = O.expert_forward(gate, up, down, 2560, 640, f0["x_q8"], down_q41=True)
    assert np.array_equal(out["middle"].view(np.uint32), f["middle"].view(np.uint32))
    assert np.array_equal(q8_bytes(out["middle_q8"]), f["middle_q8"].reshape(-1))
    assert np.array_equal(out["y"].view(np.uint32), f["y"].view(np.uint32))
    # Unrounded products, same order otherwise (numpy restatement of one row).
    mq = O.as_q8(out["middle_q8"]).reshape(3, 20)
    blk = down.reshape(2560, 20, 20)
    r = 7
    lane = np.zeros(128, np.float32)
    d4 = blk[r, :, :2].copy().view(np.float16).astype(np.float32).reshape(20)
    m4 = blk[r, :, 2:4].copy().view(np.float16).astype(np.float32).reshape(20)
    d8 = mq["d"][0].view(np.float16).astype(np.float32)
    s8 = mq["s"][0].view(np.float16).astype(np.float32)
    for k in range(20):
        qs = blk[r, k, 4:]
        c = mq["qs"][0, k].astype(np.int32)
        for fr in range(2):
            j = np.arange(8 * fr, 8 * fr + 8)
            dot = int(np.sum((qs[j] & 15).astype(np.int32) * c[j] + (qs[j] >> 4).astype(np.int32) * c[j + 16]))
            dd, ms = np.float32(d4[k] * d8[k]), np.float32(m4[k] * s8[k])
            lane[2 * k + fr] = np.float32(lane[2 * k + fr] + np.float32(np.float64(dot) * dd + np.float64(ms * np.float32(0.5))))
    lane[:64] = lane[:64] + lane[64:]
    for mask in (1, 2, 4, 8, 16, 32):
        lane[:64] = (lane[:64] + lane[np.arange(64) ^ mask]).astype(np.float32)
    assert lane[0] != out["y"][0, r]


def test_expert_columns_are_independent(expert_fixture):
    f, gate, up, down = expert_fixture
    xq = O.as_q8(f["x_q8"]).reshape(3, 80)
    grouped = O.expert_forward(gate, up, down, 2560, 640, xq)["y"]
    for c in range(3):
        single = O.expert_forward(gate, up, down, 2560, 640, xq[c:c + 1])["y"]
        assert np.array_equal(single.view(np.uint32), grouped[c:c + 1].view(np.uint32))


def test_gpu_order_differs_from_serial_order(expert_fixture):
    # The two reference orders are distinct: a test that mixed them up fails.
    f, gate, *_ = expert_fixture
    xq = O.as_q8(f["x_q8"]).reshape(3, 80)
    a = O.matrix_gpu_order(gate, 2560, 640, xq)
    b = O.matmul_full(gate, 2560, 640, xq)
    assert not np.array_equal(a, b)
    assert np.max(np.abs(a - b)) < 1e-3 * np.sqrt(np.mean(b * b))


# ---------------------------------------------------------------- routes ---
def test_routes_match_reference_fixture():
    f = load("routes.npz")
    for name, (ids, w) in route_cases().items():
        if int(f[f"{name}_status"]) != 0:
            with pytest.raises(O.OracleError):
                O.route_groups(ids, w, 512)
            continue
        g = O.route_groups(ids, w, 512)
        for key in ("token", "rank", "expert", "counts"):
            assert np.array_equal(g[key], f[f"{name}_{key}"]), (name, key)
        assert np.array_equal(g["weight"].view(np.uint32), f[f"{name}_weight_bits"]), name
        assert np.array_equal(g["offsets"][1:], np.cumsum(g["counts"]))


def test_routes_brute_force_stable_sort():
    rng = np.random.default_rng(9)
    ids = np.array([rng.permutation(64)[:6] for _ in range(40)], np.int32)
    w = rng.random((40, 6), dtype=np.float32)
    g = O.route_groups(ids, w, 64)
    keys = sorted((int(ids[t, r]), t, r) for t in range(40) for r in range(6))
    assert [(int(e), int(t), int(r)) for e, t, r in zip(g["expert"], g["token"], g["rank"])] == keys


# ------------------------------------------------------------------ fold ---
def test_fold_rank_order_and_rounding():
    # Left fold from +0 in rank order with separately rounded products: the
    # cancellation case distinguishes it from pairwise or reversed sums.
    c = np.array([[[1e8], [1.0], [-1e8]]], np.float32)
    w = np.ones((1, 3), np.float32)
    assert O.routed_fold(c, w)[0, 0] == 0.0          # (1e8 + 1) - 1e8 in fp32
    c3 = np.array([[[1e8], [-1e8], [1.0]]], np.float32)
    assert O.routed_fold(c3, w)[0, 0] == 1.0
    # One-hot weights copy a contribution exactly; a scaled product rounds once.
    rng = np.random.default_rng(1)
    c = rng.standard_normal((4, 10, 16), dtype=np.float32)
    for r in range(10):
        w = np.zeros((4, 10), np.float32)
        w[:, r] = 1.0
        assert np.array_equal(O.routed_fold(c, w), c[:, r])
    w = np.zeros((4, 10), np.float32)
    w[:, 3] = 0.3
    assert np.array_equal(O.routed_fold(c, w), (np.float32(0.3) * c[:, 3]).astype(np.float32))


# ------------------------------------------------------------ composition --
def test_moe_layer_composes_expert_and_fold():
    H, I, E, k, N = 256, 64, 8, 3, 5
    rng = np.random.default_rng(2)
    bank = np.concatenate([np.concatenate(expert_weights(H, I, seed=700 + 3 * e)) for e in range(E)])
    shared = np.concatenate(expert_weights(H, I, seed=990))
    x = rng.standard_normal((N, H), dtype=np.float32)
    ids = np.array([rng.permutation(E)[:k] for _ in range(N)], np.int32)
    w = rng.random((N, k), dtype=np.float32)
    out = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, want_contrib=True)
    xq = O.quantize_q8(x)
    eb = 3 * H // 32 * I * 18
    mb = eb // 3
    for t in range(N):
        for r in range(k):
            e = ids[t, r]
            b = bank[e * eb:(e + 1) * eb]
            y = O.expert_forward(b[:mb], b[mb:2 * mb], b[2 * mb:], H, I, xq[t:t + 1])["y"][0]
            assert np.array_equal(y, out["contrib"][t, r])
    folded = O.routed_fold(out["contrib"], w)
    s = np.stack([O.expert_forward(shared[:mb], shared[mb:2 * mb], shared[2 * mb:], H, I, xq[t:t + 1])["y"][0]
                  for t in range(N)])
    assert np.array_equal(out["y"], (folded + s).astype(np.float32))
    # Baseline pool computes the same bits.
    sec, workers, yb = O.baseline_layer(x, H, I, E, bank, ids, w, shared_q4=shared, workers=2, repeats=1)
    assert workers >= 1 and sec > 0
    assert np.array_equal(yb, out["y"])


def test_shared_sigmoid_gate_closed_forms():
    # y = fold + sigmoid(g) * shared (src/hip/session_ops.hip:375-391).  g = 0
    # gives scale 0.5 exactly (a power-of-two product rounds nowhere); g = 30
    # gives 1/(1+expf(-30)) == 1.0f in fp32, i.e. the ungated sum; a negative
    # gate scales below 1 and differs from both.
    H, I, E, k, N = 128, 64, 6, 2, 3
    rng = np.random.default_rng(4)
    bank = np.concatenate([np.concatenate(expert_weights(H, I, seed=800 + 3 * e)) for e in range(E)])
    shared = np.concatenate(expert_weights(H, I, seed=991))
    x = rng.standard_normal((N, H), dtype=np.float32)
    ids = np.array([rng.permutation(E)[:k] for _ in range(N)], np.int32)
    w = rng.random((N, k), dtype=np.float32)
    base = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, want_contrib=True)
    folded = O.routed_fold(base["contrib"], w)
    s = (base["y"] - folded).astype(np.float32)     # exact: y = folded + s, recovered below
    assert np.array_equal((folded + s).astype(np.float32), base["y"])
    half = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, shared_gate=np.zeros(N, np.float32))["y"]
    mb = 3 * H // 32 * I * 18 // 3
    sh = np.stack([O.expert_forward(shared[:mb], shared[mb:2 * mb], shared[2 * mb:], H, I,
                                    O.quantize_q8(x[t:t + 1]))["y"][0] for t in range(N)])
    assert np.array_equal(half, (folded + np.float32(0.5) * sh).astype(np.float32))
    one = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, shared_gate=np.full(N, 30.0, np.float32))["y"]
    assert np.array_equal(one, base["y"])
    neg = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, shared_gate=np.full(N, -2.0, np.float32))["y"]
    scale = np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(2.0), dtype=np.float32))
    assert np.allclose(neg, folded + scale * sh, rtol=0, atol=1e-6 * float(np.abs(sh).max()))
    assert not np.array_equal(neg, half) and not np.array_equal(neg, one)


# ------------------------------------------------------------------ router ---
def _np_router_softmax(logits):
    """Independent numpy emulation of router_softmax's order (32 lanes, lane l
    holds columns l + 32k, per-lane left sums, XOR butterfly, reciprocal
    multiply), with the C library's expf."""
    x = np.where(np.isfinite(logits), logits, 0).astype(np.float32)
    n, e = x.shape
    lanes = x.reshape(n, e // 32, 32)                       # [t][k][l] = column l + 32k
    m = lanes.max(axis=(1, 2))
    w = O.expf_libm((lanes - m[:, None, None]).astype(np.float32))
    s = np.zeros((n, 32), np.float32)
    for k in range(e // 32):
        s = (s + w[:, k, :]).astype(np.float32)
    idx = np.arange(32)
    for d in (1, 2, 4, 8, 16):
        s = (s + s[:, idx ^ d]).astype(np.float32)
    inv = (np.float32(1) / s[:, 0]).astype(np.float32)
    return (w * inv[:, None, None]).astype(np.float32).reshape(n, e)


def _np_select(prob, k):
    n, e = prob.shape
    ids = np.empty((n, k), np.int32)
    ws = np.empty((n, k), np.float32)
    for t in range(n):
        order = np.lexsort((np.arange(e), -prob[t].astype(np.float64)))[:k]   # value desc, id asc
        b = np.zeros(32, np.float32)
        for i in order:
            b[i % 32] = np.float32(b[i % 32] + prob[t, i])
        for d in (1, 2, 4, 8, 16):
            b = (b + b[np.arange(32) ^ d]).astype(np.float32)
        den = max(b[0], np.float32(1.0 / 16384.0))
        ids[t] = order
        ws[t] = prob[t, order] * (np.float32(1) / np.float32(den))
    return ids, ws


def test_router_softmax_closed_forms():
    # Equal logits: every expf is 1, the total 512 exactly, each value 1/512.
    p, f = O.router_softmax(np.full((3, 512), 0.37, np.float32))
    assert f == 0 and np.all(p == np.float32(1 / 512))
    # One logit far above the rest: that value is exactly 1 (the others underflow).
    x = np.zeros((1, 512), np.float32)
    x[0, 77] = 200.0
    p, f = O.router_softmax(x)
    assert f == 0 and p[0, 77] == 1.0 and np.all(np.delete(p[0], 77) == 0)
    # A nonfinite logit zeroes the row and sets bit 1; other rows are untouched.
    x = np.random.default_rng(1).standard_normal((3, 512)).astype(np.float32)
    x[1, 5] = np.nan
    p, f = O.router_softmax(x)
    assert f == 1 and np.all(p[1] == 0) and np.all(p[0] > 0) and np.all(p[2] > 0)


def test_router_softmax_lane_order_rounding():
    # Hand-derived order case.  Sixteen small weights t = expf(-16.7) < 2^-24
    # sit in lane 0 (columns 0, 32, .., 480) and a 1.0 (logit 0, the max) in
    # lane 31 (column 31); every other logit underflows to weight 0.  In the
    # reference's order lane 0 first sums its sixteen t's to T, and the XOR
    # butterfly then adds lane 31's 1 to T, so the total is fl(T + 1) > 1.
    # A left-to-right column sum would reach the 1 after one t, absorb each
    # later t (t is below half an ulp of 1) and total exactly 1.
    a = np.float32(-16.7)
    t = O.expf_libm(np.array([a], np.float32))[0]
    assert 0 < t < np.float32(2.0 ** -24)
    x = np.full((2, 512), -300.0, np.float32)
    x[:, 31] = 0.0
    x[:, 0:512:32] = a
    x[1] = np.roll(x[1], 7)          # the same pattern moved to lanes 7 and 6
    p, f = O.router_softmax(x)
    assert f == 0
    T = np.float32(0)
    for _ in range(16):
        T = np.float32(T + t)
    s = np.float32(T + np.float32(1))
    assert s > 1
    inv = np.float32(1) / s
    for row, big, small in ((0, 31, slice(0, 512, 32)), (1, 38, slice(7, 512, 32))):
        assert p[row, big] == np.float32(np.float32(1) * inv) != 1.0
        assert np.all(p[row, small] == np.float32(t * inv))
        others = np.ones(512, bool)
        others[big] = False
        others[small] = False
        assert np.all(p[row, others] == 0)


def test_router_softmax_matches_independent_emulation():
    x = (np.random.default_rng(2).standard_normal((64, 512)) * 3).astype(np.float32)
    p, f = O.router_softmax(x)
    assert f == 0
    assert np.array_equal(p.view(np.uint32), _np_router_softmax(x).view(np.uint32))
    ref = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.max(np.abs(p - ref) / ref) < 4e-6   # the mathematics, to float32 rounding


def test_select_routes_ties_floor_and_bucket_order():
    rng = np.random.default_rng(3)
    p = rng.random((32, 512)).astype(np.float32)
    p[0, [3, 40, 77]] = 2.0                         # a three-way tie: ids ascending
    ids, w, f = O.select_routes(p, 10)
    assert f == 0 and list(ids[0, :3]) == [3, 40, 77]
    eids, ew = _np_select(p, 10)
    assert np.array_equal(ids, eids) and np.array_equal(w.view(np.uint32), ew.view(np.uint32))
    # The bucket tree is not a left-to-right sum: with a rank-order sum as the
    # denominator some rows' weights come out different.
    seq_w = np.empty_like(w)
    for t in range(32):
        acc = np.float32(0)
        for v in p[t, ids[t]]:
            acc = np.float32(acc + v)
        seq_w[t] = p[t, ids[t]] * (np.float32(1) / acc)
    assert np.any(seq_w != w)
    # Tiny probabilities: the 1/16384 floor applies.
    small = np.full((1, 512), 1e-7, np.float32)
    ids, w, f = O.select_routes(small, 10)
    assert f == 0 and list(ids[0]) == list(range(10))
    assert np.all(w == np.float32(1e-7) * np.float32(16384.0))
    # Softmax of uniform logits: ten equal weights of exactly fl(0.1).
    ids, w, f = O.select_routes(np.full((1, 512), np.float32(1 / 512)), 10)
    assert np.all(w == np.float32(0.1))


def test_router_softmax_lane_order_pinned_by_absorption():
    """Hand-derived cases that fix router_softmax's summation order
    (src/hip/session_ops.hip:401-434): lane l holds logits l + 32j, each lane
    sums its values left to right from +0, and the 32 lane sums meet in an XOR
    butterfly.  delta = expf(x_d) ~ 0.7 * 2^-24 is below half an ulp of 1, so
    1 + delta rounds back to 1 while delta + delta = 1.4 * 2^-24 does not."""
    x_d = np.float32(np.log(0.7) - 24 * np.log(2.0))
    far = np.float32(-200.0)                         # expf underflows to exactly 0
    # (a) Logits 0, 32, ..., 480 share lane 0; the 1 comes first, so each delta
    # is absorbed and the total is exactly 1: p = expf(x) * (1/1).
    x = np.full((1, 512), far, np.float32)
    x[0, 0] = 0.0
    x[0, 32::32] = x_d
    p, f = O.router_softmax(x)
    e = O.expf_libm(np.array([x_d], np.float32))[0]
    assert f == 0 and p[0, 0] == 1.0 and np.all(p[0, 32::32] == e)
    # (b) Same lane, the 1 last (logit 480): fifteen deltas are summed first
    # and survive the add of 1, so the total exceeds 1 and p[480] < 1.
    x = np.full((1, 512), far, np.float32)
    x[0, 480] = 0.0
    x[0, 0:480:32] = x_d
    p, f = O.router_softmax(x)
    assert f == 0 and p[0, 480] < 1.0
    # (c) One value per lane (logits 0..31): lane 0 holds the 1, lanes 1..31 a
    # delta.  The butterfly pairs equal partial sums (2, 4, 8, 16 deltas,
    # exact doublings) before they reach lane 0:
    #   1 + 2d -> 1 + 1 ulp, + 4d -> 1 + 2 ulp, + 8d -> 1 + 5 ulp,
    #   + 16d -> 1 + 11 ulp  (ulp = 2^-23; none of these near a tie),
    # whereas a left-to-right sum over lanes would absorb every delta (total 1).
    x = np.full((1, 512), far, np.float32)
    x[0, 0] = 0.0
    x[0, 1:32] = x_d
    p, f = O.router_softmax(x)
    total = np.float32(1.0 + 11 * 2.0 ** -23)
    assert f == 0 and p[0, 0] == np.float32(1.0) / total


def test_combine_flags_closed_forms():
    """The fold's error semantics (routed_fold, then shared_sigmoid_add:
    src/hip/session_ops.hip:307-324, 375-391; operand/arithmetic :161-169)."""
    c = np.array([[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]], np.float32)
    w = np.array([[0.5, 0.25, 0.125]], np.float32)
    s = np.array([[10.0, 20.0]], np.float32)
    # Finite: the plain fold plus the shared row (gate absent: scale 1).
    y, f = O.combine_flags(c, w, shared=s)
    assert f == 0 and np.array_equal(y, O.routed_fold(c, w) + s)
    # A NaN contribution: bit 1, the routed value of that element becomes 0,
    # the shared add still happens from 0 (the other element is untouched).
    cb = c.copy()
    cb[0, 1, 0] = np.nan
    y, f = O.combine_flags(cb, w, shared=s)
    assert f == 1 and y[0, 0] == 10.0 and y[0, 1] == np.float32(0.5 * 2 + 0.25 * 4 + 0.125 * 6 + 20)
    # With a gate of 0 the shared scale is exactly 1/2: y = 0 + 0.5 * 10.
    y, f = O.combine_flags(cb, w, shared=s, shared_gate=np.zeros(1, np.float32))
    assert f == 1 and y[0, 0] == 5.0
    # An overflowing product is an arithmetic flag (bit 2) and reads as 0.
    cb = c.copy()
    cb[0, 0, 1] = np.float32(3e38)
    wb = w.copy()
    wb[0, 0] = 4.0
    y, f = O.combine_flags(cb, wb, shared=s)
    assert f == 2 and y[0, 1] == 20.0 and y[0, 0] == np.float32(4 * 1 + 0.25 * 3 + 0.125 * 5 + 10)
    # A nonfinite shared value zeroes the output element (bit 1).
    sb = s.copy()
    sb[0, 1] = np.inf
    y, f = O.combine_flags(c, w, shared=sb)
    assert f == 1 and y[0, 1] == 0.0 and y[0, 0] == np.float32(0.5 + 0.75 + 0.625 + 10)
    # A nonfinite gate zeroes the whole token row (bit 1), routed part included.
    y, f = O.combine_flags(c, w, shared=s, shared_gate=np.array([np.nan], np.float32))
    assert f == 1 and np.all(y == 0)
    # No shared expert: only the routed fold, with its flags.
    y, f = O.combine_flags(cb, wb)
    assert f == 2 and y[0, 1] == 0.0
