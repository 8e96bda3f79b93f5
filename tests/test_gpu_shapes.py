"""GPU parity of whole layers at shapes other than the benchmark's 2048/512:
the reference model's own 2560/640 (lanes holding several blocks: the wide
streaming gate/up kernel, the MFMA kernel's multi-block fold, the wide down
kernel, the decode kernels' two-blocks-per-lane forms) and a narrower
1024/256 (lanes past the row end: the decode and lean kernels' partial-row
forms, the MFMA kernel's staged fold).

On every path each middle Q8 row equals the oracle's byte for byte (the
gate/up kernels follow the reference's fp32 order, src/cpu_expert.cpp:156-213);
outputs are bit-identical where the down kernel keeps that order too (the
decode and lean streaming kernels, one or two blocks per lane) and within
1e-5 rms on the MFMA down kernel.
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


def q8_bytes(q):
    return np.ascontiguousarray(q).view(np.uint8).reshape(-1)


def _layer_env(env, *args, **kw):
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


@pytest.fixture(scope="module", autouse=True)
def gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


PATHS = {
    "decode": {"MOE_FFN_DECODE": 1},
    "stream": {"MOE_FFN_DECODE": 0, "MOE_FFN_MFMA_MIN": 0},
    "mfma": {"MOE_FFN_DECODE": 0, "MOE_FFN_MFMA_MIN": 1},
    "auto": {},
}


# (1344, 512): 10.5 row slices of 128, so the down kernel's last
# four-slice work unit is short and its last slice half empty.  (1024, 384)
# and (512, 128): 12 and 4 down blocks per row, where the down kernel takes
# one slice per work unit and its 8-block weight window does not wrap.
# (2112, 544) and (3072, 1024): 66 and 96 gate/up blocks per row (the
# shortest layer row past 64 blocks, hidden being a multiple of 64, and the
# longest row of the MFMA gate/up form whose reference lanes chain a second
# block; the decode gate/up's spread and plain two-slot forms)
# with 17 and 32 down blocks (the MFMA down kernel's second staging round
# holding one block and a full 16).  (4096, 256): 128 gate/up blocks, the
# MFMA gate/up form that chains every block through per-block loads.
@pytest.mark.parametrize("H,I", [(2560, 640), (1024, 256), (1344, 512), (1024, 384), (512, 128), (2112, 544),
                                 (3072, 1024), (4096, 256)])
@pytest.mark.parametrize("path", list(PATHS))
def test_layer_shape_paths(H, I, path):
    E, K, N = 16, 4, 40
    if path == "decode" and (H > 4096 or I > 1024):
        pytest.skip("the decode kernels cover H <= 4096 and I <= 1024")
    bank = W.q4_bank(E, hidden=H, intermediate=I, seed=H + I)
    shared = W.q4_bank(1, hidden=H, intermediate=I, seed=H + I + 1)
    x = W.activations(N, hidden=H, seed=H + 2)
    ids, w = W.routes_zipf(N, 1.0, experts=E, k=K, seed=I + 3)
    g = np.random.default_rng(H + 4).standard_normal(N).astype(np.float32)
    L = _layer_env(PATHS[path], H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
    y, err = L.forward(dev(x), dev(ids), dev(w), shared_gate=dev(g))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, shared_gate=g)
    dbg = L.debug_last(N)
    assert np.array_equal(host(dbg["x_q8"]).reshape(-1), q8_bytes(ref["x_q8"]))
    # every middle Q8 row against the oracle's cpu_expert middle
    nbi = I // 32
    mid = host(dbg["middle_q8"]).reshape(-1, nbi * 36)
    groups = O.route_groups(ids, w, E)
    P = int(groups["offsets"][-1])
    eb = len(bank) // E
    mb = eb // 3
    xq = O.quantize_q8(x)
    for p in range(P + N):
        if p < P:
            t, e_bytes = int(groups["token"][p]), bank[int(groups["expert"][p]) * eb:(int(groups["expert"][p]) + 1) * eb]
        else:
            t, e_bytes = p - P, shared
        ro = O.expert_forward(e_bytes[:mb], e_bytes[mb:2 * mb], e_bytes[2 * mb:], H, I, xq[t:t + 1])
        assert np.array_equal(mid[p], q8_bytes(ro["middle_q8"])), (path, p)
    exact = path in ("decode", "stream")
    if exact:
        assert np.array_equal(yh.view(np.uint32), ref["y"].view(np.uint32))
    else:
        err_ = float(np.max(np.abs(yh.astype(np.float64) - ref["y"])))
        scale = float(np.sqrt(np.mean(np.square(ref["y"].astype(np.float64)))))
        assert err_ <= 1e-5 * scale, (path, err_, scale)
    L.close()


def test_reference_shape_grouped_layer_multi_tile_items():
    """The reference model's shape (2560/640, Q4_0 downs) on a batch whose
    groups span several 32-pair token tiles and several 128-pair items (600
    tokens, 64 experts + shared, top-8, Zipf(1.1)), every group on the MFMA
    path: the gate/up form whose reference lanes chain a second block and the
    20-block down kernel that takes two slices per workgroup.  Sampled tokens
    against the oracle (outputs within 1e-5 rms); every token's middle Q8 rows
    equal to the streaming path's, whose order is the reference's, and every
    output within 1e-5 rms of it; deterministic."""
    H, I, E, K, N = 2560, 640, 64, 8, 600
    bank = W.q4_bank(E, hidden=H, intermediate=I, seed=91)
    shared = W.q4_bank(1, hidden=H, intermediate=I, seed=92)
    x = W.activations(N, hidden=H, seed=93)
    ids, w = W.routes_zipf(N, 1.1, experts=E, k=K, seed=94)
    sizes = np.bincount(ids.reshape(-1), minlength=E)
    assert sizes.max() > 128   # at least one group of several items
    L = _layer_env(PATHS["mfma"], H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    st = L.last_stats()
    assert st["stream_items"] == 0 and st["mfma_items"] > E
    sample = np.random.default_rng(95).choice(N, 12, replace=False)
    mask = np.zeros(N, np.uint8)
    mask[sample] = 1
    ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, token_mask=mask)
    ref_y = ref["y"][sample].astype(np.float64)
    scale = float(np.sqrt(np.mean(np.square(ref_y))))
    assert float(np.max(np.abs(yh[sample].astype(np.float64) - ref_y))) <= 1e-5 * scale
    S = _layer_env(PATHS["stream"], H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
    ys, es = S.forward(dev(x), dev(ids), dev(w))
    ysh = host(ys)
    assert int(host(es)[0]) == 0 and S.last_stats()["mfma_items"] == 0
    assert np.array_equal(host(S.debug_last(N)["middle_q8"]), host(L.debug_last(N)["middle_q8"]))
    s_all = float(np.sqrt(np.mean(np.square(ysh.astype(np.float64)))))
    assert float(np.max(np.abs(yh.astype(np.float64) - ysh))) <= 1e-5 * s_all
    S.close()
    y2, _ = L.forward(dev(x), dev(ids), dev(w))
    assert np.array_equal(host(y2), yh)
    L.close()


EXTREME_SHAPES = [
    # H, I, down type: rows past every specialised form, and the smallest layer
    (4160, 2080, moe_ffn.DOWN_Q4_0),   # 130 gate/up blocks (H > 4096: the streaming gate/up re-reads its rows per
                                       # token, the MFMA gate/up chains blocks through per-block loads); 65 down
                                       # blocks (the streaming down's 64-lane rows, the MFMA down's tile form)
    (4160, 2080, moe_ffn.DOWN_Q4_1),
    (1024, 1088, moe_ffn.DOWN_Q4_1),   # 34 down blocks with Q4_1 mins; the decode path stops at 32
    (64, 32, moe_ffn.DOWN_Q4_0),       # 2 gate/up blocks and 1 down block a row
    (16384, 64, moe_ffn.DOWN_Q4_0),    # the longest gate/up rows: 512 blocks, 8 per lane
    (64, 16384, moe_ffn.DOWN_Q4_1),    # the longest down rows: 512 blocks, 8 per lane
]


@pytest.mark.parametrize("H,I,down", EXTREME_SHAPES)
@pytest.mark.parametrize("path", list(PATHS))
def test_layer_extreme_shapes(H, I, down, path):
    """Layers at shapes the benchmark never uses, on every path: each middle
    Q8 row equals the oracle's cpu_expert middle byte for byte; outputs are
    bit-identical on the decode and streaming paths (the reference's fp32
    order for any row length) and within 1e-5 rms on the MFMA down."""
    E, K, N = 8, 2, 24
    q41 = down == moe_ffn.DOWN_Q4_1
    if path == "decode" and (H > 4096 or I > 1024):
        pytest.skip("the decode kernels cover H <= 4096 and I <= 1024")
    bank = W.q4_bank(E, hidden=H, intermediate=I, seed=H + 3 * I, down_type=1 if q41 else 0)
    shared = W.q4_bank(1, hidden=H, intermediate=I, seed=H + 3 * I + 1, down_type=1 if q41 else 0)
    x = W.activations(N, hidden=H, seed=H + 5)
    ids, w = W.routes_zipf(N, 1.0, experts=E, k=K, seed=I + 7)
    L = _layer_env(PATHS[path], H, I, E, K, True, N, experts_q4=bank, shared_q4=shared, down_type=down)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, down_q41=q41)
    dbg = L.debug_last(N)
    assert np.array_equal(host(dbg["x_q8"]).reshape(-1), q8_bytes(ref["x_q8"]))
    nbi = I // 32
    mid = host(dbg["middle_q8"]).reshape(-1, nbi * 36)
    groups = O.route_groups(ids, w, E)
    P = int(groups["offsets"][-1])
    eb = len(bank) // E
    mb = (H // 32) * I * 18
    xq = O.quantize_q8(x)
    for p in range(P + N):
        if p < P:
            t, e_bytes = int(groups["token"][p]), bank[int(groups["expert"][p]) * eb:(int(groups["expert"][p]) + 1) * eb]
        else:
            t, e_bytes = p - P, shared
        ro = O.expert_forward(e_bytes[:mb], e_bytes[mb:2 * mb], e_bytes[2 * mb:], H, I, xq[t:t + 1], down_q41=q41)
        assert np.array_equal(mid[p], q8_bytes(ro["middle_q8"])), (path, p)
    if path in ("decode", "stream"):
        assert np.array_equal(yh.view(np.uint32), ref["y"].view(np.uint32)), path
    else:
        err_ = float(np.max(np.abs(yh.astype(np.float64) - ref["y"])))
        scale = float(np.sqrt(np.mean(np.square(ref["y"].astype(np.float64)))))
        assert err_ <= 1e-5 * scale, (path, err_, scale)
    # The same rows as canonical Q8_1 input (moe_ffn_forward_q8): the same bits.
    yq, errq = L.forward_q8(dev(q8_bytes(ref["x_q8"]).reshape(N, -1)), dev(ids), dev(w))
    assert int(host(errq)[0]) == 0
    assert np.array_equal(host(yq).view(np.uint32), yh.view(np.uint32)), (path, "forward_q8")
    L.close()


@pytest.mark.parametrize("E", [1024, 4096])
@pytest.mark.parametrize("N", [16, 300])
def test_layer_many_experts(E, N):
    """Up to the 4096 experts a layer accepts, on both grouping forms (one
    workgroup at 16 tokens, the multi-kernel form at 300): every middle Q8
    row byte-equal to the oracle's, outputs within 1e-5 rms (bit-identical
    where every group streams)."""
    H, I, K = 64, 32, 8
    bank = W.q4_bank(E, hidden=H, intermediate=I, seed=E + N)
    shared = W.q4_bank(1, hidden=H, intermediate=I, seed=E + N + 1)
    x = W.activations(N, hidden=H, seed=E + 2)
    ids, w = W.routes_zipf(N, 1.1, experts=E, k=K, seed=N + 3)
    L = moe_ffn.MoeLayer(H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
    y, err = L.forward(dev(x), dev(ids), dev(w))
    yh = host(y)
    assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh))
    ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared)
    dbg = L.debug_last(N)
    nbi = I // 32
    mid = host(dbg["middle_q8"]).reshape(-1, nbi * 36)
    groups = O.route_groups(ids, w, E)
    P = int(groups["offsets"][-1])
    eb = len(bank) // E
    mb = eb // 3
    xq = O.quantize_q8(x)
    for p in range(P + N):
        if p < P:
            t, e_bytes = int(groups["token"][p]), bank[int(groups["expert"][p]) * eb:(int(groups["expert"][p]) + 1) * eb]
        else:
            t, e_bytes = p - P, shared
        ro = O.expert_forward(e_bytes[:mb], e_bytes[mb:2 * mb], e_bytes[2 * mb:], H, I, xq[t:t + 1])
        assert np.array_equal(mid[p], q8_bytes(ro["middle_q8"])), (E, N, p)
    err_ = float(np.max(np.abs(yh.astype(np.float64) - ref["y"])))
    scale = float(np.sqrt(np.mean(np.square(ref["y"].astype(np.float64)))))
    assert err_ <= 1e-5 * scale, (E, N, err_, scale)
    L.close()


def _random_configs(n, seed):
    """Seeded layer configurations inside the ranges the shape tests cover
    (H multiple of 64 up to 4096, I multiple of 32 up to 1024)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        H = 64 * int(rng.integers(1, 65))
        I = 32 * int(rng.integers(1, 33))
        E = int(rng.choice([1, 2, 3, 7, 16, 33, 64]))
        k = int(rng.integers(1, min(E, 20) + 1))
        shared = bool(rng.integers(0, 2))
        q41 = bool(rng.integers(0, 2))
        N = int(rng.choice([1, 2, 5, 17, 40, 96]))
        out.append((H, I, E, k, shared, q41, N))
    return out


@pytest.mark.parametrize("cfg", _random_configs(16, 2026))
def test_layer_random_configs(cfg):
    """Seeded random layers (hidden, intermediate, experts, top-k, shared
    expert or not, Q4_0 or Q4_1 downs, batch size) on every path they allow:
    every middle Q8 row byte-equal to the oracle's; outputs bit-identical on
    the streaming path and, where it applies, the decode path, within 1e-5
    rms on the MFMA path and the automatic choice."""
    H, I, E, k, shared, q41, N = cfg
    down = moe_ffn.DOWN_Q4_1 if q41 else moe_ffn.DOWN_Q4_0
    seed = H * 7 + I * 3 + E + k + N
    bank = W.q4_bank(E, hidden=H, intermediate=I, seed=seed, down_type=1 if q41 else 0)
    sh = W.q4_bank(1, hidden=H, intermediate=I, seed=seed + 1, down_type=1 if q41 else 0) if shared else None
    x = W.activations(N, hidden=H, seed=seed + 2)
    ids, w = W.routes_zipf(N, 1.0, experts=E, k=k, seed=seed + 3)
    ref = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=sh, down_q41=q41)
    groups = O.route_groups(ids, w, E)
    P = int(groups["offsets"][-1])
    eb = len(bank) // E
    mb = (H // 32) * I * 18
    xq = O.quantize_q8(x)
    middles = []
    for p in range(P + (N if shared else 0)):
        if p < P:
            t, e_bytes = int(groups["token"][p]), bank[int(groups["expert"][p]) * eb:(int(groups["expert"][p]) + 1) * eb]
        else:
            t, e_bytes = p - P, sh
        ro = O.expert_forward(e_bytes[:mb], e_bytes[mb:2 * mb], e_bytes[2 * mb:], H, I, xq[t:t + 1], down_q41=q41)
        middles.append(q8_bytes(ro["middle_q8"]))
    decode_fits = H <= 4096 and I <= 1024 and k + (1 if shared else 0) <= 16
    for path in PATHS:
        if path == "decode" and not decode_fits:
            continue
        L = _layer_env(PATHS[path], H, I, E, k, shared, N, experts_q4=bank, shared_q4=sh, down_type=down)
        y, err = L.forward(dev(x), dev(ids), dev(w))
        yh = host(y)
        assert int(host(err)[0]) == 0 and np.all(np.isfinite(yh)), (cfg, path)
        mid = host(L.debug_last(N)["middle_q8"]).reshape(-1, (I // 32) * 36)
        for p, m in enumerate(middles):
            assert np.array_equal(mid[p], m), (cfg, path, p)
        if path in ("decode", "stream"):
            assert np.array_equal(yh.view(np.uint32), ref["y"].view(np.uint32)), (cfg, path)
        else:
            err_ = float(np.max(np.abs(yh.astype(np.float64) - ref["y"])))
            scale = float(np.sqrt(np.mean(np.square(ref["y"].astype(np.float64)))))
            assert err_ <= 1e-5 * scale, (cfg, path, err_, scale)
        L.close()


@pytest.mark.parametrize("N", [8, 300])
def test_two_layers_on_two_streams(N):
    """Two layer handles forwarding at once on two streams (decode path at 8
    tokens, grouped at 300) give the bits each gives alone: no state is
    shared between handles."""
    H, I, E, K = 1024, 256, 64, 8
    layers, inputs, alone = [], [], []
    for j in range(2):
        bank = W.q4_bank(E, hidden=H, intermediate=I, seed=300 + j)
        shared = W.q4_bank(1, hidden=H, intermediate=I, seed=310 + j)
        L = moe_ffn.MoeLayer(H, I, E, K, True, N, experts_q4=bank, shared_q4=shared)
        x = dev(W.activations(N, hidden=H, seed=320 + j))
        ids, w = W.routes_zipf(N, 1.1, experts=E, k=K, seed=330 + j)
        inp = (x, dev(ids), dev(w))
        y, err = L.forward(*inp)
        alone.append(host(y).copy())
        assert int(host(err)[0]) == 0
        layers.append(L)
        inputs.append(inp)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for _ in range(3):
        for j in range(2):
            y = torch.empty((N, H), dtype=torch.float32, device=DEV)
            err = torch.zeros(1, dtype=torch.int32, device=DEV)
            streams[j].wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(streams[j]):
                layers[j].forward(*inputs[j], y=y, error=err, stream=streams[j])
            outs.append((j, y, err))
    torch.cuda.synchronize()
    for j, y, err in outs:
        assert int(host(err)[0]) == 0
        assert np.array_equal(host(y).view(np.uint32), alone[j].view(np.uint32)), (N, j)
    for L in layers:
        L.close()
