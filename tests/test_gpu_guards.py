"""Memory-safety checks of the device path, in the manner of the reference's
MoE fixtures (tests/moe_route_copy_test.hip:41, 79-111): every caller buffer
sits inside one arena filled with 0xa5, with guard bands before and after it;
after each call the guard bytes must still be 0xa5 and the read-only inputs
unchanged.  And, as the reference proves for its CPU jobs
(tests/cpu_expert_test.cpp:25-55), the hot path allocates nothing: 100
forwards leave the device's free memory (hipMemGetInfo) unchanged.

Paths covered: quantize, device router, the decode path (8 tokens), grouped
streaming (64 tokens), grouped MFMA + streaming (1024 tokens, Zipf 1.1), a
Q4_1-down layer (decode and grouped), forward_q8, debug_last's middle rows,
the combine, and the quantized linear (vector and MFMA kernels).
"""
import numpy as np
import pytest

import moe_ffn
import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
DEV = "cuda:0"
GUARD = 4096
FILL = 0xA5


@pytest.fixture(scope="module", autouse=True)
def gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


class Arena:
    """Caller buffers carved out of one 0xa5-filled device allocation, each
    256-byte aligned with at least GUARD guard bytes on both sides."""

    def __init__(self, nbytes):
        self.buf = torch.full((nbytes,), FILL, dtype=torch.uint8, device=DEV)
        self.off = GUARD
        self.regions = []
        self.inputs = []

    def take(self, shape, dtype, init=None, readonly=False):
        n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
        start = (self.off + 255) // 256 * 256
        end = start + n
        assert end + GUARD <= self.buf.numel(), "arena too small"
        t = self.buf[start:end].view(dtype).view(shape)
        if init is not None:
            t.copy_(torch.from_numpy(np.ascontiguousarray(init)).to(DEV))
        self.regions.append((start, end))
        if readonly:
            self.inputs.append((t, t.clone()))
        self.off = end + GUARD
        return t

    def check(self, what):
        torch.cuda.synchronize()
        h = self.buf.cpu().numpy()
        mask = np.ones(h.size, bool)
        for s, e in self.regions:
            mask[s:e] = False
        bad = np.flatnonzero(h[mask] != FILL)
        assert bad.size == 0, f"{what}: {bad.size} guard bytes changed (first at arena offset {np.flatnonzero(mask)[bad[0]]})"
        for t, ref in self.inputs:
            assert torch.equal(t, ref), f"{what}: a read-only input changed"


def _forward_case(L, N, routing, seed, gated=False, q8_input=False):
    x = W.activations(N, seed=seed)
    ids, w = (W.routes_uniform(N, seed=seed + 1) if routing == "uniform" else
              W.routes_zipf(N, 1.1, seed=seed + 1))
    A = Arena(64 << 20)
    xt = A.take((N, L.H), torch.float32, x, readonly=True)
    xq = None
    if q8_input:
        xq = A.take((N, L.H // 32 * 36), torch.uint8, np.ascontiguousarray(O.quantize_q8(x)).view(np.uint8).reshape(N, -1),
                    readonly=True)
    it = A.take((N, L.k), torch.int32, ids, readonly=True)
    wt = A.take((N, L.k), torch.float32, w, readonly=True)
    gt = A.take((N,), torch.float32, np.random.default_rng(seed + 2).standard_normal(N).astype(np.float32),
                readonly=True) if gated else None
    y = A.take((N, L.H), torch.float32)
    err = A.take((1,), torch.int32, np.zeros(1, np.int32))
    if q8_input:
        L.forward_q8(xq, it, wt, shared_gate=gt, y=y, error=err)
    else:
        L.forward(xt, it, wt, shared_gate=gt, y=y, error=err)
    A.check(f"forward N={N} {routing}")
    assert int(err.cpu()[0]) == 0 and bool(torch.isfinite(y).all())
    # debug_last copies of the x Q8 rows, the middle rows and the grouped routes.
    P = N * L.k + (N if L.has_shared else 0)
    xq_d = A.take((N, L.H // 32 * 36), torch.uint8)
    mq_d = A.take((P, L.I // 32 * 36), torch.uint8)
    rt = A.take((N * L.k,), torch.int32)
    rr = A.take((N * L.k,), torch.int32)
    st = moe_ffn.library().moe_ffn_debug_last(L.handle, moe_ffn._ptr(xq_d), moe_ffn._ptr(mq_d), moe_ffn._ptr(rt),
                                              moe_ffn._ptr(rr), moe_ffn._stream(None))
    assert st == 0
    A.check(f"debug_last N={N} {routing}")
    assert int(err.cpu()[0]) == 0, "debug_last wrote into the forward's error word"
    return y


@pytest.fixture(scope="module")
def layer512():
    L = moe_ffn.MoeLayer(2048, 512, 512, 10, True, 1024, synthetic_seed=3100)
    yield L
    L.close()


@pytest.mark.parametrize("N,routing", [(8, "uniform"), (64, "uniform"), (1024, "zipf")])
def test_forward_guards(layer512, N, routing):
    """Decode (8 tokens), grouped streaming (64) and MFMA + streaming (1024)."""
    _forward_case(layer512, N, routing, seed=3200 + N)
    _forward_case(layer512, N, routing, seed=3300 + N, gated=True)


@pytest.mark.parametrize("N", [8, 300])
def test_forward_q8_guards(layer512, N):
    _forward_case(layer512, N, "zipf", seed=3400 + N, q8_input=True)


@pytest.mark.parametrize("N,routing", [(8, "uniform"), (300, "zipf")])
def test_q41_down_guards(N, routing):
    L = moe_ffn.MoeLayer(2048, 512, 64, 10, True, 300, synthetic_seed=3500, down_type=moe_ffn.DOWN_Q4_1)
    x = W.activations(N, seed=3600)
    ids, w = (W.routes_uniform(N, experts=64, seed=3601) if routing == "uniform" else
              W.routes_zipf(N, 1.1, experts=64, seed=3601))
    A = Arena(32 << 20)
    xt = A.take((N, 2048), torch.float32, x, readonly=True)
    it = A.take((N, 10), torch.int32, ids, readonly=True)
    wt = A.take((N, 10), torch.float32, w, readonly=True)
    y = A.take((N, 2048), torch.float32)
    err = A.take((1,), torch.int32, np.zeros(1, np.int32))
    L.forward(xt, it, wt, y=y, error=err)
    A.check(f"Q4_1 forward N={N}")
    assert int(err.cpu()[0]) == 0
    L.close()


def test_quantize_router_combine_guards():
    rng = np.random.default_rng(3700)
    A = Arena(32 << 20)
    x = A.take((37, 2048), torch.float32, rng.standard_normal((37, 2048)).astype(np.float32), readonly=True)
    q = A.take((37, 64 * 36), torch.uint8)
    err = A.take((1,), torch.int32, np.zeros(1, np.int32))
    lib = moe_ffn.library()
    assert lib.moe_quantize_q8_1(moe_ffn._ptr(x), moe_ffn._ptr(q), 2048, 37, moe_ffn._ptr(err),
                                 moe_ffn._stream(None)) == 0
    A.check("quantize")
    lg = A.take((19, 512), torch.float32, rng.standard_normal((19, 512)).astype(np.float32), readonly=True)
    p = A.take((19, 512), torch.float32)
    ids = A.take((19, 10), torch.int32)
    w = A.take((19, 10), torch.float32)
    moe_ffn.router_select(lg, top_k=10, error=err, ids=ids, weights=w)
    assert lib.moe_router_select(moe_ffn._ptr(lg), 19, 512, 10, moe_ffn._ptr(p), moe_ffn._ptr(ids), moe_ffn._ptr(w),
                                 moe_ffn._ptr(err), moe_ffn._stream(None)) == 0
    A.check("router")
    c = A.take((9, 10, 2048), torch.float32, rng.standard_normal((9, 10, 2048)).astype(np.float32), readonly=True)
    cw = A.take((9, 10), torch.float32, rng.random((9, 10)).astype(np.float32), readonly=True)
    s = A.take((9, 2048), torch.float32, rng.standard_normal((9, 2048)).astype(np.float32), readonly=True)
    g = A.take((9,), torch.float32, rng.standard_normal(9).astype(np.float32), readonly=True)
    y = A.take((9, 2048), torch.float32)
    assert lib.moe_combine(moe_ffn._ptr(c), moe_ffn._ptr(cw), moe_ffn._ptr(s), moe_ffn._ptr(g), 9, 10, 2048,
                           moe_ffn._ptr(y), moe_ffn._ptr(err), moe_ffn._stream(None)) == 0
    A.check("combine")
    assert int(err.cpu()[0]) == 0


@pytest.mark.parametrize("K,M,N", [(2048, 2048, 1), (2048, 2048, 8), (2048, 2048, 256), (2560, 640, 33)])
def test_linear_guards(K, M, N):
    """Vector kernel (1, 8 and 33 columns) and MFMA kernel (256 columns)."""
    rng = np.random.default_rng(K + M + N)
    lin = moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, K, M, W.q4_blocks(M * K // 32, rng).reshape(-1), max_columns=N)
    A = Arena(16 << 20)
    x = A.take((N, K), torch.float32, rng.standard_normal((N, K)).astype(np.float32), readonly=True)
    y = A.take((N, M), torch.float32)
    err = A.take((1,), torch.int32, np.zeros(1, np.int32))
    lin.apply(x, y=y, error=err)
    A.check(f"linear apply {K}x{M} N={N}")
    xq = A.take((N, K // 32 * 36), torch.uint8, np.ascontiguousarray(O.quantize_q8(x.cpu().numpy())).view(np.uint8)
                .reshape(N, -1), readonly=True)
    y2 = A.take((N, M), torch.float32)
    lin.forward_q8(xq, N, y=y2)
    A.check(f"linear forward_q8 {K}x{M} N={N}")
    assert torch.equal(y, y2) and int(err.cpu()[0]) == 0
    lin.close()


def test_forwards_allocate_nothing(layer512):
    """100 forwards (decode, grouped streaming and grouped MFMA batches, with
    caller-owned outputs) leave the device's free memory unchanged."""
    cases = []
    for N, routing in ((8, "uniform"), (64, "uniform"), (1024, "zipf")):
        ids, w = (W.routes_uniform(N, seed=3800 + N) if routing == "uniform" else W.routes_zipf(N, 1.1, seed=3800 + N))
        x = torch.from_numpy(W.activations(N, seed=3900 + N)).to(DEV)
        cases.append((x, torch.from_numpy(ids).to(DEV), torch.from_numpy(w).to(DEV),
                      torch.empty((N, 2048), dtype=torch.float32, device=DEV)))
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    for x, i, w, y in cases:   # first launches load code objects
        layer512.forward(x, i, w, y=y, error=err)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for n in range(100):
        x, i, w, y = cases[n % 3]
        layer512.forward(x, i, w, y=y, error=err)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"free device memory changed by {free0 - free1} bytes over 100 forwards"
    assert int(err.cpu()[0]) == 0
