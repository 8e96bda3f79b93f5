"""GPU parity of the quantized linear projections (moe_linear_*, the
counterpart of the reference's launch_quantized_linear{,_short,_tiled} and
Matrix::apply for Q4_0 / Q4_1 weights).

The reference's MMVQ kernel and its CPU expert share one fp32 order
(src/hip/linear.hip:195-262, src/cpu_expert.cpp:156-213), so:
  * the compiled reference's cpu_expert gate, up and down outputs at its
    2560/640 shape (golden fixtures) are matched bit for bit;
  * every other shape is matched bit for bit against the oracle's restatement
    of that order (pinned bitwise against the same fixtures), including rows
    whose 64-lane slots hold several blocks (K > 2048), partial slots, row
    counts that are not multiples of 8 and column counts past one tile.
"""
import os

import numpy as np
import pytest

import moe_ffn
import oracle as O
from golden_inputs import expert_weights, q4_1_matrix, q4_matrix

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
Q40, Q41 = moe_ffn.TYPE_Q4_0, moe_ffn.TYPE_Q4_1


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_bytes(q):
    return np.ascontiguousarray(q).view(np.uint8).reshape(-1)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module", autouse=True)
def gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def test_linear_reference_expert_matrices_vs_golden():
    """The reference cpu_expert's three projections at 2560/640 (gate / up:
    Q4_0 2560 -> 640, 80 blocks a row; down: Q4_0 or Q4_1 640 -> 2560) as
    standalone linear layers: outputs bit-identical to the compiled
    reference's."""
    f = np.load(os.path.join(GOLDEN, "cpu_expert_2560x640.npz"), allow_pickle=False)
    g, u, d = expert_weights(2560, 640)
    xq = f["x_q8"].reshape(3, -1)
    for w, ref, what in ((g, f["gate"], "gate"), (u, f["up"], "up")):
        L = moe_ffn.MoeLinear(Q40, 2560, 640, w)
        assert np.array_equal(bits(host(L.forward_q8(dev(xq), 3))), bits(ref)), what
        L.close()
    mq = f["middle_q8"].reshape(3, -1)
    L = moe_ffn.MoeLinear(Q40, 640, 2560, d)
    assert np.array_equal(bits(host(L.forward_q8(dev(mq), 3))), bits(f["y"])), "down Q4_0"
    L.close()
    f41 = np.load(os.path.join(GOLDEN, "cpu_expert_2560x640_q41.npz"), allow_pickle=False)
    d41 = q4_1_matrix(404, 640, 2560)
    mq41 = f41["middle_q8"].reshape(3, -1)
    L = moe_ffn.MoeLinear(Q41, 640, 2560, d41)
    assert np.array_equal(bits(host(L.forward_q8(dev(mq41), 3))), bits(f41["y"])), "down Q4_1"
    L.close()


def _weights(type_, K, M, seed):
    return q4_1_matrix(seed, K, M) if type_ == Q41 else q4_matrix(seed, K, M)


def _oracle(type_, w, K, M, xq):
    return O.matrix_gpu_order_q41(w, K, M, xq) if type_ == Q41 else O.matrix_gpu_order(w, K, M, xq)


def _columns(K, N, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((N, K)) * np.exp2(rng.integers(-6, 6, (N, 1)))).astype(np.float32)
    return x, O.quantize_q8(x)


CASES = [
    # type, K, M, N
    (Q40, 32, 1, 1),          # one block, one row (7 padding rows)
    (Q40, 2048, 2048, 1),     # decode projection, one block per lane
    (Q40, 2080, 1000, 1),     # 65 blocks, one column: both slots per load round
    (Q40, 6144, 40, 1),       # three slots, two held per round (odd count)
    (Q40, 2048, 13, 5),       # rows not a multiple of 8
    (Q40, 2080, 1000, 8),     # 65 blocks: lane 0 holds two
    (Q40, 4096, 264, 33),     # two full slots, several column groups
    (Q40, 16384, 64, 3),      # 512 blocks: eight slots per lane
    (Q41, 2560, 200, 9),
    (Q41, 6144, 40, 2),       # three slots, one per load round
    (Q41, 6144, 40, 1),       # three slots, two held per round (odd count)
    (Q41, 2560, 200, 1),      # 80 blocks, both slots held
    (Q40, 2048, 512, 128),    # the reference's tiled maximum
    (Q40, 1024, 256, 300),    # past it, one launch
    (Q40, 8192, 64, 8),       # 256 blocks: four slots per lane
    (Q41, 8192, 24, 7),
    (Q40, 4096, 40, 13),
    (Q40, 1024, 8192, 5),     # 1024 row slices
    (Q41, 2048, 6000, 16),
]


@pytest.mark.parametrize("type_,K,M,N", CASES)
def test_linear_bit_exact_vs_oracle(type_, K, M, N):
    """Vector kernel (every batch here is below the MFMA size threshold)."""
    w = _weights(type_, K, M, seed=K + M + N)
    x, xq = _columns(K, N, seed=K * 3 + N)
    L = moe_ffn.MoeLinear(type_, K, M, w)
    y = host(L.forward_q8(dev(q8_bytes(xq).reshape(N, -1)), N))
    assert np.array_equal(bits(y), bits(_oracle(type_, w, K, M, xq))), (type_, K, M, N)
    L.close()


MFMA_CASES = [
    # K, M, N: every fold form of the MFMA kernel
    (2048, 264, 32),      # 64 blocks (grouped leaves), the narrowest MFMA batch
    (2048, 512, 128),     # one full column group
    (1024, 256, 300),     # 32 blocks (staged leaves), partial column tile
    (32, 1, 40),          # one block, one row (31 padding rows)
    (2560, 640, 40),      # 80 blocks (lanes holding several blocks)
    (2080, 1000, 33),     # 65 blocks, rows not a multiple of 32
    (3072, 256, 64),      # 96 blocks, the last row length of the chained-second-block leaves
    (4096, 96, 32),       # 128 blocks, every block chained through per-block loads
]


def _linear_envs(env, *args, **kw):
    """A linear handle created with the environment variables in `env` set
    (the handle reads them at creation)."""
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return moe_ffn.MoeLinear(*args, **kw)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


def _linear_env(mode, *args, **kw):
    """A linear handle created with MOE_LINEAR_MFMA = mode."""
    return _linear_envs({"MOE_LINEAR_MFMA": mode}, *args, **kw)


G_CASES = [
    # type, K, M, N: the vector kernel with 1, 2 and 4 columns per pass and
    # 4 or 8 rows per wave
    (Q40, 2560, 640, 8),      # 80 blocks, 80 row slices
    (Q40, 8192, 64, 5),       # four slots per lane, a partial last pass
    (Q40, 2080, 1000, 3),     # 65 blocks, rows not a multiple of 8
    (Q41, 640, 2560, 6),      # the reference model's Q4_1 down
    (Q41, 2560, 200, 9),
    (Q41, 8192, 24, 7),       # four slots per lane
]


@pytest.mark.parametrize("rows", [4, 8])
@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("type_,K,M,N", G_CASES)
def test_linear_columns_per_pass_bit_exact(rows, G, type_, K, M, N):
    """Every column count per pass over the held weights (MOE_LINEAR_G) and
    row count per wave (MOE_LINEAR_ROWS; both read at creation, by default
    chosen from the launch's wave count) gives the oracle's bits: each
    column's chain is the same whatever its pass, and each row's fold the
    same whatever rows share its wave."""
    w = _weights(type_, K, M, seed=K + 5 * M + N)
    _, xq = _columns(K, N, seed=K * 7 + N)
    L = _linear_envs({"MOE_LINEAR_G": G, "MOE_LINEAR_ROWS": rows}, type_, K, M, w)
    y = host(L.forward_q8(dev(q8_bytes(xq).reshape(N, -1)), N))
    assert np.array_equal(bits(y), bits(_oracle(type_, w, K, M, xq))), (rows, G, type_, K, M, N)
    L.close()


@pytest.mark.parametrize("K,M,N", MFMA_CASES)
def test_linear_mfma_bit_exact_vs_oracle(K, M, N):
    """Q4_0 batches of 32 columns or more within the workspace, forced onto
    int8 MFMA (by default only large ones go there): the same bits as the
    oracle (and so as the vector kernel), from canonical Q8 input
    (forward_q8) and from fp32 input (apply, quantized straight into planes)."""
    w = q4_matrix(K + 2 * M + N, K, M)
    x, xq = _columns(K, N, seed=K * 5 + N)
    ref = O.matrix_gpu_order(w, K, M, xq)
    L = _linear_env(1, Q40, K, M, w, max_columns=N)
    y = host(L.forward_q8(dev(q8_bytes(xq).reshape(N, -1)), N))
    assert np.array_equal(bits(y), bits(ref)), ("forward_q8", K, M, N)
    ya, err = L.apply(dev(x))
    assert np.array_equal(bits(host(ya)), bits(ref)), ("apply", K, M, N)
    assert int(host(err)[0]) == 0
    L.close()


@pytest.mark.parametrize("K,M,N", [(2048, 264, 200), (1024, 256, 77), (2560, 640, 64), (4096, 96, 40)])
def test_linear_mfma_forward_q8_past_the_workspace(K, M, N):
    """forward_q8's MFMA kernel reads the canonical Q8_1 blocks in place, so a
    handle with a small workspace (max_columns 8) still takes wide batches
    onto MFMA: the same bits as the oracle, for each fold form."""
    w = q4_matrix(K + 3 * M + N, K, M)
    _, xq = _columns(K, N, seed=K * 3 + N)
    L = _linear_env(1, Q40, K, M, w, max_columns=8)
    y = host(L.forward_q8(dev(q8_bytes(xq).reshape(N, -1)), N))
    assert np.array_equal(bits(y), bits(O.matrix_gpu_order(w, K, M, xq))), (K, M, N)
    L.close()


def test_linear_apply_device_weights_and_flags():
    """apply(x) quantizes with the reference quantizer's bytes and then gives
    forward_q8's bits; a handle built from device-resident weights gives the
    same bits; a nonfinite input sets bit 1 and zeroes its block's codes as
    the quantizer does."""
    K, M, N = 2560, 384, 12
    w = q4_matrix(77, K, M)
    x, xq = _columns(K, N, seed=78)
    A = moe_ffn.MoeLinear(Q40, K, M, w, max_columns=16)
    y, err = A.apply(dev(x))
    ref = O.matrix_gpu_order(w, K, M, xq)
    assert np.array_equal(bits(host(y)), bits(ref))
    assert int(host(err)[0]) == 0
    B = moe_ffn.MoeLinear(Q40, K, M, dev(w))
    assert np.array_equal(bits(host(B.forward_q8(dev(q8_bytes(xq).reshape(N, -1)), N))), bits(ref))
    assert A.weight_bytes() == w.size
    xb = x.copy()
    xb[3, 100] = np.nan
    yb, errb = A.apply(dev(xb))
    assert int(host(errb)[0]) & 1
    qb = O.quantize_q8(np.where(np.isfinite(xb), xb, 0).astype(np.float32))
    qb_bytes = q8_bytes(qb).reshape(N, K // 32, 36).copy()
    qb_bytes[3, 100 // 32] = 0   # a poisoned block is written as all zero
    assert np.array_equal(bits(host(yb)), bits(O.matrix_gpu_order(w, K, M, qb_bytes.reshape(-1))))
    with pytest.raises(moe_ffn.MoeError):
        A.apply(dev(np.zeros((17, K), np.float32)))   # more columns than the workspace
    A.close()
    B.close()


def test_linear_rejects_bad_shapes():
    w = q4_matrix(5, 64, 8)
    for args in ((Q40, 48, 8), (Q40, 64, 0), (7, 64, 8), (Q40, 64, 16385)):
        with pytest.raises(moe_ffn.MoeError):
            moe_ffn.MoeLinear(args[0], args[1], args[2], w)


@pytest.mark.parametrize("type_,K,M", [(Q40, 2048, 256), (Q41, 640, 64)])
def test_linear_maximum_columns(type_, K, M):
    """65536 columns in one call, the entry point's limit: Q4_0 on the MFMA
    kernel (canonical blocks read in place, 151 MB of them), Q4_1 on the
    vector kernel.  256 distinct columns repeat across the batch; sampled
    columns at both ends and inside are bit-identical to the oracle, and
    65537 columns are rejected before any launch."""
    N, base = 65536, 256
    w = _weights(type_, K, M, seed=K + M)
    _, xq = _columns(K, base, seed=K + 11)
    xb = q8_bytes(xq).reshape(base, -1)
    ref = _oracle(type_, w, K, M, xq).reshape(base, M)
    L = moe_ffn.MoeLinear(type_, K, M, w)
    x = dev(np.tile(xb, (N // base, 1)))
    y = host(L.forward_q8(x, N))
    for c in (0, 1, 255, 256, 31 * 1024 + 7, 40000, N - 2, N - 1):
        assert np.array_equal(bits(y[c]), bits(ref[c % base])), (type_, c)
    with pytest.raises((moe_ffn.MoeError, ValueError)):
        L.forward_q8(dev(np.tile(xb, (N // base + 1, 1))[: N + 1]), N + 1)
    L.close()
