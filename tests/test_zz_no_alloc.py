"""moe_linear_apply_noalloc (the no-allocation variant of moe_linear_apply,
whose Q8_1 staging is a static device array of the library) against
moe_linear_apply on the same handle: outputs and error flags bit-identical,
on two calls in a row with the second smaller, on the vector kernel and on
the MFMA kernel; sizes past the 4 MiB array are rejected before any launch;
the calls leave the device's free memory unchanged.

Every call here is issued on torch's current stream, one after another: the
static array is shared by all calls on a GPU, so calls on two streams that
are not ordered against each other would race on it (the entry point only
refuses a second host thread entering while one is inside it)."""
import numpy as np
import pytest

import moe_ffn
import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def _run_pair(lin, n, seed):
    assert torch.cuda.current_stream() == torch.cuda.default_stream(), "calls share one stream"
    x = torch.from_numpy(W.activations(n, hidden=lin.K, seed=seed)).to(DEV)
    y_ref, e_ref = lin.apply(x)
    y = torch.full((n, lin.M), float("nan"), dtype=torch.float32, device=DEV)
    e = torch.zeros(1, dtype=torch.int32, device=DEV)
    lin.apply_noalloc(x, y, e)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), f"{lin.K}x{lin.M} N={n}"
    assert int(e.cpu()[0]) == int(e_ref.cpu()[0])
    return y


@pytest.mark.parametrize("K,M,first,second,qtype", [
    (2048, 2048, 256, 100, moe_ffn.TYPE_Q4_0),   # MFMA kernel, then MFMA again on fewer columns
    (2048, 2048, 96, 8, moe_ffn.TYPE_Q4_0),      # MFMA, then the vector kernel
    (2560, 640, 33, 3, moe_ffn.TYPE_Q4_0),       # vector kernel (rows of 80 blocks)
    (640, 2560, 128, 1, moe_ffn.TYPE_Q4_1),      # Q4_1 (vector kernel only)
])
def test_noalloc_matches_apply_two_calls(K, M, first, second, qtype):
    rng = np.random.default_rng(K * 3 + M + first)
    blocks = W.q4_1_blocks(M * K // 32, rng) if qtype == moe_ffn.TYPE_Q4_1 else W.q4_blocks(M * K // 32, rng)
    lin = moe_ffn.MoeLinear(qtype, K, M, blocks.reshape(-1), max_columns=first)
    _run_pair(lin, first, seed=1)
    _run_pair(lin, second, seed=2)
    lin.close()


def test_noalloc_without_workspace_and_limits():
    """A handle created with max_columns = 0 (no workspace) still applies;
    the staging limit is enforced before any launch; nothing is allocated."""
    rng = np.random.default_rng(7)
    blocks = W.q4_blocks(2048 * 64, rng).reshape(-1)
    lin0 = moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, 2048, 2048, blocks, max_columns=0)
    ref = moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, 2048, 2048, blocks, max_columns=512)
    n = 512
    x = torch.from_numpy(W.activations(n, seed=8)).to(DEV)
    y = torch.empty((n, 2048), dtype=torch.float32, device=DEV)
    e = torch.zeros(1, dtype=torch.int32, device=DEV)
    y_ref, _ = ref.apply(x)
    lin0.apply_noalloc(x, y, e)   # warm-up: first launches load code
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(20):
        lin0.apply_noalloc(x, y, e)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)) and int(e.cpu()[0]) == 0
    # 1821 columns of 64 blocks need 1821 * 64 * 36 B > 4 MiB.
    big = torch.zeros((1821, 2048), dtype=torch.float32, device=DEV)
    yb = torch.empty((1821, 2048), dtype=torch.float32, device=DEV)
    with pytest.raises(moe_ffn.MoeError) as ex:
        lin0.apply_noalloc(big, yb, e)
    assert ex.value.status == 1
    ok = torch.zeros((1820, 2048), dtype=torch.float32, device=DEV)
    lin0.apply_noalloc(ok, yb[:1820], e)
    torch.cuda.synchronize()
    assert int(e.cpu()[0]) == 0 and bool((yb[:1820] == 0).all())
    lin0.close()
    ref.close()
