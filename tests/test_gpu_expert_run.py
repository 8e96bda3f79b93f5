"""moe_ffn_expert_run, the counterpart of GpuExpert::run (src/hip/expert.hip:
228-241): one resident expert's whole fp32 forward from host memory, timed.
Run at the reference harness's own expert shape and inputs (hidden 2560,
intermediate 640, Q4_0 gate/up and Q4_1 down; columns 1, 2, 3, 128; x_i =
0.7 sin(0.137 i) + 0.2 cos(0.071 i), src/expert_main.cpp:88-90), with
synthetic weights in place of the checkpoint's layer-0 expert.

Bars: the streaming kernels follow the reference's order, so their outputs
are bit-identical to the oracle's cpu_expert (quantize -> gate/up -> SiLU*up
-> quantize -> Q4_1 down); the int8-MFMA down sums blocks in its own order
and is held to 1e-5 rms (the reference harness's own gate is 2e-3 abs /
2e-4 rel, src/expert_main.cpp:137).  A nonfinite input raises the error word
and does not poison the next call (src/expert_main.cpp:119-126)."""
import numpy as np
import pytest

import moe_ffn
import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
H, I = 2560, 640


def harness_input(columns):
    i = np.arange(H * columns, dtype=np.float32)
    x = np.float32(0.7) * np.sin(i * np.float32(0.137)) + np.float32(0.2) * np.cos(i * np.float32(0.071))
    return x.astype(np.float32).reshape(columns, H)


def rms(a):
    return float(np.sqrt(np.mean(np.square(np.asarray(a, np.float64)))))


@pytest.fixture(scope="module")
def expert():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    bank = W.q4_bank(1, hidden=H, intermediate=I, seed=4100, down_type=moe_ffn.DOWN_Q4_1)
    gb = H // 32 * I * 18
    per = np.asarray(bank).reshape(-1)
    g, u, d = per[:gb], per[gb:2 * gb], per[2 * gb:]
    layer = moe_ffn.MoeLayer(H, I, 1, 1, False, 128, experts_q4=bank, down_type=moe_ffn.DOWN_Q4_1)
    yield dict(layer=layer, g=g, u=u, d=d)
    layer.close()


@pytest.mark.parametrize("columns", [1, 2, 3, 128])
def test_expert_run_matches_oracle(expert, columns):
    L = expert["layer"]
    x = harness_input(columns)
    print(f"\n[expert_run] H={H} I={I} columns={columns}", flush=True)
    ref = O.expert_forward(expert["g"], expert["u"], expert["d"], H, I, O.quantize_q8(x), down_q41=True)["y"]
    for path in (moe_ffn.PATH_AUTO, moe_ffn.PATH_STREAM):   # AUTO streams below 1024 routes
        y, t, flags = L.expert_run(0, x, repeats=5, path=path)
        assert flags == 0
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), path
        assert t["upload_ms"] > 0 and t["resident_ms"] > 0
        assert t["completed_wall_ms"] >= 0.5 * t["resident_ms"]
    y, t, flags = L.expert_run(0, x, repeats=5, path=moe_ffn.PATH_MFMA)
    assert flags == 0
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    assert err <= 1e-5 * rms(ref), f"MFMA expert: max abs err {err:.3e} > 1e-5 * rms {rms(ref):.3e}"


def test_expert_run_rejects_nonfinite_input_then_recovers(expert):
    L = expert["layer"]
    for value in (np.inf, np.nan):
        bad = np.full((1, H), value, np.float32)
        y, t, flags = L.expert_run(0, bad, repeats=1)
        assert flags & 1 and y is None and t is None, value
    x = harness_input(1)
    y, t, flags = L.expert_run(0, x, repeats=1)
    ref = O.expert_forward(expert["g"], expert["u"], expert["d"], H, I, O.quantize_q8(x), down_q41=True)["y"]
    assert flags == 0 and np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_expert_run_argument_checks(expert):
    L = expert["layer"]
    lib = moe_ffn.library()
    x = harness_input(1)
    flags = moe_ffn._I(0)
    t = moe_ffn.ExpertTiming()
    p = moe_ffn.ctypes.c_void_p(x.ctypes.data)
    for args in ((1, p, 1, p, 1, 0), (0, p, 0, p, 1, 0), (0, p, 129, p, 1, 0), (0, p, 1, p, 0, 0),
                 (0, p, 1, p, 10001, 0), (0, p, 1, p, 1, 3), (0, None, 1, p, 1, 0)):
        st = lib.moe_ffn_expert_run(L.handle, *args, moe_ffn.ctypes.byref(flags), moe_ffn.ctypes.byref(t), None)
        assert st == 1, args
