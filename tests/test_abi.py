"""The C-ABI library loads on a machine without a GPU, exports every entry
point include/moe_ffn.h declares, and rejects bad arguments before any HIP
call (src/hip/linear.cuh:40-43 convention).  No compute calls here."""
import ctypes
import subprocess

import moe_ffn


def test_library_exports_every_declared_symbol():
    lib = moe_ffn.library()
    declared = moe_ffn.header_symbols()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", moe_ffn.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared) <= exported


def test_invalid_arguments_rejected_before_hip():
    lib = moe_ffn.library()
    # null / misaligned / bad shapes -> hipErrorInvalidValue (1)
    assert lib.moe_quantize_q8_1(None, None, 64, 1, None, None) == 1
    buf = (ctypes.c_float * 64)()
    assert lib.moe_quantize_q8_1(buf, buf, 33, 1, buf, None) == 1
    assert lib.moe_quantize_q8_1(buf, buf, 64, 0, buf, None) == 1
    assert lib.moe_ffn_forward(None, None, None, None, 1, None, None, None, None) == 1
    assert lib.moe_combine(None, None, None, None, 1, 1, 1, None, None, None) == 1
    ok = moe_ffn.Config(2048, 512, 512, 10, 1, 8)
    h = ctypes.c_void_p()
    assert lib.moe_ffn_create_tensors(ctypes.byref(ok), buf, None, buf, buf, buf, buf, 0, ctypes.byref(h)) == 1
    assert lib.moe_ffn_create_tensors(ctypes.byref(ok), buf, buf, buf, None, buf, buf, 0, ctypes.byref(h)) == 1
    assert lib.moe_ffn_create(ctypes.byref(ok), None, buf, 0, ctypes.byref(h)) == 1
    bad = moe_ffn.Config(2048, 500, 512, 10, 1, 8)      # intermediate not a multiple of 32
    w, s = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.moe_ffn_memory_bytes(ctypes.byref(bad), ctypes.byref(w), ctypes.byref(s)) == 1
    bad_down = moe_ffn.Config(2048, 512, 512, 10, 1, 8, 2)   # no such down block type
    assert lib.moe_ffn_memory_bytes(ctypes.byref(bad_down), ctypes.byref(w), ctypes.byref(s)) == 1
    q41 = moe_ffn.Config(2048, 512, 512, 10, 1, 8, moe_ffn.DOWN_Q4_1)
    assert lib.moe_ffn_memory_bytes(ctypes.byref(q41), ctypes.byref(w), ctypes.byref(s)) == 0
    assert w.value >= 513 * moe_ffn.expert_bytes(2048, 512, moe_ffn.DOWN_Q4_1)
    assert lib.moe_ffn_forward_q8(None, None, None, None, 1, None, None, None, None) == 1
    assert lib.moe_router_select(None, 8, 512, 10, None, None, None, None, None) == 1
    # quantized linear: type, shape and pointer checks come first
    lin = ctypes.c_void_p()
    for args in ((7, 64, 8, 0), (moe_ffn.TYPE_Q4_0, 48, 8, 0), (moe_ffn.TYPE_Q4_0, 64, 0, 0),
                 (moe_ffn.TYPE_Q4_1, 64, 16385, 0), (moe_ffn.TYPE_Q4_0, 64, 8, -1)):
        assert lib.moe_linear_create(*args, buf, 0, 0, ctypes.byref(lin)) == 1, args
    assert lib.moe_linear_create(moe_ffn.TYPE_Q4_0, 64, 8, 0, None, 0, 0, ctypes.byref(lin)) == 1
    assert lib.moe_linear_forward_q8(None, buf, 1, buf, None) == 1
    assert lib.moe_linear_apply(None, buf, 1, buf, buf, None) == 1
    assert lib.moe_linear_destroy(None) == 1


def test_memory_footprint_baseline_shape():
    w, s = moe_ffn.memory_bytes(2048, 512, 512, 10, True, 16384)
    # 513 experts x 3 x 1,048,576 weights x 18/32 bytes, plus alignment padding.
    assert 513 * 1769472 <= w < 513 * 1769472 + 4096
    assert s > 16384 * 11 * 2048 * 4       # contributions dominate the workspace


def _expf_sample():
    """Every 509th float32 bit pattern (8.4M values over all signs and
    exponents) plus every 997th float in [-20, 20] (the arguments SiLU sees
    in practice)."""
    import numpy as np
    bits = np.arange(0, 1 << 32, 509, dtype=np.uint64).astype(np.uint32)
    pos = np.arange(0, np.float32(20).view(np.uint32), 997, dtype=np.uint32)
    return np.concatenate([bits, pos, pos | np.uint32(0x80000000)]).view(np.float32)


def test_expf_host_build_matches_libm():
    """The kernels' expf (moe_expf.h, run here on the CPU) equals the C
    library's expf bit for bit (NaN payloads aside).  An exhaustive run over
    all 2^32 inputs had 0 mismatches; this is a dense sample of it."""
    import numpy as np
    import oracle as O
    x = _expf_sample()
    got = moe_ffn.expf_host(x)
    ref = O.expf_libm(x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_binding_rejects_mismatched_tensors():
    """The Python binding checks dtype, exact shape, contiguity and device of
    every tensor before it hands raw pointers to the C ABI (a short or int64
    ids tensor would otherwise be read past its end on the GPU)."""
    import pytest
    torch = pytest.importorskip("torch")
    ids = torch.zeros((4, 10), dtype=torch.int32)
    w = torch.zeros((4, 10), dtype=torch.float32)
    with pytest.raises(TypeError):
        moe_ffn._routes_check(ids.to(torch.int64), w, 4, 10, None)
    with pytest.raises(ValueError):
        moe_ffn._routes_check(ids[:3], w, 4, 10, None)
    with pytest.raises(ValueError):
        moe_ffn._routes_check(torch.zeros((10, 4), dtype=torch.int32).t(), w, 4, 10, None)
    with pytest.raises(ValueError):   # CPU tensors never reach the library
        moe_ffn._routes_check(ids, w, 4, 10, None)
    with pytest.raises(TypeError):
        moe_ffn._need(w.to(torch.float64), "w", torch.float32, (4, 10))
