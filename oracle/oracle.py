"""ctypes binding to the CPU oracle (oracle/libmoe_oracle.so) and to the
compiled reference CPU path (oracle/_ref/libref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the CPU baseline.  The product
library never imports this module.

Formats (reference src/quant.hpp:8-18): Q4_0 = 18-byte blocks (half d, 16 code
bytes), Q8_1 = 36-byte blocks (half d, half raw sum s, 32 int8 codes).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libmoe_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

Q8_DTYPE = np.dtype([("d", "<u2"), ("s", "<u2"), ("qs", "i1", (32,))])
assert Q8_DTYPE.itemsize == 36
Q4_BLOCK = 18

_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t


def _ptr(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def as_q8(a):
    """View raw canonical Q8_1 bytes (uint8, 36 per block) as Q8_DTYPE records."""
    a = np.ascontiguousarray(a)
    if a.dtype == Q8_DTYPE:
        return a
    assert a.dtype == np.uint8 and a.size % 36 == 0
    return a.reshape(-1).view(Q8_DTYPE)


def _load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run make -C oracle)")
    lib = ctypes.CDLL(ORACLE_SO)
    lib.mo_half_to_float.restype = ctypes.c_float
    lib.mo_half_to_float.argtypes = [ctypes.c_uint16]
    lib.mo_float_to_half.restype = ctypes.c_uint16
    lib.mo_float_to_half.argtypes = [ctypes.c_float]
    lib.mo_quantize_q8.argtypes = [_P, _SZ, _P]
    lib.mo_expf_libm.restype = None
    lib.mo_expf_libm.argtypes = [_P, _P, _SZ]
    lib.mo_router_softmax.argtypes = [_P, _I, _I, _P]
    lib.mo_matrix_gpu_order_q41.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.mo_expert_forward_q41.argtypes = [_P, _P, _P, _I, _I, _P, _I, _P, _P, _P, _P, _P]
    lib.mo_moe_layer_q41.argtypes = [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P]
    lib.mo_select_routes.argtypes = [_P, _I, _I, _I, _P, _P]
    lib.mo_block_dot.argtypes = [_P, _P]
    lib.mo_scaled_dot_q4_0.restype = ctypes.c_float
    lib.mo_scaled_dot_q4_0.argtypes = [ctypes.c_int32, ctypes.c_uint16, _P]
    lib.mo_block_dots.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.mo_matmul_full.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.mo_matrix_gpu_order.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.mo_matrix_gpu_order_avx2.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.mo_expert_forward.argtypes = [_P, _P, _P, _I, _I, _P, _I, _P, _P, _P, _P, _P, _I]
    lib.mo_route_groups.argtypes = [_P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P]
    lib.mo_routed_fold.argtypes = [_P, _P, _I, _I, _I, _P]
    lib.mo_combine_flags.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P]
    lib.mo_moe_layer.argtypes = [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I]
    lib.mo_baseline_layer.argtypes = [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                      ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]
    lib.mo_allowed_physical_cpus.argtypes = [_P, _I, ctypes.POINTER(_I)]
    return lib


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load_oracle()
    return _lib


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    """The compiled reference CPU path (only in the container that has it)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError("oracle/_ref/libref.so is not built")
        r = ctypes.CDLL(REF_SO)
        r.ref_half_to_float.restype = ctypes.c_float
        r.ref_half_to_float.argtypes = [ctypes.c_uint16]
        r.ref_float_to_half.restype = ctypes.c_uint16
        r.ref_float_to_half.argtypes = [ctypes.c_float]
        r.ref_quantize_q8.argtypes = [_P, _SZ, _P]
        r.ref_dot_q4_0.restype = ctypes.c_float
        r.ref_dot_q4_0.argtypes = [_P, _P]
        r.ref_matmul.argtypes = [_I, _P, _I, _I, _P, _I, _P]
        r.ref_cpu_expert.argtypes = [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P]
        r.ref_route_groups.argtypes = [_P, _P, _I, _P, _P, _P, _P, _P]
        r.ref_cpu_expert_q41.argtypes = [_P, _P, _P, _P, _I, _P, _P, _P]
        _ref = r
    return _ref


# ----------------------------------------------------------------- helpers ---
class OracleError(RuntimeError):
    pass


def _check(rc, what):
    if rc != 0:
        raise OracleError(f"{what}: oracle status {rc}")


def quantize_q8(x):
    """fp32 [..., K] -> Q8_1 [..., K/32] (src/quant.cpp:275-325)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape[-1] % 32 == 0
    out = np.zeros(x.shape[:-1] + (x.shape[-1] // 32,), dtype=Q8_DTYPE)
    _check(lib().mo_quantize_q8(_ptr(x), x.size, _ptr(out)), "quantize_q8")
    return out


def expf_libm(x):
    """The C library's expf, elementwise (float32 in, float32 out)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().mo_expf_libm(_ptr(x), _ptr(y), x.size)
    return y


def router_softmax(logits):
    """Row softmax in the reference's GPU order (C library expf); returns
    (probabilities float32 [N][E], flags)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    n, e = logits.shape
    prob = np.empty_like(logits)
    flags = lib().mo_router_softmax(_ptr(logits), n, e, _ptr(prob))
    return prob, flags


def select_routes(prob, top_k=10):
    """Top-k ids (ties to the lower id) and XOR-bucket normalised weights;
    returns (ids int32 [N][k], weights float32 [N][k], flags)."""
    prob = np.ascontiguousarray(prob, dtype=np.float32)
    n, e = prob.shape
    ids = np.empty((n, top_k), np.int32)
    w = np.empty((n, top_k), np.float32)
    flags = lib().mo_select_routes(_ptr(prob), n, e, top_k, _ptr(ids), _ptr(w))
    return ids, w, flags


def block_dots(w, K, M, xq):
    """int32 per-block dots [cols][M][K/32] (src/quant.cpp:48-55)."""
    xq = as_q8(xq).reshape(-1, K // 32)
    cols = xq.shape[0]
    out = np.zeros((cols, M, K // 32), dtype=np.int32)
    lib().mo_block_dots(_ptr(np.ascontiguousarray(w)), K, M, _ptr(xq), cols, _ptr(out))
    return out


def matmul_full(w, K, M, xq):
    xq = as_q8(xq).reshape(-1, K // 32)
    out = np.zeros((xq.shape[0], M), dtype=np.float32)
    lib().mo_matmul_full(_ptr(np.ascontiguousarray(w)), K, M, _ptr(xq), xq.shape[0], _ptr(out))
    return out


def matrix_gpu_order(w, K, M, xq, avx2=False):
    xq = as_q8(xq).reshape(-1, K // 32)
    out = np.zeros((xq.shape[0], M), dtype=np.float32)
    f = lib().mo_matrix_gpu_order_avx2 if avx2 else lib().mo_matrix_gpu_order
    rc = f(_ptr(np.ascontiguousarray(w)), K, M, _ptr(xq), xq.shape[0], _ptr(out))
    if avx2:
        _check(rc, "matrix_gpu_order_avx2")
    return out


def matrix_gpu_order_q41(w, K, M, xq):
    """Q4_1 matrix x Q8_1 columns in the reference cpu_expert order
    (src/cpu_expert.cpp:167-194)."""
    xq = as_q8(xq).reshape(-1, K // 32)
    out = np.zeros((xq.shape[0], M), dtype=np.float32)
    lib().mo_matrix_gpu_order_q41(_ptr(np.ascontiguousarray(w)), K, M, _ptr(xq), xq.shape[0], _ptr(out))
    return out


def expert_forward(gate, up, down, H, I, xq, avx2=False, down_q41=False):
    """cpu_expert whole stage (down Q4_0, or Q4_1 with down_q41).  Returns
    dict(y, gate, up, middle, middle_q8)."""
    xq = as_q8(xq).reshape(-1, H // 32)
    cols = xq.shape[0]
    y = np.zeros((cols, H), np.float32)
    g = np.zeros((cols, I), np.float32)
    u = np.zeros((cols, I), np.float32)
    m = np.zeros((cols, I), np.float32)
    mq = np.zeros((cols, I // 32), Q8_DTYPE)
    args = (_ptr(np.ascontiguousarray(gate)), _ptr(np.ascontiguousarray(up)), _ptr(np.ascontiguousarray(down)),
            H, I, _ptr(xq), cols, _ptr(y), _ptr(g), _ptr(u), _ptr(m), _ptr(mq))
    if down_q41:
        rc = lib().mo_expert_forward_q41(*args)
    else:
        rc = lib().mo_expert_forward(*args, 1 if avx2 else 0)
    _check(rc, "expert_forward")
    return dict(y=y, gate=g, up=u, middle=m, middle_q8=mq)


def route_groups(ids, weights, experts):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    tokens, k = ids.shape
    n = tokens * k
    at, ar, ae = (np.zeros(n, np.int32) for _ in range(3))
    aw = np.zeros(n, np.float32)
    counts = np.zeros(experts, np.int32)
    offsets = np.zeros(experts + 1, np.int32)
    rc = lib().mo_route_groups(_ptr(ids), _ptr(weights), tokens, k, experts, _ptr(at), _ptr(ar),
                               _ptr(ae), _ptr(aw), _ptr(counts), _ptr(offsets))
    _check(rc, "route_groups")
    return dict(token=at, rank=ar, expert=ae, weight=aw, counts=counts, offsets=offsets)


def routed_fold(contrib, weights):
    contrib = np.ascontiguousarray(contrib, dtype=np.float32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    tokens, k, H = contrib.shape
    y = np.zeros((tokens, H), np.float32)
    lib().mo_routed_fold(_ptr(contrib), _ptr(weights), tokens, k, H, _ptr(y))
    return y


def combine_flags(contrib, weights, shared=None, shared_gate=None):
    """routed_fold then shared_sigmoid_add with the reference's flag semantics
    (session_ops.hip:307-324, 375-391).  Returns (y, flags)."""
    contrib = np.ascontiguousarray(contrib, dtype=np.float32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    tokens, k, H = contrib.shape
    sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
    g = None if shared_gate is None else np.ascontiguousarray(shared_gate, dtype=np.float32)
    y = np.zeros((tokens, H), np.float32)
    flags = lib().mo_combine_flags(_ptr(contrib), _ptr(weights), _ptr(sh), _ptr(g), tokens, k, H, _ptr(y))
    return y, int(flags)


def moe_layer(x, H, I, E, experts_q4, ids, weights, shared_q4=None, shared_gate=None,
              token_mask=None, avx2=True, want_contrib=False, down_q41=False):
    """Whole MoE layer in the reference order (down Q4_1 with down_q41).
    Returns dict(y, x_q8[, contrib])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    tokens = x.shape[0]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    k = ids.shape[1]
    y = np.zeros((tokens, H), np.float32)
    xq = np.zeros((tokens, H // 32), Q8_DTYPE)
    contrib = np.zeros((tokens, k, H), np.float32) if want_contrib else None
    sg = None if shared_gate is None else np.ascontiguousarray(shared_gate, dtype=np.float32)
    mask = None if token_mask is None else np.ascontiguousarray(token_mask, dtype=np.uint8)
    args = (_ptr(x), tokens, H, I, E, k, _ptr(experts_q4), _ptr(shared_q4) if shared_q4 is not None else None,
            _ptr(ids), _ptr(weights), _ptr(sg), _ptr(y), _ptr(contrib), _ptr(xq), _ptr(mask))
    if down_q41:
        rc = lib().mo_moe_layer_q41(*args)
    else:
        rc = lib().mo_moe_layer(*args, 1 if avx2 else 0)
    _check(rc, "moe_layer")
    out = dict(y=y, x_q8=xq)
    if want_contrib:
        out["contrib"] = contrib
    return out


def baseline_layer(x, H, I, E, experts_q4, ids, weights, shared_q4=None, shared_gate=None,
                   workers=0, pin=True, repeats=3):
    """Time the pinned-pool CPU layer.  Returns (seconds_per_layer, workers, y)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    tokens = x.shape[0]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    y = np.zeros((tokens, H), np.float32)
    sec = ctypes.c_double(0)
    used = ctypes.c_int(0)
    sg = None if shared_gate is None else np.ascontiguousarray(shared_gate, dtype=np.float32)
    rc = lib().mo_baseline_layer(_ptr(x), tokens, H, I, E, ids.shape[1], _ptr(experts_q4),
                                 _ptr(shared_q4) if shared_q4 is not None else None, _ptr(ids),
                                 _ptr(weights), _ptr(sg), _ptr(y), int(workers), 1 if pin else 0,
                                 int(repeats), ctypes.byref(sec), ctypes.byref(used))
    _check(rc, "baseline_layer")
    return sec.value, used.value, y


def physical_cpus():
    buf = np.zeros(4096, np.int32)
    n = ctypes.c_int(0)
    lib().mo_allowed_physical_cpus(_ptr(buf), 4096, ctypes.byref(n))
    return buf[: n.value].tolist()


# --------------------------------------------------- reference wrappers ---
def ref_quantize_q8(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape[:-1] + (x.shape[-1] // 32,), dtype=Q8_DTYPE)
    rc = ref().ref_quantize_q8(_ptr(x), x.size, _ptr(out))
    return rc, out


def ref_matmul(variant, w, K, M, xq):
    xq = as_q8(xq).reshape(-1, K // 32)
    out = np.zeros((xq.shape[0], M), np.float32)
    rc = ref().ref_matmul(variant, _ptr(np.ascontiguousarray(w)), K, M, _ptr(xq), xq.shape[0], _ptr(out))
    if rc:
        raise OracleError(f"reference matmul status {rc}")
    return out


def ref_cpu_expert(gate, up, down, xq):
    xq = as_q8(xq).reshape(-1, 80)
    cols = xq.shape[0]
    y = np.zeros((cols, 2560), np.float32)
    g = np.zeros((cols, 640), np.float32)
    u = np.zeros((cols, 640), np.float32)
    m = np.zeros((cols, 640), np.float32)
    mq = np.zeros((cols, 20), Q8_DTYPE)
    st = ref().ref_cpu_expert(_ptr(gate), _ptr(up), _ptr(down), _ptr(xq), cols, _ptr(y), _ptr(g),
                              _ptr(u), _ptr(m), _ptr(mq))
    return st, dict(y=y, gate=g, up=u, middle=m, middle_q8=mq)


def ref_cpu_expert_q41(gate, up, down, xq):
    """The reference's CPU expert with a Q4_1 down matrix (2560/640)."""
    xq = as_q8(xq).reshape(-1, 80)
    cols = xq.shape[0]
    y = np.zeros((cols, 2560), np.float32)
    m = np.zeros((cols, 640), np.float32)
    mq = np.zeros((cols, 20), Q8_DTYPE)
    st = ref().ref_cpu_expert_q41(_ptr(gate), _ptr(up), _ptr(down), _ptr(xq), cols, _ptr(y), _ptr(m), _ptr(mq))
    return st, dict(y=y, middle=m, middle_q8=mq)


def ref_route_groups(ids, weights):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    n = ids.size
    at, ar, ae = (np.zeros(n, np.int32) for _ in range(3))
    aw = np.zeros(n, np.float32)
    counts = np.zeros(512, np.int32)
    rc = ref().ref_route_groups(_ptr(ids), _ptr(weights), ids.shape[0], _ptr(at), _ptr(ar), _ptr(ae),
                                _ptr(aw), _ptr(counts))
    return rc, dict(token=at, rank=ar, expert=ae, weight=aw, counts=counts)
