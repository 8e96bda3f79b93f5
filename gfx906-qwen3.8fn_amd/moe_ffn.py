"""Python binding of the MI355X routed-MoE expert FFN C ABI (include/moe_ffn.h).

This is the host-side operator surface used by the tests and bench.py.  It
mirrors the reference's expert operator (src/gpu_expert.hpp:7-17, the Experts /
Layer::ffn path of src/session.hip:976-1078, 1446-1541): token activations,
top-k expert ids and route weights go in, the routing-weighted FFN output in
token order comes out.  Every call goes through libmoe_ffn.so; there is no
CPU or PyTorch fallback -- a missing library raises.

PyTorch is only used to own device memory and streams.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoe_ffn.so")
ROOT = os.path.dirname(HERE)
HEADER = os.path.join(ROOT, "include", "moe_ffn.h")

Q8_BLOCK = 36
Q4_BLOCK = 18
Q4_1_BLOCK = 20
DOWN_Q4_0, DOWN_Q4_1 = 0, 1     # MOE_DOWN_Q4_0 / MOE_DOWN_Q4_1
PATH_AUTO, PATH_STREAM, PATH_MFMA = 0, 1, 2
TYPE_Q4_0, TYPE_Q4_1 = 2, 3     # MOE_TYPE_Q4_0 / MOE_TYPE_Q4_1 (the reference's TensorType ids)
STAGE_PREPARE, STAGE_GATE_UP, STAGE_DOWN, STAGE_FOLD = 0, 1, 2, 3


class MoeError(RuntimeError):
    def __init__(self, what, status):
        super().__init__(f"{what} failed with status {status}")
        self.status = status


class Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int), ("experts", ctypes.c_int),
                ("top_k", ctypes.c_int), ("has_shared", ctypes.c_int), ("max_tokens", ctypes.c_int),
                ("down_type", ctypes.c_int)]


class ExpertTiming(ctypes.Structure):
    """moe_expert_timing (ExpertTiming, src/gpu_expert.hpp:6)."""
    _fields_ = [("upload_ms", ctypes.c_double), ("resident_ms", ctypes.c_double),
                ("completed_wall_ms", ctypes.c_double)]


_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int


def library():
    """Load libmoe_ffn.so (built in-tree by __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP extension missing: {LIB_PATH}; run __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        lib.moe_ffn_create.argtypes = [ctypes.POINTER(Config), _P, _P, _I, ctypes.POINTER(_P)]
        lib.moe_ffn_create_from_device.argtypes = [ctypes.POINTER(Config), _P, _P, _I, ctypes.POINTER(_P)]
        lib.moe_ffn_create_tensors.argtypes = [ctypes.POINTER(Config), _P, _P, _P, _P, _P, _P, _I,
                                               ctypes.POINTER(_P)]
        lib.moe_ffn_create_synthetic.argtypes = [ctypes.POINTER(Config), ctypes.c_uint64, _I, ctypes.POINTER(_P)]
        lib.moe_ffn_destroy.argtypes = [_P]
        lib.moe_ffn_memory_bytes.argtypes = [ctypes.POINTER(Config), ctypes.POINTER(ctypes.c_size_t),
                                             ctypes.POINTER(ctypes.c_size_t)]
        lib.moe_ffn_export_expert.argtypes = [_P, _I, _P]
        lib.moe_ffn_forward.argtypes = [_P, _P, _P, _P, _I, _P, _P, _P, _P]
        lib.moe_ffn_forward_q8.argtypes = [_P, _P, _P, _P, _I, _P, _P, _P, _P]
        lib.moe_quantize_q8_1.argtypes = [_P, _P, _I, _I, _P, _P]
        lib.moe_ffn_group_routes.argtypes = [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P]
        lib.moe_ffn_expert_gate_up.argtypes = [_P, _I, _P, _I, _P, _P, _P, _P, _I, _P, _P]
        lib.moe_ffn_expert_down.argtypes = [_P, _I, _P, _I, _P, _P, _I, _P, _P]
        lib.moe_ffn_expert_run.argtypes = [_P, _I, _P, _I, _P, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(ExpertTiming),
                                           _P]
        lib.moe_combine.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P, _P]
        lib.moe_ffn_debug_last.argtypes = [_P, _P, _P, _P, _P, _P]
        lib.moe_ffn_replay_stage.argtypes = [_P, _I, _P]
        lib.moe_ffn_profile.argtypes = [_P, _I]
        lib.moe_ffn_profile_read.argtypes = [_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]
        lib.moe_expf_device.argtypes = [_P, _P, _I, _P]
        lib.moe_expf_host.argtypes = [_P, _P, ctypes.c_size_t]
        lib.moe_read_probe.argtypes = [_P, ctypes.c_size_t, _P, _P]
        lib.moe_router_select.argtypes = [_P, _I, _I, _I, _P, _P, _P, _P, _P]
        lib.moe_ffn_last_stats.argtypes = [_P, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(ctypes.c_int32)]
        lib.moe_linear_create.argtypes = [_I, _I, _I, _I, _P, _I, _I, ctypes.POINTER(_P)]
        lib.moe_linear_destroy.argtypes = [_P]
        lib.moe_linear_bytes.argtypes = [_P, ctypes.POINTER(ctypes.c_size_t)]
        lib.moe_linear_forward_q8.argtypes = [_P, _P, _I, _P, _P]
        lib.moe_linear_apply.argtypes = [_P, _P, _I, _P, _P, _P]
        lib.moe_linear_apply_noalloc.argtypes = [_P, _P, _I, _P, _P, _P]
        _lib = lib
    return _lib


def header_symbols():
    """Function names declared in include/moe_ffn.h."""
    import re
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^int\s+(moe_\w+)\s*\(", text, flags=re.M)))


def _check(status, what):
    if status != 0:
        raise MoeError(what, status)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t, name, dtype, shape, device=None):
    """Check a tensor handed to the C ABI: dtype, exact shape, contiguity and
    device.  The ABI takes raw pointers and sizes, so a tensor with fewer rows,
    another element type or a strided view would be read past its end on the
    GPU; the reference's RouteGroups::prepare likewise rejects a size
    mismatch before touching anything (src/routes.cpp:63-68)."""
    import torch
    if t is None:
        raise ValueError(f"{name} is required")
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device.type != "cuda" or (device is not None and t.device != device):
        raise ValueError(f"{name} must be on {device if device is not None else 'a GPU'}, got {t.device}")
    return t


def _routes_check(ids, weights, n, k, device):
    import torch
    _need(ids, "ids", torch.int32, (n, k), device)
    _need(weights, "weights", torch.float32, (n, k), device)


def _stream(stream):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def expert_bytes(hidden, intermediate, down_type=DOWN_Q4_0):
    """Canonical bytes of one expert: gate and up Q4_0, down Q4_0 or Q4_1."""
    return hidden // 32 * intermediate * (2 * Q4_BLOCK + (Q4_1_BLOCK if down_type == DOWN_Q4_1 else Q4_BLOCK))


class MoeLayer:
    """One MoE layer resident on the GPU (weights + workspace for max_tokens)."""

    def __init__(self, hidden, intermediate, experts, top_k, has_shared, max_tokens, experts_q4=None,
                 shared_q4=None, synthetic_seed=None, device=0, tensors=None, shared_tensors=None,
                 down_type=DOWN_Q4_0):
        self.cfg = Config(hidden, intermediate, experts, top_k, 1 if has_shared else 0, max_tokens, down_type)
        self.down_type = down_type
        self.H, self.I, self.E, self.k = hidden, intermediate, experts, top_k
        self.has_shared = bool(has_shared)
        self.max_tokens = max_tokens
        self.device = device
        handle = ctypes.c_void_p()
        lib = library()
        if tensors is not None:   # (gate_exps, up_exps, down_exps) host arrays, reference tensor layout
            ts = [np.ascontiguousarray(t, dtype=np.uint8) for t in tensors]
            nb = hidden // 32 * intermediate
            mb = [nb * Q4_BLOCK, nb * Q4_BLOCK, nb * (Q4_1_BLOCK if down_type == DOWN_Q4_1 else Q4_BLOCK)]
            assert all(t.size == experts * m for t, m in zip(ts, mb))
            ss = [None, None, None]
            if has_shared:
                ss = [np.ascontiguousarray(t, dtype=np.uint8) for t in shared_tensors]
                assert all(t.size == m for t, m in zip(ss, mb))
            ptr = lambda a: None if a is None else ctypes.c_void_p(a.ctypes.data)
            st = lib.moe_ffn_create_tensors(ctypes.byref(self.cfg), *[ptr(t) for t in ts], *[ptr(t) for t in ss],
                                            device, ctypes.byref(handle))
        elif synthetic_seed is not None:
            st = lib.moe_ffn_create_synthetic(ctypes.byref(self.cfg), ctypes.c_uint64(synthetic_seed), device,
                                              ctypes.byref(handle))
        elif isinstance(experts_q4, np.ndarray):
            experts_q4 = np.ascontiguousarray(experts_q4, dtype=np.uint8)
            assert experts_q4.size == experts * expert_bytes(hidden, intermediate, down_type)
            sh = None
            if has_shared:
                sh = np.ascontiguousarray(shared_q4, dtype=np.uint8)
                assert sh.size == expert_bytes(hidden, intermediate, down_type)
            st = lib.moe_ffn_create(ctypes.byref(self.cfg), ctypes.c_void_p(experts_q4.ctypes.data),
                                    None if sh is None else ctypes.c_void_p(sh.ctypes.data), device,
                                    ctypes.byref(handle))
        else:   # torch device tensors
            st = lib.moe_ffn_create_from_device(ctypes.byref(self.cfg), _ptr(experts_q4), _ptr(shared_q4), device,
                                                ctypes.byref(handle))
        _check(st, "moe_ffn_create")
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            library().moe_ffn_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------ queries --
    def export_expert(self, expert):
        out = np.zeros(expert_bytes(self.H, self.I, self.down_type), np.uint8)
        _check(library().moe_ffn_export_expert(self.handle, expert, ctypes.c_void_p(out.ctypes.data)),
               "moe_ffn_export_expert")
        return out

    def last_stats(self):
        a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        _check(library().moe_ffn_last_stats(self.handle, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)),
               "moe_ffn_last_stats")
        return dict(stream_items=a.value, mfma_items=b.value, active_experts=c.value)

    # ------------------------------------------------------------ forward --
    def _io_check(self, n, dev, ids, weights, shared_gate, y, error):
        import torch
        if not 1 <= n <= self.max_tokens:
            raise ValueError(f"tokens {n} outside 1..{self.max_tokens}")
        _routes_check(ids, weights, n, self.k, dev)
        if shared_gate is not None:
            _need(shared_gate, "shared_gate", torch.float32, (n,), dev)
        if y is None:
            y = torch.empty((n, self.H), dtype=torch.float32, device=dev)
        _need(y, "y", torch.float32, (n, self.H), dev)
        if error is None:
            error = torch.zeros(1, dtype=torch.int32, device=dev)
        _need(error, "error", torch.int32, (1,), dev)
        return y, error

    def forward(self, x, ids, weights, shared_gate=None, y=None, error=None, stream=None):
        import torch
        n = x.shape[0]
        _need(x, "x", torch.float32, (n, self.H), x.device)
        y, error = self._io_check(n, x.device, ids, weights, shared_gate, y, error)
        _check(library().moe_ffn_forward(self.handle, _ptr(x), _ptr(ids), _ptr(weights), n, _ptr(shared_gate),
                                         _ptr(y), _ptr(error), _stream(stream)), "moe_ffn_forward")
        return y, error

    def bind_forward(self, x, ids, weights, y, error, shared_gate=None, stream=None):
        """Validate the tensors of a forward() once and return a no-argument
        callable that enqueues that forward with no per-call checks (the
        pointers and the stream handle are resolved here).  For loops that
        time the library rather than the Python checks; the tensors must stay
        alive and keep their shapes while the callable is used."""
        import torch
        n = x.shape[0]
        _need(x, "x", torch.float32, (n, self.H), x.device)
        self._io_check(n, x.device, ids, weights, shared_gate, y, error)
        fn, handle = library().moe_ffn_forward, self.handle
        args = (_ptr(x), _ptr(ids), _ptr(weights), n, _ptr(shared_gate), _ptr(y), _ptr(error), _stream(stream))

        def call():
            st = fn(handle, *args)
            if st != 0:
                raise MoeError("moe_ffn_forward", st)
        return call

    def forward_q8(self, x_q8, ids, weights, shared_gate=None, y=None, error=None, stream=None):
        """forward() from canonical Q8_1 rows x_q8 (uint8 [tokens][H/32*36])."""
        import torch
        n = ids.shape[0]
        _need(x_q8, "x_q8", torch.uint8, (n, self.H // 32 * Q8_BLOCK), ids.device)
        y, error = self._io_check(n, ids.device, ids, weights, shared_gate, y, error)
        _check(library().moe_ffn_forward_q8(self.handle, _ptr(x_q8), _ptr(ids), _ptr(weights), n, _ptr(shared_gate),
                                            _ptr(y), _ptr(error), _stream(stream)), "moe_ffn_forward_q8")
        return y, error

    def replay_stage(self, stage, stream=None):
        _check(library().moe_ffn_replay_stage(self.handle, stage, _stream(stream)), "moe_ffn_replay_stage")

    def profile(self, forwards):
        """Record stage timing events for the next `forwards` forward() calls."""
        _check(library().moe_ffn_profile(self.handle, forwards), "moe_ffn_profile")

    def profile_read(self):
        """(seconds per stage summed over the recorded forwards, count)."""
        ms = (ctypes.c_double * (STAGE_FOLD + 1))()
        n = ctypes.c_int()
        _check(library().moe_ffn_profile_read(self.handle, ms, ctypes.byref(n)), "moe_ffn_profile_read")
        return [v / 1e3 for v in ms], n.value

    def debug_last(self, tokens, stream=None):
        import torch
        P = tokens * self.k + (tokens if self.has_shared else 0)
        dev = f"cuda:{self.device}"
        xq = torch.empty((tokens, self.H // 32 * Q8_BLOCK), dtype=torch.uint8, device=dev)
        mq = torch.empty((P, self.I // 32 * Q8_BLOCK), dtype=torch.uint8, device=dev)
        rt = torch.empty(tokens * self.k, dtype=torch.int32, device=dev)
        rr = torch.empty(tokens * self.k, dtype=torch.int32, device=dev)
        _check(library().moe_ffn_debug_last(self.handle, _ptr(xq), _ptr(mq), _ptr(rt), _ptr(rr), _stream(stream)),
               "moe_ffn_debug_last")
        return dict(x_q8=xq, middle_q8=mq, route_token=rt, route_rank=rr)

    def group_routes(self, ids, weights, stream=None):
        import torch
        n = ids.shape[0]
        dev = ids.device
        if not 1 <= n <= self.max_tokens:
            raise ValueError(f"tokens {n} outside 1..{self.max_tokens}")
        _routes_check(ids, weights, n, self.k, dev)
        counts = torch.empty(self.E, dtype=torch.int32, device=dev)
        offsets = torch.empty(self.E + 1, dtype=torch.int32, device=dev)
        rt = torch.empty(n * self.k, dtype=torch.int32, device=dev)
        rr = torch.empty(n * self.k, dtype=torch.int32, device=dev)
        error = torch.zeros(1, dtype=torch.int32, device=dev)
        _check(library().moe_ffn_group_routes(self.handle, _ptr(ids), _ptr(weights), n, _ptr(counts), _ptr(offsets),
                                              _ptr(rt), _ptr(rr), _ptr(error), _stream(stream)),
               "moe_ffn_group_routes")
        return dict(counts=counts, offsets=offsets, token=rt, rank=rr, error=error)

    def expert_gate_up(self, expert, x_q8, columns, path=PATH_AUTO, dots=False, stream=None):
        import torch
        dev = x_q8.device
        middle = torch.empty((columns, self.I), dtype=torch.float32, device=dev)
        mq = torch.empty((columns, self.I // 32 * Q8_BLOCK), dtype=torch.uint8, device=dev)
        gd = ud = None
        if dots:
            gd = torch.full((columns, self.I, self.H // 32), -2**31, dtype=torch.int32, device=dev)
            ud = torch.full((columns, self.I, self.H // 32), -2**31, dtype=torch.int32, device=dev)
        error = torch.zeros(1, dtype=torch.int32, device=dev)
        _check(library().moe_ffn_expert_gate_up(self.handle, expert, _ptr(x_q8), columns, _ptr(middle), _ptr(mq),
                                                _ptr(gd), _ptr(ud), path, _ptr(error), _stream(stream)),
               "moe_ffn_expert_gate_up")
        return dict(middle=middle, middle_q8=mq, gate_dots=gd, up_dots=ud, error=error)

    def expert_down(self, expert, middle_q8, columns, path=PATH_AUTO, dots=False, stream=None):
        import torch
        dev = middle_q8.device
        y = torch.empty((columns, self.H), dtype=torch.float32, device=dev)
        dd = None
        if dots:
            dd = torch.full((columns, self.H, self.I // 32), -2**31, dtype=torch.int32, device=dev)
        error = torch.zeros(1, dtype=torch.int32, device=dev)
        _check(library().moe_ffn_expert_down(self.handle, expert, _ptr(middle_q8), columns, _ptr(y), _ptr(dd), path,
                                             _ptr(error), _stream(stream)), "moe_ffn_expert_down")
        return dict(y=y, down_dots=dd, error=error)

    def expert_run(self, expert, x, repeats, path=PATH_AUTO, stream=None):
        """GpuExpert::run (src/hip/expert.hip:228-241): host float32 x
        [columns][H] through one resident expert's whole forward, `repeats`
        timed forwards.  Returns (y, timing dict, error word); y and timing are
        None when the warm-up forward raised the error word."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != self.H:
            raise ValueError(f"x: expected [columns][{self.H}] float32, got {x.shape}")
        columns = x.shape[0]
        y = np.empty_like(x)
        flags = _I(0)
        t = ExpertTiming()
        _check(library().moe_ffn_expert_run(self.handle, expert, ctypes.c_void_p(x.ctypes.data), columns,
                                            ctypes.c_void_p(y.ctypes.data), repeats, path, ctypes.byref(flags),
                                            ctypes.byref(t), _stream(stream)), "moe_ffn_expert_run")
        if flags.value:
            return None, None, flags.value
        return y, dict(upload_ms=t.upload_ms, resident_ms=t.resident_ms,
                       completed_wall_ms=t.completed_wall_ms), 0


def expf_host(x):
    """The kernels' expf (moe_expf.h) run on the CPU: float32 array in, out."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    _check(library().moe_expf_host(ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(y.ctypes.data), x.size),
           "moe_expf_host")
    return y


def expf_device(x, stream=None):
    """The kernels' expf on the GPU: float32 device tensor in, out."""
    import torch
    y = torch.empty_like(x)
    _check(library().moe_expf_device(_ptr(x), _ptr(y), x.numel(), _stream(stream)), "moe_expf_device")
    return y


def router_select(logits, top_k=10, probabilities=False, error=None, stream=None, ids=None, weights=None):
    """Device router: fp32 logits [tokens][experts] -> (ids int32 [tokens][top_k],
    weights fp32 [tokens][top_k], probabilities or None, error).  `ids` /
    `weights` may be given to write into existing tensors."""
    import torch
    n, e = logits.shape
    dev = logits.device
    _need(logits, "logits", torch.float32, (n, e), dev)
    if ids is None:
        ids = torch.empty((n, top_k), dtype=torch.int32, device=dev)
    w = weights if weights is not None else torch.empty((n, top_k), dtype=torch.float32, device=dev)
    _routes_check(ids, w, n, top_k, dev)
    p = torch.empty((n, e), dtype=torch.float32, device=dev) if probabilities else None
    if error is None:
        error = torch.zeros(1, dtype=torch.int32, device=dev)
    _need(error, "error", torch.int32, (1,), dev)
    _check(library().moe_router_select(_ptr(logits), n, e, top_k, _ptr(p), _ptr(ids), _ptr(w), _ptr(error),
                                       _stream(stream)), "moe_router_select")
    return ids, w, p, error


def read_probe(buffer, sink, nbytes=None, stream=None):
    """Enqueue a plain streaming read of `nbytes` (default: all) of a device tensor."""
    n = buffer.numel() * buffer.element_size() if nbytes is None else nbytes
    _check(library().moe_read_probe(_ptr(buffer), n, _ptr(sink), _stream(stream)), "moe_read_probe")


def quantize_q8_1(x, error=None, stream=None):
    """fp32 [cols, width] (device) -> uint8 [cols, width/32*36] canonical Q8_1."""
    import torch
    cols, width = x.shape
    _need(x, "x", torch.float32, (cols, width), x.device)
    out = torch.empty((cols, width // 32 * Q8_BLOCK), dtype=torch.uint8, device=x.device)
    if error is None:
        error = torch.zeros(1, dtype=torch.int32, device=x.device)
    _need(error, "error", torch.int32, (1,), x.device)
    _check(library().moe_quantize_q8_1(_ptr(x), _ptr(out), width, cols, _ptr(error), _stream(stream)),
           "moe_quantize_q8_1")
    return out, error


def combine(contributions, weights, shared=None, shared_gate=None, stream=None):
    import torch
    n, k, h = contributions.shape
    dev = contributions.device
    _need(contributions, "contributions", torch.float32, (n, k, h), dev)
    _need(weights, "weights", torch.float32, (n, k), dev)
    if shared is not None:
        _need(shared, "shared", torch.float32, (n, h), dev)
    if shared_gate is not None:
        _need(shared_gate, "shared_gate", torch.float32, (n,), dev)
    y = torch.empty((n, h), dtype=torch.float32, device=contributions.device)
    error = torch.zeros(1, dtype=torch.int32, device=contributions.device)
    _check(library().moe_combine(_ptr(contributions), _ptr(weights), _ptr(shared), _ptr(shared_gate), n, k, h,
                                 _ptr(y), _ptr(error), _stream(stream)), "moe_combine")
    return y, error


def memory_bytes(hidden, intermediate, experts, top_k, has_shared, max_tokens):
    cfg = Config(hidden, intermediate, experts, top_k, 1 if has_shared else 0, max_tokens)
    w, s = ctypes.c_size_t(), ctypes.c_size_t()
    _check(library().moe_ffn_memory_bytes(ctypes.byref(cfg), ctypes.byref(w), ctypes.byref(s)), "memory_bytes")
    return w.value, s.value


class MoeLinear:
    """One resident Q4_0 / Q4_1 matrix [output][input/32] (moe_linear_create):
    forward_q8 takes canonical Q8_1 columns, apply takes fp32 columns."""

    def __init__(self, type_, input, output, weights, max_columns=0, device=0):
        import torch
        self.type, self.K, self.M, self.max_columns = type_, input, output, max_columns
        self.device = device
        handle = ctypes.c_void_p()
        if isinstance(weights, np.ndarray):
            w = np.ascontiguousarray(weights, dtype=np.uint8)
            st = library().moe_linear_create(type_, input, output, max_columns, ctypes.c_void_p(w.ctypes.data), 0,
                                             device, ctypes.byref(handle))
        else:
            assert isinstance(weights, torch.Tensor) and weights.is_cuda
            st = library().moe_linear_create(type_, input, output, max_columns, _ptr(weights), 1, device,
                                             ctypes.byref(handle))
        _check(st, "moe_linear_create")
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            library().moe_linear_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_bytes(self):
        n = ctypes.c_size_t()
        _check(library().moe_linear_bytes(self.handle, ctypes.byref(n)), "moe_linear_bytes")
        return n.value

    def forward_q8(self, x_q8, columns, y=None, stream=None):
        import torch
        if x_q8.dtype != torch.uint8 or not x_q8.is_contiguous() or x_q8.numel() < columns * (self.K // 32) * Q8_BLOCK:
            raise ValueError("x_q8 must be contiguous uint8 holding columns x input/32 Q8_1 blocks")
        if y is None:
            y = torch.empty((columns, self.M), dtype=torch.float32, device=x_q8.device)
        _need(y, "y", torch.float32, (columns, self.M), x_q8.device)
        _check(library().moe_linear_forward_q8(self.handle, _ptr(x_q8), columns, _ptr(y), _stream(stream)),
               "moe_linear_forward_q8")
        return y

    def apply(self, x, y=None, error=None, stream=None):
        import torch
        n = x.shape[0]
        _need(x, "x", torch.float32, (n, self.K), x.device)
        if y is None:
            y = torch.empty((n, self.M), dtype=torch.float32, device=x.device)
        _need(y, "y", torch.float32, (n, self.M), x.device)
        if error is None:
            error = torch.zeros(1, dtype=torch.int32, device=x.device)
        _need(error, "error", torch.int32, (1,), x.device)
        _check(library().moe_linear_apply(self.handle, _ptr(x), n, _ptr(y), _ptr(error), _stream(stream)),
               "moe_linear_apply")
        return y, error

    def apply_noalloc(self, x, y, error, stream=None):
        """apply() through moe_linear_apply_noalloc: the activation staging is
        the library's static per-device array (4 MiB), not the handle's
        workspace; y and error must be given (nothing is allocated)."""
        import torch
        n = x.shape[0]
        dev = torch.device("cuda", self.device)   # the static array is set up for the handle's GPU
        _need(x, "x", torch.float32, (n, self.K), dev)
        _need(y, "y", torch.float32, (n, self.M), dev)
        _need(error, "error", torch.int32, (1,), dev)
        _check(library().moe_linear_apply_noalloc(self.handle, _ptr(x), n, _ptr(y), _ptr(error), _stream(stream)),
               "moe_linear_apply_noalloc")
        return y, error


class MoeStack:
    """A stack of resident MoE layers run back to back on one stream, eagerly
    or replayed from one captured HIP graph (torch.cuda.CUDAGraph over the
    library's launches).

    Layer l takes its own input batch x[l] (fp32 [N_l][H], device).  With
    `projections` (MoeLinear H -> H per layer) the layer input is
    h = projection.apply(x); with `routers` (MoeLinear H -> E per layer) the
    routes are chosen on the device from router.apply(h) by router_select;
    otherwise fixed device ids / weights are given to bind().  Every buffer is
    allocated by bind(), so run() allocates nothing and can be captured."""

    def __init__(self, layers, projections=None, routers=None):
        self.layers = list(layers)
        self.projections = projections
        self.routers = routers
        self.graph = None

    def bind(self, xs, ids=None, weights=None):
        import torch
        dev = xs[0].device
        self.error = torch.zeros(1, dtype=torch.int32, device=dev)
        self.steps = []
        for l, (L, x) in enumerate(zip(self.layers, xs)):
            n = x.shape[0]
            st = {"x": x, "y": torch.empty((n, L.H), dtype=torch.float32, device=dev)}
            st["h"] = torch.empty((n, L.H), dtype=torch.float32, device=dev) if self.projections else x
            if self.routers:
                st["logits"] = torch.empty((n, L.E), dtype=torch.float32, device=dev)
                st["ids"] = torch.empty((n, L.k), dtype=torch.int32, device=dev)
                st["w"] = torch.empty((n, L.k), dtype=torch.float32, device=dev)
            else:
                st["ids"], st["w"] = ids[l], weights[l]
            self.steps.append(st)
        self.graph = None

    def run(self, stream=None):
        for l, (L, st) in enumerate(zip(self.layers, self.steps)):
            if self.projections:
                self.projections[l].apply(st["x"], y=st["h"], error=self.error, stream=stream)
            if self.routers:
                self.routers[l].apply(st["h"], y=st["logits"], error=self.error, stream=stream)
                router_select(st["logits"], top_k=L.k, error=self.error, stream=stream, ids=st["ids"],
                              weights=st["w"])
            L.forward(st["h"], st["ids"], st["w"], y=st["y"], error=self.error, stream=stream)

    def capture(self):
        """Record one run() into a HIP graph (after one eager run as warm-up)."""
        import torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run()
        return self.graph

    def replay(self):
        self.graph.replay()

    def outputs(self):
        return [st["y"] for st in self.steps]
