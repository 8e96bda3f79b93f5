"""Benchmark of the routed-MoE Q4_0 expert FFN layer on one MI355X.

A "step" is one MoE layer forward (quantize + group + gate/up/SiLU/Q8 + down +
rank-order fold + shared expert) over one batch of synthetic tokens with all
inputs resident in HBM.  The headline workload is BASELINE configs[1], B8
decode (8 tokens, top-10 of 512 experts + 1 shared, H 2048, I 512), measured
cold: step i runs layer i % 48 of 48 resident layers with their own weights
(43.5 GB, far past the 256 MB Infinity Cache) on route set i % 64, so no step
finds its weights in any cache.  The K timed steps are captured into one HIP
graph (every rotated layer run once eagerly first) and the graph is replayed
--repeats times, each replay its own timed region bracketed by synchronize;
the value is the median replay, the line gives min / median / max, and the
same steps launched eagerly from Python are reported beside it
("b8_decode_eager").  The same rotation over ONE layer's bank is
reported as "b8_decode_warm" (consecutive route sets share experts, so part
of a step can hit the Infinity Cache).  Reported alongside: the 4K Zipf(1.1) prefill layer (configs[2], "prefill_4k"), the 16K
uniform prefill layer (configs[3], "prefill_16k"), the 48-layer stack of 8 + 1024
tokens with Zipf(1.3) routing (configs[4], "stack_48"), and the practical HBM
ceiling at the decode gate/up kernel's byte count ("read_ceiling": a plain
streaming read of the same number of bytes, cold).

Prints ONE JSON line.  --gpus above 1 is refused: this build runs on one GPU.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gfx906-qwen3.8fn_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
GATE_UP_BYTES_PER_EXPERT = 2 * 512 * (2048 // 32) * 18     # gate + up Q4_0 planes of one expert
DOWN_BYTES_PER_EXPERT = 2048 * (512 // 32) * 18


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_forward(layer, x, sets, steps, warmup, repeats=1):
    """Wall and GPU-event seconds per forward; step i uses route set i % len(sets)
    and, when `layer` is a list of layers, layer i % len(layer) (each with its
    own resident weights, so a rotation over many layers reads every step's
    weights from HBM).  Every forward is validated once and then enqueued
    through MoeLayer.bind_forward, so the loop times the library, not the
    per-call tensor checks.  The warm-up runs at least one forward on every
    layer of the rotation.  With repeats > 1 the timed loop of `steps` forwards
    runs that many times; returns (walls, gpus, y): per-repeat lists."""
    import torch
    layers = layer if isinstance(layer, (list, tuple)) else [layer]
    y = torch.empty((x.shape[0], layers[0].H), dtype=torch.float32, device=x.device)
    err = torch.zeros(1, dtype=torch.int32, device=x.device)
    n_calls = max(steps, warmup, len(layers))
    calls = [layers[i % len(layers)].bind_forward(x, *sets[i % len(sets)], y=y, error=err) for i in range(n_calls)]
    for i in range(max(warmup, len(layers))):
        calls[i % n_calls]()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    walls, gpus = [], []
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            calls[i]()
        e1.record(stream)
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - t0) / steps)
        gpus.append(e0.elapsed_time(e1) / 1e3 / steps)
    if int(err.cpu()[0]) != 0:
        raise RuntimeError(f"error flags {int(err.cpu()[0])}")
    if repeats == 1:
        return walls[0], gpus[0], y
    return walls, gpus, y


def time_forward_graph(layers, x, sets, steps, repeats):
    """B8 steps replayed from one captured HIP graph: step i = layers[i % L]
    on route set i % len(sets), each with its own output rows; the graph
    holds exactly `steps` steps, so one replay is one timed region of `steps`
    steps, bracketed by synchronize.  Every layer of the rotation runs once
    eagerly before the capture.  Returns (walls, gpus): seconds per step of
    each of `repeats` timed replays (wall clock and GPU events)."""
    import torch
    import moe_ffn
    order = [layers[i % len(layers)] for i in range(steps)]
    st = moe_ffn.MoeStack(order)
    st.bind([x] * steps, [sets[i % len(sets)][0] for i in range(steps)],
            [sets[i % len(sets)][1] for i in range(steps)])
    err = torch.zeros(1, dtype=torch.int32, device=x.device)
    y = torch.empty((x.shape[0], layers[0].H), dtype=torch.float32, device=x.device)
    for i, L in enumerate(layers):   # every rotated layer once, outside the graph
        L.forward(x, *sets[i % len(sets)], y=y, error=err)
    st.capture()
    st.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    walls, gpus = [], []
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        st.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - t0) / steps)
        gpus.append(e0.elapsed_time(e1) / 1e3 / steps)
    if int(st.error.cpu()[0]) != 0 or int(err.cpu()[0]) != 0:
        raise RuntimeError(f"error flags {int(st.error.cpu()[0])} / {int(err.cpu()[0])}")
    outs = st.outputs()
    st.graph = None
    return walls, gpus, outs


def spread(values, scale=1.0):
    """min / median / max of a list of timings (scaled), for the JSON line."""
    v = np.sort(np.asarray(values, dtype=np.float64)) * scale
    return {"min": float(v[0]), "median": float(np.median(v)), "max": float(v[-1]), "n": int(v.size)}


def time_stages(layer, x, sets, steps):
    """Per-stage durations of real forwards (same rotation as time_forward):
    the library records timing events (no system-scope fence) on the forward's
    stream before the first and after every stage; read once at the end.
    Returns the summed seconds per stage."""
    import torch
    layers = layer if isinstance(layer, (list, tuple)) else [layer]
    y = torch.empty((x.shape[0], layers[0].H), dtype=torch.float32, device=x.device)
    err = torch.zeros(1, dtype=torch.int32, device=x.device)
    per = -(-steps // len(layers))
    for L in layers:
        L.profile(per)
    for i in range(steps):
        layers[i % len(layers)].forward(x, *sets[i % len(sets)], y=y, error=err)
    total, count = np.zeros(4), 0
    for L in layers:
        t, n = L.profile_read()
        L.profile(0)
        total += np.array(t)
        count += n
    assert count == steps
    if int(err.cpu()[0]) != 0:
        raise RuntimeError(f"error flags {int(err.cpu()[0])}")
    return total


def pmc_traffic(kernel, units, record="pmc_b8_decode.json"):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc record
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a 1 GiB copy calibration),
    at `units` expert units per launch; None when no record exists."""
    path = os.path.join(ROOT, "profiles", record)
    try:
        rec = json.load(open(path))["kernels"][kernel]
    except (OSError, KeyError, ValueError):
        return None
    # The record holds the mean bytes per launch at its mean unit count; the
    # traffic of this kernel is linear in units (one weight set per unit).
    return rec["traffic_bytes"] / rec["units"] * units


def read_ceiling(nbytes, buffers=12, iters=48):
    """Time the library's plain streaming-read kernel (moe_read_probe) over
    `nbytes`, rotating `buffers` distinct buffers (together larger than the
    256 MB Infinity Cache) so every read is cold.  Returns seconds per read
    (back to back: `iters` launches between two events; alone: the median of
    `iters` launches each timed by its own events after a synchronize)."""
    import torch
    import moe_ffn
    nbytes = nbytes // 16 * 16
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0") for _ in range(buffers)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    for b in bufs[:2]:
        moe_ffn.read_probe(b, sink)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(iters):
        moe_ffn.read_probe(bufs[i % buffers], sink)
    e1.record(stream)
    torch.cuda.synchronize()
    back = e0.elapsed_time(e1) / 1e3 / iters
    lone = []
    for i in range(iters):
        torch.cuda.synchronize()
        e0.record(stream)
        moe_ffn.read_probe(bufs[i % buffers], sink)
        e1.record(stream)
        torch.cuda.synchronize()
        lone.append(e0.elapsed_time(e1) / 1e3)
    del bufs
    return back, float(np.median(lone))


def time_graph(stack, steps):
    """Seconds per replay of the stack's captured graph (one pass)."""
    import torch
    stack.capture()
    stack.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        stack.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    if int(stack.error.cpu()[0]) != 0:
        raise RuntimeError(f"error flags {int(stack.error.cpu()[0])}")
    stack.graph = None
    return wall, e0.elapsed_time(e1) / 1e3 / steps


def time_stack(layers, inputs, steps, warmup, repeats=1):
    """Seconds per pass of the whole stack: layer l runs on its own resident
    batch inputs[l] = (x, ids, weights), back to back on one stream.  With
    repeats > 1 the timed loop runs that many times; returns (walls, gpus):
    per-repeat lists."""
    import torch
    outs = [torch.empty((x.shape[0], L.H), dtype=torch.float32, device=x.device) for L, (x, _, _) in
            zip(layers, inputs)]
    err = torch.zeros(1, dtype=torch.int32, device="cuda:0")

    def one_pass():
        for L, (x, i, w), y in zip(layers, inputs, outs):
            L.forward(x, i, w, y=y, error=err)

    for _ in range(warmup):
        one_pass()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    walls, gpus = [], []
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            one_pass()
        e1.record(stream)
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - t0) / steps)
        gpus.append(e0.elapsed_time(e1) / 1e3 / steps)
    if int(err.cpu()[0]) != 0:
        raise RuntimeError(f"error flags {int(err.cpu()[0])}")
    if repeats == 1:
        return walls[0], gpus[0]
    return walls, gpus


def time_linear(K, M, N, iters=64, cold_bytes=320e6):
    """Seconds per moe_linear_forward_q8 of a Q4_0 [M][K/32] matrix on N
    columns, rotating enough resident copies (> the 256 MB Infinity Cache)
    that every launch reads its weights from HBM.  Returns (seconds, bytes)."""
    import torch
    import moe_ffn
    import workloads as W
    rng = np.random.default_rng(K * 7 + M)
    wts = W.q4_blocks(M * K // 32, rng).reshape(-1)
    copies = int(min(128, max(2, -(-cold_bytes // wts.size))))
    mats = [moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, K, M, wts, max_columns=N) for _ in range(copies)]
    xq, _ = moe_ffn.quantize_q8_1(torch.from_numpy(W.activations(N, hidden=K, seed=N)).to("cuda:0"))
    y = torch.empty((N, M), dtype=torch.float32, device="cuda:0")
    for L in mats[:2]:
        L.forward_q8(xq, N, y=y)
    torch.cuda.synchronize()
    # The launches are replayed from a captured graph: a few-microsecond
    # kernel launched from Python one call at a time would time the host.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            mats[i % copies].forward_q8(xq, N, y=y)
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    del graph
    for L in mats:
        L.close()
    nbytes = wts.size + N * K // 32 * 36 + N * M * 4
    return e0.elapsed_time(e1) / 1e3 / iters, nbytes


def time_calls(fn, iters=32):
    """Seconds per fn() call, fn's launches replayed from one captured graph
    (iters calls per replay, the median of 5 replays)."""
    import torch
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3 / iters)
    del graph
    return float(np.median(times))


def reference_components():
    """The reference's published component timings at its own expert shape
    (hidden 2560, intermediate 640; gfx906, results.jsonl), measured here with
    the same operations: a resident expert's whole forward (fp32 x -> quantize
    -> gate/up -> SiLU*up -> quantize -> down, GpuExpert::run) and the Q4_0 /
    Q4_1 linear projections.  Weights stay resident and are reused across
    calls, as in the reference's repeated launches."""
    import torch
    import moe_ffn
    import workloads as W
    H, I = 2560, 640
    dev0 = "cuda:0"
    out = {"expert_forward_us": {}, "expert_run": {}, "linear_us": {}}
    bank = W.q4_bank(1, hidden=H, intermediate=I, seed=4100, down_type=moe_ffn.DOWN_Q4_1)
    L = moe_ffn.MoeLayer(H, I, 1, 1, False, 128, experts_q4=bank, down_type=moe_ffn.DOWN_Q4_1)
    for n in (1, 2, 3, 128):
        x = torch.from_numpy(W.activations(n, hidden=H, seed=4101)).to(dev0)
        ids = torch.zeros((n, 1), dtype=torch.int32, device=dev0)
        w = torch.ones((n, 1), dtype=torch.float32, device=dev0)
        y = torch.empty((n, H), dtype=torch.float32, device=dev0)
        err = torch.zeros(1, dtype=torch.int32, device=dev0)
        out["expert_forward_us"][str(n)] = time_calls(lambda: L.forward(x, ids, w, y=y, error=err)) * 1e6
        if int(err.cpu()[0]) != 0:
            raise RuntimeError("reference-shape expert flagged an error")
        # GpuExpert::run's protocol (src/expert_main.cpp:88-90, 135-138): the
        # harness input, 50 repeats (5 at 128 columns), ExpertTiming fields.
        i = np.arange(H * n, dtype=np.float32)
        xh = (np.float32(0.7) * np.sin(i * np.float32(0.137)) +
              np.float32(0.2) * np.cos(i * np.float32(0.071))).astype(np.float32).reshape(n, H)
        _, t, flags = L.expert_run(0, xh, repeats=5 if n == 128 else 50)
        if flags:
            raise RuntimeError("expert_run flagged an error")
        out["expert_run"][str(n)] = t
    L.close()
    # B8 decode at this shape, Q4_1 downs (the checkpoint's layers 0-5):
    # 512 experts + shared, top-10, 64 rotated route sets.
    L = moe_ffn.MoeLayer(H, I, 512, 10, True, 8, synthetic_seed=4104, down_type=moe_ffn.DOWN_Q4_1)
    sets = [tuple(torch.from_numpy(a).to(dev0) for a in W.routes_uniform(8, seed=4105 + r)) for r in range(64)]
    x = torch.from_numpy(W.activations(8, hidden=H, seed=4106)).to(dev0)
    y = torch.empty((8, H), dtype=torch.float32, device=dev0)
    err = torch.zeros(1, dtype=torch.int32, device=dev0)
    step = [0]

    def b8():
        ids, w = sets[step[0] % 64]
        step[0] += 1
        L.forward(x, ids, w, y=y, error=err)
    out["b8_decode_q4_1_us"] = time_calls(b8, iters=64) * 1e6
    if int(err.cpu()[0]) != 0:
        raise RuntimeError("reference-shape B8 layer flagged an error")
    L.close()
    # 4K Zipf(1.1) prefill layer at this shape, Q4_1 and Q4_0 downs.
    NP = 4096
    xp = torch.from_numpy(W.activations(NP, hidden=H, seed=4107)).to(dev0)
    idp, wp = (torch.from_numpy(a).to(dev0) for a in W.routes_zipf(NP, 1.1, seed=4108))
    for name, dt in (("prefill_4k_q4_1_ms", moe_ffn.DOWN_Q4_1), ("prefill_4k_q4_0_ms", moe_ffn.DOWN_Q4_0)):
        L = moe_ffn.MoeLayer(H, I, 512, 10, True, NP, synthetic_seed=4109, down_type=dt)
        wall, _, _ = time_forward(L, xp, [(idp, wp)], 10, 2)
        out[name] = wall * 1e3
        L.close()
    rng = np.random.default_rng(4102)
    mats = {("q4_0", H, I): W.q4_blocks(I * H // 32, rng).reshape(-1),
            ("q4_0", I, H): W.q4_blocks(H * I // 32, rng).reshape(-1),
            ("q4_1", I, H): W.q4_1_blocks(H * I // 32, rng).reshape(-1)}
    cases = [("q4_0", H, I, n) for n in (1, 8, 16, 32, 128)] + [("q4_0", I, H, 128)] + \
            [("q4_1", I, H, n) for n in (1, 8, 32, 128)]
    for kind, K, M, n in cases:
        t = moe_ffn.TYPE_Q4_1 if kind == "q4_1" else moe_ffn.TYPE_Q4_0
        lin = moe_ffn.MoeLinear(t, K, M, mats[(kind, K, M)], max_columns=n)
        xq, _ = moe_ffn.quantize_q8_1(torch.from_numpy(W.activations(n, hidden=K, seed=4103)).to(dev0))
        y = torch.empty((n, M), dtype=torch.float32, device=dev0)
        out["linear_us"][f"{kind}_{K}x{M}_n{n}"] = time_calls(lambda: lin.forward_q8(xq, n, y=y)) * 1e6
        lin.close()
    return out


def cpu_baseline(x, bank, shared, ids, w, target_seconds, workers):
    """Seconds per B8 layer of the oracle's pinned pool with `workers` workers
    (one per allowed physical core), repeated for about target_seconds."""
    import oracle as O
    sec, used, _ = O.baseline_layer(x, 2048, 512, 512, bank, ids, w, shared_q4=shared, workers=workers, repeats=2)
    repeats = max(3, int(target_seconds / max(sec, 1e-6)))
    sec, used, _ = O.baseline_layer(x, 2048, 512, 512, bank, ids, w, shared_q4=shared, workers=workers,
                                    repeats=repeats)
    return sec, used, repeats


def sparse_bank(layer, experts):
    """Canonical host bank of `layer` with only `experts` exported from the
    device (the others left zero: a layer forward reads only routed experts)."""
    eb = layer.export_expert(0).size
    bank = np.zeros(layer.E * eb, np.uint8)
    for e in sorted(set(int(e) for e in np.asarray(experts).reshape(-1))):
        bank[e * eb:(e + 1) * eb] = layer.export_expert(e)
    return bank


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--repeats", type=int, default=5, help="timed repeats of the B8 headline (min/median/max)")
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-16k", action="store_true", help="skip the 16K uniform prefill layer (configs[3])")
    ap.add_argument("--no-stack", action="store_true", help="skip the 48-layer stack (configs[4])")
    ap.add_argument("--stack-steps", type=int, default=5)
    ap.add_argument("--no-linear", action="store_true", help="skip the quantized linear projections")
    ap.add_argument("--no-graph", action="store_true", help="skip the graph-captured stack passes")
    ap.add_argument("--no-refshapes", action="store_true", help="skip the reference's component shapes (2560/640)")
    ap.add_argument("--only", choices=["b8", "4k", "16k", "ep", "stack", "refshapes", "router", "linear"],
                    help="run one section alone (for profiler runs); the JSON line then holds that section only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy x5 (FETCH_SIZE/WRITE_SIZE scale for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] copy calibration: 5 x 1 GiB device copies")
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the MoE layer on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import moe_ffn
    import workloads as W

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    only = args.only
    want = lambda section: only is None or only == section
    if only is not None:
        args.no_cpu = True
        args.no_linear = only != "linear"
        args.no_refshapes = only != "refshapes"
        args.no_prefill = only not in ("4k", "16k")
        args.no_16k = only != "16k"
        args.no_stack = only != "stack"
    NL, NS = 48, 8 + 1024
    result = {}
    layers = []
    if want("b8") or want("stack"):
        # ---- resident layers: 48 with their own synthetic weights (configs[4]'s
        # stack, also the cold rotation of the B8 headline) ------------------
        log(f"[bench] creating {NL} resident layers (synthetic Q4_0, 512 experts + shared each)")
        layers = [moe_ffn.MoeLayer(2048, 512, 512, 10, True, NS, synthetic_seed=5000 + l) for l in range(NL)]

    # ---- B8 decode (headline, cold) ---------------------------------------
    route_sets = []
    if want("b8"):
        N, R = 8, 64
        xh = W.activations(N, seed=1002)
        route_sets = [W.routes_uniform(N, seed=1003 + r) for r in range(R)]
        x = dev(xh)
        sets = [(dev(i), dev(w)) for i, w in route_sets]
        touched = np.array([W.group_histogram(i)["touched"] for i, _ in route_sets])
        log(f"[bench] b8 decode: {R} route sets over {NL} layers, touched experts mean {touched.mean():.1f} "
            f"(min {touched.min()}, max {touched.max()})")
        # Headline: the steps replayed from one captured HIP graph (the
        # library's launches on the GPU's clock, no Python between them).
        walls_g, gpus_g, outs = time_forward_graph(layers, x, sets, args.steps, args.repeats)
        wall, gpu = float(np.median(walls_g)), float(np.median(gpus_g))
        # The graph's first step against the same forward run eagerly.
        y_chk, _ = layers[0].forward(x, *sets[0])
        torch.cuda.synchronize()
        if not torch.equal(outs[0].view(torch.int32), y_chk.view(torch.int32)):
            raise RuntimeError("graph replay output differs from the eager forward")
        # The same rotation launched eagerly, one Python call per step
        # (pre-validated forwards; every rotated layer warmed first).
        walls_e, gpus_e, _ = time_forward(layers, x, sets, args.steps, args.warmup, repeats=args.repeats)
        stats = layers[0].last_stats()
        # Stage durations over the same rotation; step i touched[i % R] + 1 units.
        n_stage = max(R, args.steps)
        t_stages = [time_stages(layers, x, sets, n_stage) for _ in range(args.repeats)]
        gate_rep = [float(t[1]) / n_stage for t in t_stages]
        pick = int(np.argsort(gate_rep)[len(gate_rep) // 2])   # the repeat with the median gate/up time
        t_stage = t_stages[pick]
        units = touched[np.arange(n_stage) % R] + 1
        gate_bytes = float(np.sum(units)) * GATE_UP_BYTES_PER_EXPERT
        down_bytes = float(np.sum(units)) * DOWN_BYTES_PER_EXPERT
        t_prep, t_gate, t_down, t_fold = (t_stage / n_stage).tolist()
        achieved = gate_bytes / float(t_stage[1]) / 1e9
        layer_bytes = float(np.mean([W.algorithmic_bytes(N, int(t)) for t in touched]))
        log(f"[bench] b8 cold graph wall {wall*1e6:.2f} us (repeats {[round(w*1e6, 2) for w in walls_g]}) gpu "
            f"{gpu*1e6:.2f} us; eager wall {np.median(walls_e)*1e6:.2f} us gpu {np.median(gpus_e)*1e6:.2f} us; "
            f"stages prep {t_prep*1e6:.1f} gate/up {t_gate*1e6:.2f} (repeats {[round(g*1e6, 2) for g in gate_rep]}) "
            f"down {t_down*1e6:.2f} fold {t_fold*1e6:.1f} us; items {stats}")

        result.update({
            "metric": "MoE Q4_0 expert FFN tokens/s (B8 decode, 4K prefill); % HBM/MFMA-i8 roofline",
            "value": N / wall,
            "unit": "tokens/s per MoE layer",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": wall * 1e3,
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "int8xint4->int32, fp32 accumulate",
            "data": "synthetic (seeded Q4_0 weights d=|N(0,.02)|, x~N(0,1), uniform top-10 routing, "
                    f"{R} route sets x {NL} resident layers rotated per step: cold weights)",
            "config": {"workload": "b8_decode", "tokens": N, "hidden": 2048, "intermediate": 512, "experts": 512,
                       "top_k": 10, "shared_experts": 1, "route_sets": R, "layers_rotated": NL,
                       "rotated_weight_gb": moe_ffn.memory_bytes(2048, 512, 512, 10, True, NS)[0] * NL / 1e9,
                       "touched_experts_mean": float(touched.mean()),
                       "timing": f"median of {args.repeats} timed replays of one HIP graph holding the "
                                 f"{args.steps} steps (each replay bracketed by synchronize)",
                       "gpu_event_us_per_layer": gpu * 1e6,
                       "layer_hbm_frac": layer_bytes / gpu / 1e9 / HBM_PEAK_GBS},
            "b8_spread_us": {"graph_wall": spread(walls_g, 1e6), "graph_gpu": spread(gpus_g, 1e6),
                             "eager_wall": spread(walls_e, 1e6), "eager_gpu": spread(gpus_e, 1e6),
                             "gate_up_stage": spread(gate_rep, 1e6)},
            "b8_decode_eager": {"tokens_per_s": N / float(np.median(walls_e)),
                                "us_per_layer": float(np.median(walls_e)) * 1e6,
                                "gpu_event_us": float(np.median(gpus_e)) * 1e6,
                                "note": "the same rotation launched one Python call per step (pre-validated "
                                        "forwards through ctypes), every rotated layer warmed first"},
            "roofline": {"kernel": "k_decode_gate_up (x Q8 + gate/up + SiLU + middle Q8)", "bound": "hbm",
                         "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                         "traffic": pmc_traffic("k_decode_gate_up", float(touched.mean()) + 1),
                         "bytes_per_launch": gate_bytes / n_stage, "us_per_launch": t_gate * 1e6},
            "stages_us": {"prepare": t_prep * 1e6, "gate_up": t_gate * 1e6, "down": t_down * 1e6, "fold": t_fold * 1e6},
            "down_stage_hbm_frac": down_bytes / float(t_stage[2]) / 1e9 / HBM_PEAK_GBS,
        })
    if only is None:
        # Warm extra: the same rotation of route sets over ONE layer's bank.
        wall_w, gpu_w, _ = time_forward(layers[0], x, sets, args.steps, args.warmup)
        tw = time_stages(layers[0], x, sets, n_stage) / n_stage
        result["b8_decode_warm"] = {
            "tokens_per_s": N / wall_w, "us_per_layer": wall_w * 1e6, "gpu_event_us": gpu_w * 1e6,
            "gate_up_us": tw[1] * 1e6, "down_us": tw[2] * 1e6,
            "gate_up_hbm_frac": gate_bytes / n_stage / tw[1] / 1e9 / HBM_PEAK_GBS,
            "note": "one layer's bank, 64 rotated route sets, eager: consecutive steps share experts, so part of "
                    "a step can be served from the 256 MB Infinity Cache",
        }
        log(f"[bench] b8 warm (one bank) wall {wall_w*1e6:.1f} us; gate/up {tw[1]*1e6:.1f} down {tw[2]*1e6:.1f} us")
        # Practical ceiling: a plain streaming read of the same byte count,
        # launched back to back (as the layer's kernels follow each other)
        # and launched alone (each read after a synchronize).
        nb_gate = int(gate_bytes / n_stage)
        t_read, t_lone = read_ceiling(nb_gate)
        gbs = lambda t: gate_bytes / n_stage / t / 1e9
        result["read_ceiling"] = {
            "bytes": nb_gate // 16 * 16,
            "back_to_back_us": t_read * 1e6, "back_to_back_GB/s": gbs(t_read),
            "back_to_back_frac_of_peak": gbs(t_read) / HBM_PEAK_GBS,
            "lone_us": t_lone * 1e6, "lone_GB/s": gbs(t_lone), "lone_frac_of_peak": gbs(t_lone) / HBM_PEAK_GBS,
            "gate_up_frac_of_back_to_back": t_read / t_gate, "gate_up_frac_of_lone": t_lone / t_gate,
        }
        log(f"[bench] read ceiling at {gate_bytes / n_stage / 1e6:.1f} MB: back to back {t_read * 1e6:.2f} us "
            f"({gbs(t_read):.0f} GB/s), alone {t_lone * 1e6:.2f} us ({gbs(t_lone):.0f} GB/s)")

    # ---- 4K Zipf prefill and 16K uniform prefill ----
    layer = None
    if not args.no_prefill:
        layer = moe_ffn.MoeLayer(2048, 512, 512, 10, True, 4096 if args.no_16k else 16384, synthetic_seed=1000)
    if layer is not None and want("4k"):
        NP = 4096
        xph = W.activations(NP, seed=2002)
        idp, wp = W.routes_zipf(NP, 1.1, seed=2003)
        hp = W.group_histogram(idp)
        log(f"[bench] 4k prefill: {hp}")
        walls, gpus, _ = time_forward(layer, dev(xph), [(dev(idp), dev(wp))], args.prefill_steps, 3, repeats=3)
        wall_p, gpu_p = float(np.median(walls)), float(np.median(gpus))
        ops = W.int8_ops(NP)
        pbytes = W.algorithmic_bytes(NP, hp["touched"])
        result["prefill_4k"] = {
            "tokens_per_s": NP / wall_p, "ms_per_layer": wall_p * 1e3, "gpu_event_ms": gpu_p * 1e3,
            "ms_spread": {"wall": spread(walls, 1e3), "gpu": spread(gpus, 1e3)},
            "int8_tops": ops / gpu_p / 1e12, "int8_mfma_frac": ops / gpu_p / 1e12 / INT8_PEAK_TOPS,
            "hbm_frac": pbytes / gpu_p / 1e9 / HBM_PEAK_GBS, "group_hist": hp, "items": layer.last_stats(),
        }
        log(f"[bench] 4k prefill {wall_p*1e3:.3f} ms/layer, {NP/wall_p:.0f} tok/s")
    if layer is not None and not args.no_16k:
        NP = 16384
        xph = W.activations(NP, seed=3002)
        idp, wp = W.routes_uniform(NP, seed=3003)
        hp = W.group_histogram(idp)
        log(f"[bench] 16k prefill: {hp}")
        walls, gpus, _ = time_forward(layer, dev(xph), [(dev(idp), dev(wp))], max(3, args.prefill_steps // 2), 2,
                                      repeats=3)
        wall_p, gpu_p = float(np.median(walls)), float(np.median(gpus))
        ops = W.int8_ops(NP)
        pbytes = W.algorithmic_bytes(NP, hp["touched"])
        result["prefill_16k"] = {
            "tokens_per_s": NP / wall_p, "ms_per_layer": wall_p * 1e3, "gpu_event_ms": gpu_p * 1e3,
            "ms_spread": {"wall": spread(walls, 1e3), "gpu": spread(gpus, 1e3)},
            "int8_tops": ops / gpu_p / 1e12, "int8_mfma_frac": ops / gpu_p / 1e12 / INT8_PEAK_TOPS,
            "hbm_frac": pbytes / gpu_p / 1e9 / HBM_PEAK_GBS, "group_hist": hp, "items": layer.last_stats(),
        }
        log(f"[bench] 16k prefill {wall_p*1e3:.3f} ms/layer, {NP/wall_p:.0f} tok/s")
    if layer is not None:
        layer.close()
        layer = None
        torch.cuda.empty_cache()

    # ---- one GPU's share of the 4K batch under 8-way expert parallelism ----
    # Experts 0..63 (popularity is over a seeded permutation, so the share
    # mixes popular and rare experts) and the (token, rank) pairs routed to
    # them, received as rows with one local route of weight 1.  The routed
    # fold and the shared expert run on each token's home GPU.
    if (only is None and not args.no_prefill) or only == "ep":
        NP = 4096
        xph = W.activations(NP, seed=2002)
        idp, _ = W.routes_zipf(NP, 1.1, seed=2003)
        sel = idp < 64
        tok = np.nonzero(sel)[0]
        M = int(tok.size)
        share = moe_ffn.MoeLayer(2048, 512, 64, 1, False, M, synthetic_seed=1500)
        xs = dev(np.ascontiguousarray(xph[tok]))
        ids_s = dev(np.ascontiguousarray(idp[sel].reshape(M, 1).astype(np.int32)))
        w_s = dev(np.ones((M, 1), np.float32))
        wall_s, gpu_s, _ = time_forward(share, xs, [(ids_s, w_s)], args.prefill_steps, 3)
        hs = W.group_histogram(idp[sel].reshape(M, 1), experts=64)
        result["prefill_4k_ep8_share"] = {
            "experts": 64, "rows": M, "ms": wall_s * 1e3, "gpu_event_ms": gpu_s * 1e3,
            "rows_per_s": M / wall_s, "group_hist": hs,
            "note": "routed rows of experts 0..63 of the 4K batch, k=1, no shared expert; no all-to-all",
        }
        log(f"[bench] 4k ep8 share: {M} rows on 64 experts {wall_s*1e3:.3f} ms ({hs})")
        share.close()

    # ---- device router (softmax + top-10 of 512), the step before the layer --
    router = {}
    for NR in ((8, 4096) if only in (None, "router") else ()):
        lg = dev(np.random.default_rng(4000 + NR).standard_normal((NR, 512)).astype(np.float32))
        ids_r = torch.empty((NR, 10), dtype=torch.int32, device="cuda:0")
        w_r = torch.empty((NR, 10), dtype=torch.float32, device="cuda:0")
        err_r = torch.zeros(1, dtype=torch.int32, device="cuda:0")
        lib = moe_ffn.library()
        call = lambda: lib.moe_router_select(moe_ffn._ptr(lg), NR, 512, 10, None, moe_ffn._ptr(ids_r),
                                             moe_ffn._ptr(w_r), moe_ffn._ptr(err_r), moe_ffn._stream(None))
        # Launches replayed from a graph: a few-microsecond kernel launched one
        # Python call at a time would time the host.
        router[f"tokens_{NR}_us"] = time_calls(call, iters=50) * 1e6
    if router:
        result["router_us"] = router
        log(f"[bench] router (softmax + top-10 of 512): {router}")

    # ---- non-expert Q4_0 projections (moe_linear_forward_q8), cold weights --
    if not args.no_linear:
        lin = {}
        for lk, lm, ln in ((2048, 2048, 1), (2048, 2048, 8), (2048, 2048, 128), (2048, 2048, 1032), (8192, 8192, 1),
                           (8192, 8192, 8), (8192, 8192, 128)):
            sec, nbytes = time_linear(lk, lm, ln)
            lin[f"{lk}x{lm}_n{ln}"] = {"us": sec * 1e6, "GB/s": nbytes / sec / 1e9,
                                       "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS}
            log(f"[bench] linear Q4_0 {lk}->{lm} N={ln}: {sec*1e6:.2f} us, {nbytes/sec/1e9:.0f} GB/s")
        result["linear_q4_0"] = lin

    # ---- the reference's own published component shapes (2560/640) ---------
    if not args.no_refshapes:
        result["reference_shapes"] = reference_components()
        log(f"[bench] reference shapes: {json.dumps(result['reference_shapes'])}")

    # ---- 48-layer stack, 8 decode + 1024 prefill tokens per layer --
    if not args.no_stack:
        inputs, touched_s = [], []
        for l in range(NL):
            ids_l, w_l = W.routes_zipf(NS, 1.3, seed=6000 + l)
            touched_s.append(W.group_histogram(ids_l)["touched"])
            inputs.append((dev(W.activations(NS, seed=7000 + l)), dev(ids_l), dev(w_l)))
        walls, gpus = time_stack(layers, inputs, args.stack_steps, 1, repeats=3)
        wall_s, gpu_s = float(np.median(walls)), float(np.median(gpus))
        sbytes = float(sum(W.algorithmic_bytes(NS, t) for t in touched_s))
        resident = moe_ffn.memory_bytes(2048, 512, 512, 10, True, NS)[0] * NL
        result["stack_48"] = {
            "ms_per_stack": wall_s * 1e3, "gpu_event_ms": gpu_s * 1e3, "us_per_layer": wall_s / NL * 1e6,
            "ms_spread": {"wall": spread(walls, 1e3), "gpu": spread(gpus, 1e3)},
            "tokens_per_s": NS / wall_s, "tokens_per_layer": NS,
            "hbm_frac": sbytes / gpu_s / 1e9 / HBM_PEAK_GBS, "int8_tops": W.int8_ops(NS) * NL / gpu_s / 1e12,
            "touched_experts_mean": float(np.mean(touched_s)), "resident_weight_gb": resident / 1e9,
        }
        log(f"[bench] stack of {NL}: {wall_s*1e3:.2f} ms/pass, {wall_s/NL*1e6:.1f} us/layer, "
            f"touched {np.mean(touched_s):.1f}, resident {resident/1e9:.2f} GB")
        if not args.no_graph:
            # The same pass replayed from one captured HIP graph, then the full
            # per-layer pipeline in a graph: Q4_0 H -> H projection, Q4_0 router
            # H -> E, device top-10, MoE layer (routes chosen on the device).
            S = moe_ffn.MoeStack(layers)
            S.bind([x for x, _, _ in inputs], [i for _, i, _ in inputs], [w for _, _, w in inputs])
            wall_g, gpu_g = time_graph(S, args.stack_steps)
            result["stack_48"]["graph_ms_per_stack"] = wall_g * 1e3
            log(f"[bench] stack of {NL}, one HIP graph: {wall_g*1e3:.2f} ms/pass, {wall_g/NL*1e6:.1f} us/layer")
            rng = np.random.default_rng(8000)
            projections = [moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, 2048, 2048, W.q4_blocks(2048 * 64, rng).reshape(-1),
                                             max_columns=NS) for _ in range(NL)]
            routers = [moe_ffn.MoeLinear(moe_ffn.TYPE_Q4_0, 2048, 512, W.q4_blocks(512 * 64, rng).reshape(-1),
                                         max_columns=NS) for _ in range(NL)]
            P = moe_ffn.MoeStack(layers, projections=projections, routers=routers)
            P.bind([x for x, _, _ in inputs])
            wall_p, gpu_p = time_graph(P, args.stack_steps)
            # The MoE layers alone on the routes the device router chose (they
            # differ from the Zipf routes above), to split the pipeline's time.
            M = moe_ffn.MoeStack(layers)
            M.bind([st["h"] for st in P.steps], [st["ids"] for st in P.steps], [st["w"] for st in P.steps])
            wall_m, _ = time_graph(M, args.stack_steps)
            result["stack_48"]["pipeline_graph_ms_per_stack"] = wall_p * 1e3
            result["stack_48"]["pipeline_moe_only_graph_ms_per_stack"] = wall_m * 1e3
            log(f"[bench] stack of {NL} with projection + router + top-10 per layer, one HIP graph: "
                f"{wall_p*1e3:.2f} ms/pass, {wall_p/NL*1e6:.1f} us/layer; its MoE layers alone "
                f"{wall_m/NL*1e6:.1f} us/layer")
            for m in projections + routers:
                m.close()

    # ---- CPU baseline (same weights and inputs as the first B8 step) --------
    if not args.no_cpu:
        import oracle as O
        idh, wh = route_sets[0]
        bank = sparse_bank(layers[0], idh)
        shared = layers[0].export_expert(512)
        cpus = O.physical_cpus()
        workers = max(1, min(16, len(cpus)))
        sec, used, repeats = cpu_baseline(xh, bank, shared, idh, wh, args.cpu_seconds, workers)
        sec1, used1, repeats1 = cpu_baseline(xh, bank, shared, idh, wh, args.cpu_seconds, 1)
        result["cpu_baseline"] = {
            "value": N / sec, "unit": "tokens/s per MoE layer", "cores": used, "kind": "port",
            "allowed_physical_cores": len(cpus), "workers": used,
            "value_1_worker": N / sec1, "ms_per_layer": sec * 1e3, "ms_per_layer_1_worker": sec1 * 1e3,
            "sample": f"b8_decode layer (route set 0 of layer 0) x{repeats} repeats with {used} pinned workers "
                      f"(one per allowed physical core, at most 16) and x{repeats1} with 1 worker: quantize + "
                      f"group + experts + rank-order fold + shared, oracle/moe_oracle.c AVX2 cpu_expert order",
        }
        log(f"[bench] cpu {sec*1e3:.3f} ms/layer with {used} workers ({len(cpus)} allowed physical cores), "
            f"{sec1*1e3:.3f} ms/layer with 1 worker")
    print(json.dumps(result), flush=True)
    for L in layers:
        L.close()


if __name__ == "__main__":
    main()
