"""Write the golden fixtures under tests/golden/ from the reference's own CPU
code, compiled in this container into oracle/_ref/libref.so (oracle/Makefile
builds it from /root/reference/src/{quant,cpu_expert,routes,linear_reference}.cpp).

Run here (not on the GPU box, which has no reference):
    make -C oracle && python tests/golden/make_golden.py

Fixtures are data only: inputs that cannot be regenerated cheaply, and the
reference's outputs.  Large inputs (expert weights) are regenerated from the
portable splitmix64 generator in golden_inputs.py; the fixture stores their
SHA-256 so a generator change is detected.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

import oracle as O  # noqa: E402
from golden_inputs import expert_weights, quant_blocks, matmul_case, route_cases, expert_input, q4_1_matrix  # noqa: E402


def quant_fixture():
    blocks = quant_blocks()
    status = np.zeros(len(blocks), np.int32)
    q8 = np.zeros((len(blocks), 36), np.uint8)
    for i, b in enumerate(blocks):
        rc, out = O.ref_quantize_q8(b.reshape(1, 32))
        status[i] = rc
        if rc == 0:
            q8[i] = out.view(np.uint8).reshape(36)
    np.savez(os.path.join(HERE, "quant_q8.npz"), inputs=blocks, status=status, q8=q8)
    print("quant_q8.npz", len(blocks), "blocks,", int((status != 0).sum()), "rejected")


def expert_fixture():
    gate, up, down = expert_weights(2560, 640)
    x = expert_input(3, 2560)
    rc, xq = O.ref_quantize_q8(x)
    assert rc == 0
    st, out = O.ref_cpu_expert(gate, up, down, xq)
    assert st == 0, st
    sha = hashlib.sha256(gate.tobytes() + up.tobytes() + down.tobytes()).hexdigest()
    np.savez(os.path.join(HERE, "cpu_expert_2560x640.npz"), x=x, x_q8=xq.view(np.uint8), gate=out["gate"],
             up=out["up"], middle=out["middle"], middle_q8=out["middle_q8"].view(np.uint8), y=out["y"],
             weights_sha256=np.array(sha))
    print("cpu_expert_2560x640.npz sha", sha[:16])


def expert_q41_fixture():
    """The same expert shape with a Q4_1 down matrix (gate/up Q4_0)."""
    gate, up, _ = expert_weights(2560, 640)
    down = q4_1_matrix(404, 640, 2560)
    x = expert_input(3, 2560)
    rc, xq = O.ref_quantize_q8(x)
    assert rc == 0
    st, out = O.ref_cpu_expert_q41(gate, up, down, xq)
    assert st == 0, st
    sha = hashlib.sha256(gate.tobytes() + up.tobytes() + down.tobytes()).hexdigest()
    np.savez(os.path.join(HERE, "cpu_expert_2560x640_q41.npz"), middle=out["middle"],
             middle_q8=out["middle_q8"].view(np.uint8), y=out["y"], weights_sha256=np.array(sha))
    print("cpu_expert_2560x640_q41.npz sha", sha[:16])


def matmul_fixture():
    cases = {}
    for name, (w, K, M, xq) in matmul_case().items():
        for variant, tag in ((0, "scalar"), (1, "avx2")):
            cases[f"{name}_{tag}"] = O.ref_matmul(variant, w, K, M, xq)
        if O.as_q8(xq).size // (K // 32) <= 3:
            cases[f"{name}_q8ref"] = O.ref_matmul(2, w, K, M, xq)
    np.savez(os.path.join(HERE, "matmul.npz"), **cases)
    print("matmul.npz", sorted(cases))


def routes_fixture():
    out = {}
    for name, (ids, w) in route_cases().items():
        rc, g = O.ref_route_groups(ids, w)
        out[f"{name}_status"] = np.array(rc)
        if rc == 0:
            for key in ("token", "rank", "expert", "counts"):
                out[f"{name}_{key}"] = g[key]
            out[f"{name}_weight_bits"] = g["weight"].view(np.uint32)
    np.savez(os.path.join(HERE, "routes.npz"), **out)
    print("routes.npz", len(route_cases()), "cases")


if __name__ == "__main__":
    if not O.ref_available():
        sys.exit("oracle/_ref/libref.so missing: run make -C oracle (needs /root/reference)")
    quant_fixture()
    expert_fixture()
    expert_q41_fixture()
    matmul_fixture()
    routes_fixture()
