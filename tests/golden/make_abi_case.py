"""Writes tests/golden/abi_caller_case.bin, the expected outputs of the
compiled C++ caller tests/abi_caller.cpp, from the CPU oracle.

The caller builds its weights, x and router logits from an integer hash; this
script rebuilds the same bytes with numpy (the hash and layout are restated
here and must stay in step with abi_caller.cpp), runs the oracle's router
(softmax + top-k selection) and whole MoE layer on them, and stores, per
batch, the expected ids, weights and y.  Shape: H 2048, I 512, 32 experts +
shared, top-4; batches of 2 tokens (decode path, no shared gate), 24 tokens
(grouped, gated) and 3 tokens (decode path, gated).  A gated batch's shared
gate logits are the dense H -> 1 projection of x with hashed weights, fp32
products added in element order, as the caller computes them.

File layout (little endian): int32 magic 0x4D4F4532, H, I, E, k, ncases,
pad, pad; int32 tokens[ncases]; int32 gated[ncases]; then per case: int32
ids[n][k], float32 weights[n][k], float32 y[n][H].

Run in this container: python tests/golden/make_abi_case.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

H, I, E, K = 2048, 512, 32, 4
TOKENS = (2, 24, 3)
GATED = (0, 1, 1)
M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def mix(z):
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def matrix(m, e, rows, bpr):
    g = np.arange(rows * bpr, dtype=np.uint64)
    h = mix((np.uint64(m) << np.uint64(56)) ^ (np.uint64(e) << np.uint64(40)) ^ g)
    out = np.empty((rows * bpr, 18), np.uint8)
    d = (np.uint64(0x1C00) | (h & np.uint64(0x3FF))).astype(np.uint16)
    out[:, :2] = d.view(np.uint8).reshape(-1, 2)
    with np.errstate(over="ignore"):
        c1 = mix(h + np.uint64(1))
    out[:, 2:10] = mix(h).view(np.uint8).reshape(-1, 8)
    out[:, 10:18] = c1.view(np.uint8).reshape(-1, 8)
    return out.reshape(-1)


def expert(e):
    return np.concatenate([matrix(0, e, I, H // 32), matrix(1, e, I, H // 32), matrix(2, e, H, I // 32)])


def hashed(tag, n, scale):
    with np.errstate(over="ignore"):
        v = mix(np.uint64(tag) + np.arange(n, dtype=np.uint64))
    return ((v & np.uint64(0xFFFF)).astype(np.int64) - 32768).astype(np.float32) * np.float32(scale)


def main():
    bank = np.concatenate([expert(e) for e in range(E)])
    shared = expert(E)
    parts = [np.array([0x4D4F4532, H, I, E, K, len(TOKENS), 0, 0], np.int32), np.array(TOKENS, np.int32),
             np.array(GATED, np.int32)]
    gate_w = hashed(0x6A7E000000, H, 1.0 / 1048576)
    for c, n in enumerate(TOKENS):
        x = hashed(0xA5C0000000 + 0x1000000 * c, n * H, 1.0 / 16384).reshape(n, H)
        logits = hashed(0xD3F0000000 + 0x1000000 * c, n * E, 1.0 / 8192).reshape(n, E)
        prob, f1 = O.router_softmax(logits)
        ids, w, f2 = O.select_routes(prob, top_k=K)
        assert f1 == 0 and f2 == 0
        gate = None
        if GATED[c]:
            # fp32 products, accumulated left to right (add.accumulate is sequential)
            gate = np.add.accumulate((x * gate_w[None, :]).astype(np.float32), axis=1, dtype=np.float32)[:, -1]
            print(f"case {c}: gate logits {np.round(gate, 3).tolist()[:4]}...")
        y = O.moe_layer(x, H, I, E, bank, ids, w, shared_q4=shared, shared_gate=gate)["y"]
        parts += [ids.astype(np.int32).reshape(-1), w.astype(np.float32).reshape(-1), y.astype(np.float32).reshape(-1)]
        print(f"case {c}: {n} tokens, ids {ids.tolist()[:2]}..., rms(y) {float(np.sqrt(np.mean(y.astype(np.float64) ** 2))):.4f}")
    out = os.path.join(HERE, "abi_caller_case.bin")
    with open(out, "wb") as f:
        for p in parts:
            f.write(np.ascontiguousarray(p).tobytes())
    print(f"wrote {out} ({os.path.getsize(out)} bytes)")


if __name__ == "__main__":
    main()
