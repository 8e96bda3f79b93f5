"""Deterministic inputs for the golden fixtures (no reference code here).

Everything is derived from splitmix64 over integer counters with wrapping
uint64 arithmetic, so the bytes do not depend on numpy's random streams.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(counter):
    with np.errstate(over="ignore"):
        z = counter.astype(np.uint64) + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def stream(seed, n):
    return splitmix64(np.arange(n, dtype=np.uint64) + np.uint64(seed) * np.uint64(1 << 40))


def uniform(seed, n):
    """float64 in [0, 1)."""
    return (stream(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def q4_matrix(seed, K, M, negative_scales=True):
    """M rows x K/32 canonical Q4_0 blocks; scales in [2^-12, 2^-4], some negative."""
    nb = M * K // 32
    u = uniform(seed, nb)
    d = (np.exp2(-12.0 + 8.0 * u)).astype(np.float32)
    if negative_scales:
        d = np.where(stream(seed + 7, nb) % np.uint64(3) == 0, -d, d)
    blocks = np.empty((nb, 18), np.uint8)
    blocks[:, :2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    codes = stream(seed + 13, nb * 2).view(np.uint8).reshape(nb, 16)
    blocks[:, 2:] = codes
    return blocks.reshape(-1)


def q4_1_matrix(seed, K, M):
    """M rows x K/32 canonical Q4_1 blocks {half d; half m; 16 code bytes}:
    d as q4_matrix (signed), m about -8*d so values stay centred, with a
    seeded spread of +-25% and some exact zeros."""
    nb = M * K // 32
    q4 = q4_matrix(seed, K, M).reshape(nb, 18)
    d = q4[:, :2].copy().view(np.float16).astype(np.float32).reshape(nb)
    u = uniform(seed + 29, nb)
    m = (-8.0 * d * (0.75 + 0.5 * u)).astype(np.float32)
    m = np.where(stream(seed + 31, nb) % np.uint64(17) == 0, np.float32(0), m)
    blocks = np.empty((nb, 20), np.uint8)
    blocks[:, :2] = q4[:, :2]
    blocks[:, 2:4] = m.astype(np.float16).view(np.uint8).reshape(nb, 2)
    blocks[:, 4:] = q4[:, 2:]
    return blocks.reshape(-1)


def expert_weights(H, I, seed=101):
    return q4_matrix(seed, H, I), q4_matrix(seed + 1, H, I), q4_matrix(seed + 2, I, H)


def expert_input(cols, H, seed=303):
    u = uniform(seed, cols * H)
    return ((u * 6.0 - 3.0) * (1.0 + 3.0 * (np.arange(cols * H) % 7 == 0))).astype(np.float32).reshape(cols, H)


def quant_blocks():
    """[B, 32] fp32 blocks: random magnitudes across 2^-30..2^20, plus edge
    patterns (zeros, ties, tiny scales, overflow, nonfinite)."""
    rows = []
    u = uniform(11, 256 * 32).reshape(256, 32)
    e = np.floor(uniform(12, 256) * 50.0 - 30.0)
    rows.append(((u * 2.0 - 1.0) * np.exp2(e)[:, None]).astype(np.float32))
    rows.append(np.float32(np.round((u[:64] * 2.0 - 1.0) * 8.0) / 2.0))          # many exact ties
    tiny = np.full((8, 32), 0.0, np.float32)
    tiny[0, :] = 3.4e-6
    tiny[1, :] = -3.4e-6
    tiny[2, 0] = np.float32(127.0) * np.float32(np.nextafter(np.float32(2.0 ** -25), np.float32(1.0)))
    tiny[3, 0] = np.float32(np.ldexp(127.0, -25))
    tiny[4, 0] = np.float32(np.finfo(np.float32).tiny)
    tiny[5, 0] = np.float32(1.4e-45) * np.float32(128.0)                          # unsafe rounded code
    tiny[6, 0] = np.float32(1.4e-45)                                              # FP32 scale underflow
    tiny[7, :] = 3000.0                                                           # raw sum overflows half
    rows.append(tiny)
    bad = np.ones((3, 32), np.float32)
    bad[0, 5] = np.inf
    bad[1, 31] = -np.inf
    bad[2, 0] = np.nan
    rows.append(bad)
    rows.append(np.zeros((1, 32), np.float32))
    neg0 = np.zeros((1, 32), np.float32)
    neg0[0, ::2] = -0.0
    rows.append(neg0)
    return np.ascontiguousarray(np.concatenate(rows).astype(np.float32))


def q8_random(seed, cols, K):
    """Opaque Q8_1 inputs: any codes incl. -128, headers from a finite set."""
    from_set = np.array([0x2800, 0xa800, 0x3401, 0xb401, 0x0001, 0x8001, 0x3003, 0xb003], np.uint16)
    nb = cols * K // 32
    out = np.zeros((nb, 36), np.uint8)
    hdr = from_set[(stream(seed, nb * 2) % np.uint64(8)).astype(np.int64)].reshape(nb, 2)
    out[:, :4] = hdr.view(np.uint8).reshape(nb, 4)
    out[:, 4:] = stream(seed + 1, nb * 4).view(np.uint8).reshape(nb, 32)
    return out.reshape(-1)


def matmul_case():
    """name -> (weights, K, M, q8 input bytes)."""
    cases = {}
    for cols in (1, 2, 3, 4, 7):
        cases[f"k64_m5_n{cols}"] = (q4_matrix(40 + cols, 64, 5), 64, 5, q8_random(60 + cols, cols, 64))
    cases["k2048_m32_n3"] = (q4_matrix(80, 2048, 32), 2048, 32, q8_random(81, 3, 2048))
    cases["k512_m64_n3"] = (q4_matrix(82, 512, 64), 512, 64, q8_random(83, 3, 512))
    return cases


def route_cases():
    """name -> (ids [N][10] int32, weights [N][10] fp32); reference patterns plus random."""
    cases = {}
    bits = np.array([0, 0x80000000, 1, 0x007fffff, 0x00800000, 0x3dcccccd, 0x3f800000, 0x7f7fffff, 0x3f000001,
                     0x4f123456], np.uint32)
    for n in (1, 7, 64, 1024):
        t = np.arange(n)[:, None]
        r = np.arange(10)[None, :]
        ids = ((511 + 37 * t + 73 * r) % 512).astype(np.int32)
        w = bits[(11 * t + 3 * r) % 10].view(np.float32)
        cases[f"pattern_n{n}"] = (ids, np.ascontiguousarray(w))
    rnd = uniform(500, 300 * 512).reshape(300, 512)
    ids = np.argsort(rnd, axis=1)[:, :10].astype(np.int32)
    cases["random_n300"] = (np.ascontiguousarray(ids), uniform(501, 3000).astype(np.float32).reshape(300, 10))
    dup = cases["random_n300"][0].copy()
    dup[5, 3] = dup[5, 1]
    cases["duplicate"] = (dup, cases["random_n300"][1])
    badid = cases["random_n300"][0].copy()
    badid[7, 9] = 512
    cases["bad_id"] = (badid, cases["random_n300"][1])
    negw = cases["random_n300"][1].copy()
    negw[3, 2] = -0.5
    cases["negative_weight"] = (cases["random_n300"][0], negw)
    return cases
