"""Seeded synthetic weight/activation generators shared by the tests."""
import numpy as np

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ4_NL, Q5_0 = 8, 10, 11, 12, 13, 14, 17, 18, 21, 22, 23, 20, 6
TYPE_SIZE = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ2_XS: 74, IQ4_XS: 136, IQ4_NL: 18, Q5_0: 22}
BLOCK_SIZE = {Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256, IQ2_XS: 256, IQ4_XS: 256, IQ4_NL: 32, Q5_0: 32}
ALL = (Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, IQ2_XS, IQ4_XS, IQ4_NL, Q5_0)
# types whose activations are quantized (Q8_K / Q8_0-32); IQ2_XS, IQ4_NL and Q5_0 dot fp32 x
INT8_ACT = tuple(t for t in ALL if t not in (IQ2_XS, IQ4_NL, Q5_0))
NAMES = {Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ2_XS: "IQ2_XS", IQ4_XS: "IQ4_XS", IQ4_NL: "IQ4_NL", Q5_0: "Q5_0"}


def row_bytes(qt, cols):
    return cols // BLOCK_SIZE[qt] * TYPE_SIZE[qt]


def _fp16_bytes(v):
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def random_blocks(qt, rng, rows, cols):
    """Random block bytes (every bit pattern path) with realistic fp16 scales
    (normal and, for a share of blocks, subnormal). Q8_0 weights stay within
    [-127, 127] as every Q8_0 encoder emits."""
    nblk = rows * cols // BLOCK_SIZE[qt]
    b = rng.integers(0, 256, size=(nblk, TYPE_SIZE[qt]), dtype=np.uint8)
    mag = rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-16, -5, nblk)
    if qt in (Q4_K, Q5_K):
        b[:, 0:2] = _fp16_bytes(mag)
        b[:, 2:4] = _fp16_bytes(rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-12, -5, nblk))
    elif qt == Q6_K:
        b[:, 208:210] = _fp16_bytes(mag)
    elif qt == Q3_K:
        b[:, 108:110] = _fp16_bytes(mag)
    elif qt == Q2_K:
        b[:, 80:82] = _fp16_bytes(mag)
        b[:, 82:84] = _fp16_bytes(rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-12, -5, nblk))
    elif qt in (IQ3_XXS, IQ3_S, IQ2_S, IQ2_XS, IQ4_XS, IQ4_NL, Q5_0):
        b[:, 0:2] = _fp16_bytes(mag)
    else:
        b[:, 0:2] = _fp16_bytes(mag)
        q = b[:, 2:].view(np.int8)
        q[q == -128] = -127
    return b.ravel()


def gaussian(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def close(got, ref, rtol=1e-3, atol=1e-4):
    """The stated fp32 tolerance: |got - ref| <= atol + rtol * |ref|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    return bool((err <= bound).all()), float((err / bound).max()) if err.size else 0.0


def oracle_matmul_par(oracle, qt, w, x, rows, cols):
    """oracle.matmul split over row chunks run in parallel threads (the C call
    releases the GIL; rows are independent, so the result is the same array
    the single call gives)."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    rb = row_bytes(qt, cols)
    w = np.ascontiguousarray(w, np.uint8).reshape(rows, rb)
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    try:
        ncpu = len(os.sched_getaffinity(0))
    except AttributeError:
        ncpu = os.cpu_count() or 1
    nth = max(1, min(16, ncpu, rows))
    bounds = np.linspace(0, rows, nth + 1).astype(int)
    parts = [(int(a), int(b)) for a, b in zip(bounds[:-1], bounds[1:]) if b > a]
    with ThreadPoolExecutor(len(parts)) as ex:
        outs = list(ex.map(lambda ab: oracle.matmul(qt, w[ab[0]:ab[1]], x, ab[1] - ab[0], cols), parts))
    return np.concatenate(outs, axis=1)


def tile_edges(n, tile, extra, rng):
    """Sorted indices: the first and last index of every `tile`-sized tile of
    range(n), the whole last tile, and `extra` seeded random ones."""
    idx = set()
    for t0 in range(0, n, tile):
        idx.add(t0)
        idx.add(min(n, t0 + tile) - 1)
    idx.update(range((n - 1) // tile * tile, n))
    idx.update(rng.choice(n, size=min(n, extra), replace=False).tolist())
    return np.array(sorted(idx), dtype=np.int64)
