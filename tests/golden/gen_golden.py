"""Write the golden vectors in tests/golden/golden.npz from the COMPILED
REFERENCE (oracle/_ref/libtcref.so, built from the reference sources in place by
oracle/Makefile). Run in the build container, where the reference tree exists:

    make -C oracle && python tests/golden/gen_golden.py

Every array is data: inputs and the reference functions' outputs on them. The
fixture is what the CPU tests pin the C restatement (oracle/oracle.c) against,
and what the GPU tests compare the HIP library against, on the GPU box where
the reference does not exist.
"""
import ctypes
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")
# BASELINE widths of the wide mat-vec goldens: (name, type, widths)
WIDE_COLS = (3584, 4096, 5120, 17408, 18944)
WIDE_CASES = (("q4k", O.Q4_K, (3584, 5120, 17408, 18944)), ("q6k", O.Q6_K, (3584, 17408, 18944)),
              ("iq3", O.IQ3_XXS, (3584, 17408, 18944)), ("q80", O.Q8_0, (4096, 5120, 17408)))
MOE_SEED = 777


def moe_weights(encode_q4k, E, H, FF, seed=MOE_SEED):
    """MoE expert weights: Q4_K encodings of seeded N(0, 0.1^2) matrices. The bytes
    are not stored; the golden holds their SHA-256, and a test re-creates them
    with the same generator (numpy PCG64, stable across numpy versions)."""
    r = np.random.default_rng(seed)
    wg = encode_q4k((r.standard_normal((E * FF, H)) * 0.1).astype(np.float32))
    wu = encode_q4k((r.standard_normal((E * FF, H)) * 0.1).astype(np.float32))
    wd = encode_q4k((r.standard_normal((E * H, FF)) * 0.1).astype(np.float32))
    return wg, wu, wd


def iq3_random_blocks(rng, nblk, d_half=0x3CA4):
    """Random IQ3_XXS bytes with a realistic fp16 d (the reference's own
    DequantizeTest.Q8KFusedMatvecAcrossWidths, unit_tests/DequantizeTest.cpp:1216,
    uses random bytes and d = fp16 0x3CA4)."""
    b = rng.integers(0, 256, size=(nblk, 98), dtype=np.uint8)
    b[:, 0] = d_half & 0xFF
    b[:, 1] = d_half >> 8
    return b.ravel()


def q6k_random_blocks(rng, nblk):
    """Random Q6_K bytes: random 6-bit planes and int8 scales, fp16 d in
    [2^-10, 2^-6)."""
    b = rng.integers(0, 256, size=(nblk, 210), dtype=np.uint8)
    d = (rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-10, -6, nblk)).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def q4k_random_blocks(rng, nblk):
    b = rng.integers(0, 256, size=(nblk, 144), dtype=np.uint8)
    d = (rng.uniform(1.0, 2.0, (nblk, 2)) * 2.0 ** rng.integers(-9, -5, (nblk, 2))).astype(np.float16)
    b[:, 0:4] = d.view(np.uint8).reshape(nblk, 4)
    return b.ravel()


def q5k_random_blocks(rng, nblk):
    """Random Q5_K bytes (every scale/min code, qh and qs bit pattern) with
    fixed normal fp16 d and dmin."""
    b = rng.integers(0, 256, (nblk, 176), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(np.float16(0.0131).tobytes(), np.uint8)
    b[:, 2:4] = np.frombuffer(np.float16(0.0042).tobytes(), np.uint8)
    return b.ravel()


def q3k_random_blocks(rng, nblk):
    """Random Q3_K bytes (every hmask, 2-bit and 6-bit scale pattern) with a
    fixed normal fp16 d."""
    b = rng.integers(0, 256, (nblk, 110), dtype=np.uint8)
    b[:, 108:110] = np.frombuffer(np.float16(0.0027).tobytes(), np.uint8)
    return b.ravel()


def iq3s_random_blocks(rng, nblk):
    """Random IQ3_S bytes (every grid index, qh bit, sign and scale nibble)
    with a fixed normal fp16 d."""
    b = rng.integers(0, 256, (nblk, 110), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(np.float16(0.0009).tobytes(), np.uint8)
    return b.ravel()


def iq2s_random_blocks(rng, nblk):
    """Random IQ2_S bytes (every grid index, qh bits, sign and scale nibble)
    with a fixed normal fp16 d."""
    b = rng.integers(0, 256, (nblk, 82), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(np.float16(0.0011).tobytes(), np.uint8)
    return b.ravel()


def q2k_random_blocks(rng, nblk):
    """Random Q2_K bytes (every scale/min nibble and 2-bit pattern) with fixed
    normal fp16 d and dmin."""
    b = rng.integers(0, 256, (nblk, 84), dtype=np.uint8)
    b[:, 80:82] = np.frombuffer(np.float16(0.0093).tobytes(), np.uint8)
    b[:, 82:84] = np.frombuffer(np.float16(0.0051).tobytes(), np.uint8)
    return b.ravel()


def iq2xs_random_blocks(rng, nblk):
    """Random IQ2_XS bytes (every codebook index, sign index and scale nibble)
    with a fixed normal fp16 d."""
    b = rng.integers(0, 256, (nblk, 74), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(np.float16(0.0011).tobytes(), np.uint8)
    return b.ravel()


def iq4xs_random_blocks(rng, nblk):
    """Random IQ4_XS bytes (every nibble, 6-bit scale and scales_h pattern)
    with normal fp16 d of varied exponent."""
    b = rng.integers(0, 256, (nblk, 136), dtype=np.uint8)
    d = (rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-14, -8, nblk)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def iq4nl_random_blocks(rng, nblk):
    """Random IQ4_NL bytes (every nibble) with normal fp16 d of varied exponent."""
    b = rng.integers(0, 256, (nblk, 18), dtype=np.uint8)
    d = (rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-14, -6, nblk)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def q50_random_blocks(rng, nblk):
    """Random Q5_0 bytes (every nibble and high-bit pattern) with normal fp16 d
    of varied exponent."""
    b = rng.integers(0, 256, (nblk, 22), dtype=np.uint8)
    d = (rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-14, -6, nblk)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def q80_random_blocks(rng, nblk):
    b = rng.integers(0, 256, size=(nblk, 34), dtype=np.uint8)
    d = (rng.uniform(1.0, 2.0, nblk) * 2.0 ** rng.integers(-10, -6, nblk)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def act_edge_cases(rng):
    """Activation rows that exercise the quantizer's rules: a zero block, ties
    in |x| with opposite signs (first one wins), a constant block, a single
    spike, values that land exactly on .5 after scaling, and gaussians."""
    rows = []
    x = rng.standard_normal(1024).astype(np.float32)
    x[0:256] = 0.0                                    # zero block
    x[256:512] = rng.standard_normal(256).astype(np.float32)
    x[300], x[301] = -3.5, 3.5                        # tie, negative first
    x[512:768] = 0.75                                 # constant block
    x[768:1024] = 0.0
    x[900] = -2.0                                     # spike
    x[901:905] = np.array([1.0, -1.0, 0.5, 0.25], np.float32) * (2.0 / 127.0) * 0.5
    rows.append(x)
    y = rng.standard_normal(1024).astype(np.float32)
    y[10], y[20] = 4.0, -4.0                          # tie, positive first
    rows.append(y)
    rows.append((rng.standard_normal(1024) * 0.02).astype(np.float32))
    rows.append(rng.standard_normal(1024).astype(np.float32))
    return np.stack(rows)


def main():
    if not O.available_reference():
        sys.exit("oracle/_ref/libtcref.so is not built (make -C oracle ref)")
    ref = O.Reference(threads=1)
    rng = np.random.default_rng(20261201)
    g = {}

    # fp16 <-> fp32: the full halfToFloat table (digest + every 97th entry), and
    # floatToHalf on a log-spread sample that crosses the subnormal range.
    h2f = np.array([ref.lib.ref_half_to_float(h) for h in range(65536)], np.float32)
    g["h2f_sha256"] = np.frombuffer(hashlib.sha256(h2f.tobytes()).digest(), np.uint8)
    g["h2f_sample_idx"] = np.arange(0, 65536, 97, dtype=np.uint16)
    g["h2f_sample"] = h2f[g["h2f_sample_idx"]]
    f = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-9, 5, 4096)).astype(np.float32)
    g["f2h_in"] = f
    g["f2h_out"] = np.array([ref.lib.ref_float_to_half(float(v)) for v in f], np.uint16)

    # Q8_K activation quantizer (include/GGMLDequantize.hpp:2769).
    xa = act_edge_cases(rng)
    g["q8k_x"] = xa
    qs, d, bs = zip(*[ref.quantize_q8k(r) for r in xa])
    g["q8k_qs"], g["q8k_d"], g["q8k_bsums"] = np.stack(qs), np.stack(d), np.stack(bs)

    # Block decoders on random bytes (every bit pattern path).
    g["deq_q4k_w"] = q4k_random_blocks(rng, 8)
    g["deq_q4k_y"] = ref.dequant(O.Q4_K, g["deq_q4k_w"], 8, 256)
    g["deq_q6k_w"] = q6k_random_blocks(rng, 8)
    g["deq_q6k_y"] = ref.dequant(O.Q6_K, g["deq_q6k_w"], 8, 256)
    g["deq_iq3_w"] = iq3_random_blocks(rng, 8)
    g["deq_iq3_y"] = ref.dequant(O.IQ3_XXS, g["deq_iq3_w"], 8, 256)
    g["deq_q80_w"] = q80_random_blocks(rng, 64)
    g["deq_q80_y"] = ref.dequant(O.Q8_0, g["deq_q80_w"], 8, 256)

    # Q4_K encoder (src/cpp/core/GGMLQuantize.cpp:47): the representable ramp of
    # DequantizeTest.cpp:1305, unit gaussians and N(0, 0.02) rows.
    ramp = (np.arange(256) % 16 - 7.5).astype(np.float32)
    enc_x = np.stack([ramp,
                      rng.standard_normal(256).astype(np.float32),
                      (rng.standard_normal(256) * 0.02).astype(np.float32),
                      (rng.standard_normal(256) * 0.5 + 0.3).astype(np.float32)])
    g["enc_q4k_x"] = enc_x
    g["enc_q4k_out"] = ref.encode_q4k(enc_x).reshape(4, 144)

    # Mat-vec kernels, S = 1 and S = 4 tokens, cols = 512 (Q8_0 also 96 cols).
    # Weights: random bytes (full bit coverage) and, for Q4_K, the repo's own
    # quantizer on N(0,1) rows (d normal) and on N(0,0.02) rows (BASELINE's
    # distribution, where floatToHalf flushes most d to 0).
    rows, cols = 48, 512
    X1 = rng.standard_normal((1, cols)).astype(np.float32)
    X4 = rng.standard_normal((4, cols)).astype(np.float32)
    X4[2, :256] = 0.0  # one all-zero activation block
    g["mm_x1"], g["mm_x4"] = X1, X4
    nb = cols // 256
    cases = {
        "q4k_rand": (O.Q4_K, q4k_random_blocks(rng, rows * nb)),
        "q4k_enc1": (O.Q4_K, ref.encode_q4k(rng.standard_normal((rows, cols)).astype(np.float32))),
        "q4k_enc002": (O.Q4_K, ref.encode_q4k((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))),
        "q6k_rand": (O.Q6_K, q6k_random_blocks(rng, rows * nb)),
        "iq3_rand": (O.IQ3_XXS, iq3_random_blocks(rng, rows * nb)),
        "q80_rand": (O.Q8_0, q80_random_blocks(rng, rows * cols // 32)),
    }
    for name, (qt, w) in cases.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(qt, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(qt, w, X4, rows, cols)

    # Q8_0 with cols % 256 != 0 (96 = 3 blocks).
    w96 = q80_random_blocks(rng, 16 * 3)
    x96 = rng.standard_normal((2, 96)).astype(np.float32)
    g["mm_q80c96_w"], g["mm_q80c96_x"] = w96, x96
    g["mm_q80c96_y"] = ref.matmul(O.Q8_0, w96, x96, 16, 96)

    # Unit probes: Q8_0 weight rows with d = 1 and a single +1 at column i give
    # out[i] = 1 * d8 * xq[i] through the reference's own kernel, which pins the
    # kernel-internal 32-wide activation quantizer (SIMDMatMulVecAVX2.cpp:4296).
    pc = 256
    wp = np.zeros((pc, pc // 32, 34), np.uint8)
    for i in range(pc):
        wp[i, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        wp[i, i // 32, 2 + i % 32] = 1
    xp = act_edge_cases(rng)[:, :pc].copy()
    g["probe_q80_x"] = xp
    g["probe_q80_y"] = ref.matmul(O.Q8_0, wp.ravel(), xp, pc, pc)

    # IQ3_XXS unit probe of DequantizeTest.cpp:1238-1263: x = e0 makes the
    # fused result equal the first dequantized weight of each row.
    for c in (1536, 2048, 3584):
        w = iq3_random_blocks(rng, 8 * c // 256)
        e0 = np.zeros((1, c), np.float32)
        e0[0, 0] = 1.0
        g[f"iq3probe_{c}_w"] = w
        g[f"iq3probe_{c}_y"] = ref.matmul(O.IQ3_XXS, w, e0, 8, c)

    # MoE composition (src/cpp/core/ModelMoE.cpp:660-672, 990-1002) on tiny
    # experts, each matmul through the reference kernel; SwiGLU and the
    # rank-order weighted sum in float32 (tolerance-compared).
    E, K, H, FF, S = 6, 3, 512, 256, 3
    wg, wu, wd = moe_weights(ref.encode_q4k, E, H, FF)
    mrng = np.random.default_rng(MOE_SEED + 1)
    xm = mrng.standard_normal((S, H)).astype(np.float32)
    ids = np.stack([mrng.choice(E, K, replace=False) for _ in range(S)]).astype(np.int32)
    lg = mrng.standard_normal((S, K)).astype(np.float32)
    wts = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
    gB, dB = FF * (H // 256) * 144, H * (FF // 256) * 144
    out = np.zeros((S, H), np.float32)
    for s in range(S):
        for r in range(K):
            e = ids[s, r]
            gg = ref.matmul(O.Q4_K, wg[e * gB:(e + 1) * gB], xm[s], FF, H)[0]
            uu = ref.matmul(O.Q4_K, wu[e * gB:(e + 1) * gB], xm[s], FF, H)[0]
            hh = (gg / (np.float32(1.0) + np.exp(-gg))) * uu
            dd = ref.matmul(O.Q4_K, wd[e * dB:(e + 1) * dB], hh.astype(np.float32), H, FF)[0]
            out[s] = out[s] + wts[s, r] * dd
    digest = hashlib.sha256(wg.tobytes() + wu.tobytes() + wd.tobytes()).digest()
    g.update(moe_wsha256=np.frombuffer(digest, np.uint8), moe_x=xm, moe_ids=ids, moe_wts=wts,
             moe_y=out, moe_dims=np.array([E, K, H, FF, S, MOE_SEED], np.int64))

    # Q5_K (a type the reference dispatches beyond BASELINE's configs): its
    # dequant and matMulVecBatchQ5K_Q8K_AVX2 (SIMDMatMulVecAVX2.cpp:3842) on
    # random blocks and on this build's encoder output (the reference has no
    # Q5_K encoder). Own generator, so the vectors above are unchanged.
    r5 = np.random.default_rng(20261202)
    g["deq_q5k_w"] = q5k_random_blocks(r5, 8)
    g["deq_q5k_y"] = ref.dequant(O.Q5_K, g["deq_q5k_w"], 8, 256)
    cases5 = {
        "q5k_rand": q5k_random_blocks(r5, rows * nb),
        "q5k_enc1": O.Oracle().encode(O.Q5_K, r5.standard_normal((rows, cols)).astype(np.float32)),
    }
    for name, w in cases5.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.Q5_K, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.Q5_K, w, X4, rows, cols)

    # Q3_K, likewise: its dequant and matMulVecBatchQ3K_Q8K_AVX2
    # (SIMDMatMulVecAVX2.cpp:3220) on random blocks and on this build's encoder
    # output. Own generator.
    r3 = np.random.default_rng(20261203)
    g["deq_q3k_w"] = q3k_random_blocks(r3, 8)
    g["deq_q3k_y"] = ref.dequant(O.Q3_K, g["deq_q3k_w"], 8, 256)
    cases3 = {
        "q3k_rand": q3k_random_blocks(r3, rows * nb),
        "q3k_enc002": O.Oracle().encode(O.Q3_K, (r3.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in cases3.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.Q3_K, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.Q3_K, w, X4, rows, cols)

    # IQ3_S, likewise (scalar fused Q8_K path, GGMLDequantize.hpp:2102), and
    # the digest of the reference codebook the committed table must match.
    ri = np.random.default_rng(20261204)
    grid = np.zeros(512, np.uint32)
    ref.lib.ref_iq3s_grid(ctypes.c_void_p(grid.ctypes.data))
    g["iq3s_grid_sha256"] = np.frombuffer(hashlib.sha256(grid.tobytes()).digest(), np.uint8)
    g["deq_iq3s_w"] = iq3s_random_blocks(ri, 8)
    g["deq_iq3s_y"] = ref.dequant(O.IQ3_S, g["deq_iq3s_w"], 8, 256)
    casesi = {
        "iq3s_rand": iq3s_random_blocks(ri, rows * nb),
        "iq3s_enc002": O.Oracle().encode(O.IQ3_S, (ri.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in casesi.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.IQ3_S, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.IQ3_S, w, X4, rows, cols)

    # IQ2_S, likewise (row scale 0.125), and the codebook digest.
    r2 = np.random.default_rng(20261205)
    grid2 = np.zeros(1024, np.uint64)
    ref.lib.ref_iq2s_grid(ctypes.c_void_p(grid2.ctypes.data))
    g["iq2s_grid_sha256"] = np.frombuffer(hashlib.sha256(grid2.tobytes()).digest(), np.uint8)
    g["deq_iq2s_w"] = iq2s_random_blocks(r2, 8)
    g["deq_iq2s_y"] = ref.dequant(O.IQ2_S, g["deq_iq2s_w"], 8, 256)
    cases2 = {
        "iq2s_rand": iq2s_random_blocks(r2, rows * nb),
        "iq2s_enc002": O.Oracle().encode(O.IQ2_S, (r2.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in cases2.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.IQ2_S, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.IQ2_S, w, X4, rows, cols)

    # Q2_K, likewise: its dequant and the compact-block kernel
    # matMulVecBatchQ2K_Compact_Q8K_AVX2 (SIMDMatMulVecAVX2.cpp:4757).
    rq = np.random.default_rng(20261206)
    g["deq_q2k_w"] = q2k_random_blocks(rq, 8)
    g["deq_q2k_y"] = ref.dequant(O.Q2_K, g["deq_q2k_w"], 8, 256)
    casesq = {
        "q2k_rand": q2k_random_blocks(rq, rows * nb),
        "q2k_enc002": O.Oracle().encode(O.Q2_K, (rq.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in casesq.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.Q2_K, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.Q2_K, w, X4, rows, cols)

    # IQ2_XS, likewise (float path: unquantized x, double sums), and the
    # codebook digest.
    rx = np.random.default_rng(20261207)
    gridx = np.zeros(512, np.uint64)
    ref.lib.ref_iq2xs_grid(ctypes.c_void_p(gridx.ctypes.data))
    g["iq2xs_grid_sha256"] = np.frombuffer(hashlib.sha256(gridx.tobytes()).digest(), np.uint8)
    g["deq_iq2xs_w"] = iq2xs_random_blocks(rx, 8)
    g["deq_iq2xs_y"] = ref.dequant(O.IQ2_XS, g["deq_iq2xs_w"], 8, 256)
    casesx = {
        "iq2xs_rand": iq2xs_random_blocks(rx, rows * nb),
        "iq2xs_enc002": O.Oracle().encode(O.IQ2_XS, (rx.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in casesx.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.IQ2_XS, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.IQ2_XS, w, X4, rows, cols)

    # IQ4_XS, likewise: its dequant and the Q8_K kernel
    # matMulVecBatchIQ4XS_Q8K_AVX2 (SIMDMatMulVecAVX2.cpp:3988).
    r4 = np.random.default_rng(20261208)
    g["deq_iq4xs_w"] = iq4xs_random_blocks(r4, 8)
    g["deq_iq4xs_y"] = ref.dequant(O.IQ4_XS, g["deq_iq4xs_w"], 8, 256)
    cases4 = {
        "iq4xs_rand": iq4xs_random_blocks(r4, rows * nb),
        "iq4xs_enc002": O.Oracle().encode(O.IQ4_XS, (r4.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in cases4.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.IQ4_XS, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.IQ4_XS, w, X4, rows, cols)

    # IQ4_NL, likewise: its dequant and the fp32-x kernel
    # matMulVecBatchIQ4NL_Q8K_AVX2 (SIMDMatMulVecAVX2.cpp:4126).
    rn = np.random.default_rng(20261209)
    g["deq_iq4nl_w"] = iq4nl_random_blocks(rn, 16)
    g["deq_iq4nl_y"] = ref.dequant(O.IQ4_NL, g["deq_iq4nl_w"], 2, 256)
    casesn = {
        "iq4nl_rand": iq4nl_random_blocks(rn, rows * cols // 32),
        "iq4nl_enc002": O.Oracle().encode(O.IQ4_NL, (rn.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in casesn.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.IQ4_NL, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.IQ4_NL, w, X4, rows, cols)

    # Q5_0, likewise: its dequant and the float fused path around the
    # reference's block dot dotProductQ5_0 (GGMLDequantize.hpp:1820).
    r5 = np.random.default_rng(20261210)
    g["deq_q50_w"] = q50_random_blocks(r5, 16)
    g["deq_q50_y"] = ref.dequant(O.Q5_0, g["deq_q50_w"], 2, 256)
    cases5 = {
        "q50_rand": q50_random_blocks(r5, rows * cols // 32),
        "q50_enc002": O.Oracle().encode(O.Q5_0, (r5.standard_normal((rows, cols)) * 0.02).astype(np.float32)),
    }
    for name, w in cases5.items():
        g[f"mm_{name}_w"] = w
        g[f"mm_{name}_y1"] = ref.matmul(O.Q5_0, w, X1, rows, cols)
        g[f"mm_{name}_y4"] = ref.matmul(O.Q5_0, w, X4, rows, cols)

    # Mat-vec at the BASELINE widths (configs 1-4): 8 rows, S = 1 and 4 tokens
    # (the one-token input is the first row of the four), so the reference's
    # fp32 cross-block accumulation order is pinned at 14, 20, 68 and 74
    # superblocks (Q8_0: 128, 160 and 544 blocks), not only at 2.
    rw = np.random.default_rng(20261202)
    oc = O.Oracle()
    for cols in WIDE_COLS:
        g[f"mmw_x4_{cols}"] = rw.standard_normal((4, cols)).astype(np.float32)
    for name, qt, colsl in WIDE_CASES:
        for cols in colsl:
            nb = cols // 256
            if qt == O.Q4_K:
                w = ref.encode_q4k(rw.standard_normal((8, cols)).astype(np.float32))
            elif qt == O.Q6_K:
                w = q6k_random_blocks(rw, 8 * nb)
            elif qt == O.IQ3_XXS:
                w = iq3_random_blocks(rw, 8 * nb)
            else:
                w = oc.encode(O.Q8_0, (rw.standard_normal((8, cols)) * 0.02).astype(np.float32))
            x4 = g[f"mmw_x4_{cols}"]
            g[f"mmw_{name}_{cols}_w"] = w
            g[f"mmw_{name}_{cols}_y1"] = ref.matmul(qt, w, x4[:1], 8, cols)
            g[f"mmw_{name}_{cols}_y4"] = ref.matmul(qt, w, x4, 8, cols)

    # MoE router (ModelMoE.cpp:341-425): logits from the reference's F32
    # kernel (SIMDMatMulVecAVX2.cpp:2982) at a width with a 4-column tail, for
    # one token (row path) and sixteen (tile path); the selection on those
    # logits and on tie-heavy logits (multiples of 1/4: equal probabilities
    # whose order std::partial_sort fixes), for k = 1, 8 and 10.
    rr = np.random.default_rng(20261203)
    E, H = 128, 516
    wr = (rr.standard_normal((E, H)) * 0.05).astype(np.float32)
    xr = rr.standard_normal((16, H)).astype(np.float32)
    g["router_w"], g["router_x"] = wr, xr
    g["router_logits1"] = ref.matmul_f32(wr, xr[:1], E, H)
    g["router_logits16"] = ref.matmul_f32(wr, xr, E, H)
    ties = (np.round(rr.standard_normal((32, E)) * 2.0) / 4.0).astype(np.float32)
    wide = (rr.standard_normal((8, 256)) * 3.0).astype(np.float32)
    g["router_ties"], g["router_wide"] = ties, wide
    for k in (1, 8, 10):
        g[f"router_sel{k}_ids"], g[f"router_sel{k}_wts"] = ref.moe_select(g["router_logits16"], k)
        g[f"router_ties{k}_ids"], g[f"router_ties{k}_wts"] = ref.moe_select(ties, k)
    g["router_wide8_ids"], g["router_wide8_wts"] = ref.moe_select(wide, 8)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(g)} arrays")


if __name__ == "__main__":
    main()
