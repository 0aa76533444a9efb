"""CPU tests: pin the C restatement (oracle/oracle.c) before it is trusted.

Three kinds of check, chosen so that a plausible slip (dropped term, wrong
sign, transposed index, wrong nibble) fails at least one of them:
  * golden vectors written by the COMPILED REFERENCE (tests/golden), bit-exact;
  * identities the mathematics fixes (integer dot = dequant-integer dot, closed
    forms on hand-built blocks, quantizer invariants, unit probes);
  * the reference's own test thresholds (Q4_K round-trip, IQ3_XXS e0 probe).
"""
import hashlib
import os
import sys

import numpy as np
import pytest

import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
from gen_golden import moe_weights  # noqa: E402


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---- fp16 ---------------------------------------------------------------------

def test_half_to_float_matches_reference_table(oracle, golden):
    tab = np.array([oracle.half_to_float(h) for h in range(65536)], np.float32)
    assert hashlib.sha256(tab.tobytes()).digest() == golden["h2f_sha256"].tobytes()
    assert (bits(tab[golden["h2f_sample_idx"]]) == bits(golden["h2f_sample"])).all()


def test_half_to_float_closed_forms(oracle):
    # IEEE binary16 values fixed by the standard.
    assert oracle.half_to_float(0x3C00) == 1.0
    assert oracle.half_to_float(0xC000) == -2.0
    assert oracle.half_to_float(0x0001) == 2.0 ** -24
    assert oracle.half_to_float(0x03FF) == 1023 * 2.0 ** -24
    assert oracle.half_to_float(0x7BFF) == 65504.0
    assert np.isinf(oracle.half_to_float(0x7C00))
    assert np.isnan(oracle.half_to_float(0x7E00))
    # numpy's own widening agrees on every pattern that is not NaN.
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    ours = np.array([oracle.half_to_float(v) for v in range(0, 65536, 7)], np.float32)
    sel = ref[::7]
    ok = np.isnan(sel) | (bits(ours) == bits(sel))
    assert ok.all()


def test_float_to_half_matches_reference(oracle, golden):
    got = np.array([oracle.float_to_half(float(f)) for f in golden["f2h_in"]], np.uint16)
    assert (got == golden["f2h_out"]).all()


def test_float_to_half_truncates_and_flushes_like_reference(oracle):
    # Truncation (no rounding): 1 + 2^-11 + 2^-12 stays 1.0 in fp16.
    assert oracle.float_to_half(1.0 + 2.0 ** -11 + 2.0 ** -12) == 0x3C00
    # The reference's subnormal branch also takes exponent -14: values below
    # 2^-13 come out as (signed) zero.
    assert oracle.float_to_half(1.5 * 2.0 ** -14) == 0
    assert oracle.float_to_half(2.0 ** -13) == 0x0800


# ---- activation quantizers -------------------------------------------------------

def test_quantize_q8k_matches_reference(oracle, golden):
    for i, x in enumerate(golden["q8k_x"]):
        qs, d, bs = oracle.quantize_q8k(x)
        assert (qs == golden["q8k_qs"][i]).all()
        assert (bits(d) == bits(golden["q8k_d"][i])).all()
        assert (bs == golden["q8k_bsums"][i]).all()


def test_quantize_q8k_invariants(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(2048).astype(np.float32)
    qs, d, bs = oracle.quantize_q8k(x)
    xb = x.reshape(-1, 256)
    for b in range(8):
        i = int(np.argmax(np.abs(xb[b])))   # first index of the max |x|
        assert qs[256 * b + i] == -127       # iscale = -127/max maps max to -127
        assert d[b] == np.float32(1.0) / (np.float32(-127.0) / xb[b, i])
    assert (np.abs(qs.astype(int)) <= 127).all()
    assert (bs == qs.reshape(-1, 16).astype(np.int32).sum(1)).all()
    # Reconstruction error is at most half a step per element.
    rec = qs.reshape(-1, 256) * d[:, None]
    assert (np.abs(rec - xb) <= np.abs(d[:, None]) * 0.5 + 1e-7).all()


def test_quantize_q8_0_act_pinned_by_reference_probe(oracle, golden):
    # out[i] = d8 * xq[i] through the reference's own Q8_0 kernel (unit weights).
    x = golden["probe_q80_x"]
    for s in range(x.shape[0]):
        qs, d = oracle.quantize_q8_0_act(x[s])
        expect = np.repeat(d, 32) * qs.astype(np.float32)
        # the kernel multiplies (1.0 * d8) and then the int product; the sum over
        # 8 lanes has one nonzero lane, so the result is exact (the kernel's +0
        # accumulator turns a -0 product into +0, hence value equality).
        assert np.array_equal(expect, golden["probe_q80_y"][s])


# ---- block decoders ---------------------------------------------------------------

@pytest.mark.parametrize("name,qt", [("q2k", O.Q2_K), ("q3k", O.Q3_K), ("q4k", O.Q4_K), ("q5k", O.Q5_K), ("q6k", O.Q6_K), ("iq3", O.IQ3_XXS),
                                     ("iq3s", O.IQ3_S), ("iq2s", O.IQ2_S), ("iq2xs", O.IQ2_XS), ("iq4xs", O.IQ4_XS), ("iq4nl", O.IQ4_NL), ("q50", O.Q5_0),
                                     ("q80", O.Q8_0)])
def test_dequant_matches_reference(oracle, golden, name, qt):
    w = golden[f"deq_{name}_w"]
    y = golden[f"deq_{name}_y"]
    got = oracle.dequant(qt, w, y.shape[0], y.shape[1])
    assert (bits(got) == bits(y)).all()


def test_q4k_dequant_closed_form(oracle):
    # d = 1, dmin = 0.5, sub-block j scale j+1 (j<4) / 10+j (j>=4), mins 2j.
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    sc = [1, 2, 3, 4, 14, 15, 16, 17]
    mn = [0, 2, 4, 6, 8, 10, 12, 60]
    for j in range(4):
        blk[4 + j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = mn[j] | ((mn[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    q = np.arange(256) % 16
    for g in range(8):
        for i in range(32):
            blk[16 + 32 * (g // 2) + i] |= q[32 * g + i] << (4 * (g % 2))
    y = oracle.dequant(O.Q4_K, blk, 1, 256)[0]
    for g in range(8):
        expect = sc[g] * q[32 * g:32 * g + 32] - 0.5 * mn[g]
        assert np.array_equal(y[32 * g:32 * g + 32], expect.astype(np.float32))


def test_iq3_dequant_closed_form(oracle):
    # grid entry 0 = (4,4,4,4), entry 255 last; ls = 3 -> db = d*3.5*0.5.
    grid = np.array([int(v, 16) for v in open(os.path.join(os.path.dirname(O.__file__),
                                                           "iq3xxs_grid.inc")).read()
                     .split("*/")[1].replace(",", " ").split()], np.uint32)
    blk = np.zeros(98, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    blk[2:66] = np.arange(64, dtype=np.uint8) * 3
    aux = (3 << 28) | (0b0000011 << 0) | (0b1000000 << 7)  # signs per 8-group
    for c in range(8):
        blk[66 + 4 * c:70 + 4 * c] = np.frombuffer(np.uint32(aux).tobytes(), np.uint8)
    y = oracle.dequant(O.IQ3_XXS, blk, 1, 256)[0]
    db = 2.0 * 3.5 * 0.5
    for c in range(8):
        for l in range(4):
            idx7 = (aux >> (7 * l)) & 127
            sgn = idx7 | ((bin(idx7).count("1") & 1) << 7)
            for j in range(8):
                g = int(blk[2 + 8 * c + 2 * l + j // 4])
                mag = (int(grid[g]) >> (8 * (j % 4))) & 255
                v = db * mag * (-1 if (sgn >> j) & 1 else 1)
                assert y[32 * c + 8 * l + j] == np.float32(v)


# ---- per-block integer dots: brute-force identity ------------------------------------

@pytest.mark.parametrize("qt", [O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ3_XXS, O.IQ3_S, O.IQ2_S,
                                O.IQ4_XS])
def test_block_isums_identity(oracle, qt):
    """sum over blocks of the integer sums, scaled per block by the float block
    scales, reproduces dequant(W) . (d8 * xq) in exact rational arithmetic."""
    rng = np.random.default_rng(11 + qt)
    rows, cols = 6, 512
    if qt == O.Q8_0:
        from gen_golden import q80_random_blocks as gen
        w = gen(rng, rows * cols // 32)
    elif qt == O.Q4_K:
        from gen_golden import q4k_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.Q5_K:
        from gen_golden import q5k_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.Q6_K:
        from gen_golden import q6k_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.Q3_K:
        from gen_golden import q3k_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.Q2_K:
        from gen_golden import q2k_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.IQ3_S:
        from gen_golden import iq3s_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.IQ2_S:
        from gen_golden import iq2s_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    elif qt == O.IQ4_XS:
        from gen_golden import iq4xs_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    else:
        from gen_golden import iq3_random_blocks as gen
        w = gen(rng, rows * cols // 256)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    isums = oracle.block_isums(qt, w, x, rows, cols)[0]
    deq = oracle.dequant(qt, w, rows, cols).astype(np.float64)
    if qt == O.Q8_0:
        qs, d8 = oracle.quantize_q8_0_act(x[0])
        xq = qs.astype(np.float64)
        wb = w.reshape(rows, cols // 32, 34)
        d = wb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
        # deq = d * q exactly, so sum(deq*xq) over a block = d * isum exactly
        lhs = (deq * xq).reshape(rows, -1, 32).sum(2)
        assert np.array_equal(lhs, d * isums[:, :, 0])
    elif qt == O.Q4_K:
        qs, d8, _ = oracle.quantize_q8k(x[0])
        wb = w.reshape(rows, cols // 256, 144)
        nib = np.zeros((rows, cols // 256, 256), np.int64)
        for g in range(8):
            byt = wb[:, :, 16 + 32 * (g // 2):16 + 32 * (g // 2) + 32].astype(np.int64)
            nib[:, :, 32 * g:32 * g + 32] = (byt >> 4) if g % 2 else (byt & 15)
        expect = (nib * qs.reshape(1, -1, 256)).reshape(rows, -1, 8, 32).sum(3)
        assert np.array_equal(expect, isums)
    elif qt == O.Q2_K:
        # 2-bit values and 4-bit scale/min nibbles from the block bytes (layout
        # pinned by the reference dequant golden): main = sum sc*sum q*x,
        # min = sum m*bsum; and dequant = d*main-part - dmin*min-part exactly
        qs, d8, bs = oracle.quantize_q8k(x[0])
        wb = w.reshape(rows, cols // 256, 84).astype(np.int64)
        q2 = np.zeros((rows, cols // 256, 256), np.int64)
        for e in range(256):
            h, t, l = e // 128, (e // 32) % 4, e % 32
            q2[:, :, e] = (wb[:, :, 16 + 32 * h + l] >> (2 * t)) & 3
        sc, mn = wb[:, :, :16] & 15, wb[:, :, :16] >> 4
        grp = (q2 * qs.reshape(1, -1, 256)).reshape(rows, -1, 16, 16).sum(3)
        assert np.array_equal((sc * grp).sum(2), isums[:, :, 0])
        assert np.array_equal((mn * bs.reshape(1, -1, 16)).sum(2), isums[:, :, 1])
    elif qt == O.Q5_K:
        # 5-bit values from the block bytes (layout pinned by the reference
        # dequant golden): qs at 48, qh at 16, sub-block g = 2c + h
        qs, d8, _ = oracle.quantize_q8k(x[0])
        wb = w.reshape(rows, cols // 256, 176).astype(np.int64)
        q5 = np.zeros((rows, cols // 256, 256), np.int64)
        for g in range(8):
            c, h = g // 2, g % 2
            low = (wb[:, :, 48 + 32 * c:48 + 32 * c + 32] >> (4 * h)) & 15
            high = (wb[:, :, 16:48] >> (2 * c + h)) & 1
            q5[:, :, 32 * g:32 * g + 32] = low | (high << 4)
        expect = (q5 * qs.reshape(1, -1, 256)).reshape(rows, -1, 8, 32).sum(3)
        assert np.array_equal(expect, isums)
    else:
        # Q3_K / Q6_K / IQ3_XXS: dequant = c_block * (per-group integer scale * int weight),
        # so the integer sum equals sum(deq * xq) / c_block exactly (powers of two
        # or exact small-integer products in double).
        qs, d8, _ = oracle.quantize_q8k(x[0])
        xq = qs.astype(np.float64).reshape(1, -1, 256)
        if qt in (O.Q3_K, O.Q6_K):
            tb, do = (110, 108) if qt == O.Q3_K else (210, 208)
            wb = w.reshape(rows, cols // 256, tb)
            c = wb[:, :, do:do + 2].copy().view(np.float16).astype(np.float64)[:, :, 0]
            lhs = (deq.reshape(rows, -1, 256) * xq).sum(2) / c
        elif qt == O.IQ3_S:
            wb = w.reshape(rows, cols // 256, 110)
            c = wb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
            # db = d*(1+2ls)
            lhs = (deq.reshape(rows, -1, 256) * xq).sum(2) / c
        elif qt == O.IQ4_XS:
            # dequant = d * (ls-32) * kvalue (11 + 6 + 7 significant bits: exact
            # in fp32), so sum(deq * xq) / d is the integer sum exactly
            wb = w.reshape(rows, cols // 256, 136)
            c = wb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
            lhs = (deq.reshape(rows, -1, 256) * xq).sum(2) / c
        elif qt == O.IQ2_S:
            wb = w.reshape(rows, cols // 256, 82)
            c = wb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
            # db = d*(0.5+ls)*0.25 = d*(1+2ls)/8
            lhs = (deq.reshape(rows, -1, 256) * xq).sum(2) / c * 8.0
        else:
            wb = w.reshape(rows, cols // 256, 98)
            c = wb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
            # db = d*(0.5+ls)*0.5 = d*(2ls+1)/4
            lhs = (deq.reshape(rows, -1, 256) * xq).sum(2) / c * 4.0
        assert np.array_equal(lhs, isums[:, :, 0].astype(np.float64))


# ---- mat-vec kernels -----------------------------------------------------------------

MM = [("q4k_rand", O.Q4_K), ("q4k_enc1", O.Q4_K), ("q4k_enc002", O.Q4_K), ("q5k_rand", O.Q5_K),
      ("q5k_enc1", O.Q5_K), ("q3k_rand", O.Q3_K), ("q3k_enc002", O.Q3_K), ("q2k_rand", O.Q2_K),
      ("q2k_enc002", O.Q2_K), ("iq3s_rand", O.IQ3_S),
      ("iq3s_enc002", O.IQ3_S), ("iq2s_rand", O.IQ2_S), ("iq2s_enc002", O.IQ2_S),
      ("iq2xs_rand", O.IQ2_XS), ("iq2xs_enc002", O.IQ2_XS), ("iq4xs_rand", O.IQ4_XS),
      ("iq4xs_enc002", O.IQ4_XS), ("iq4nl_rand", O.IQ4_NL), ("iq4nl_enc002", O.IQ4_NL),
      ("q50_rand", O.Q5_0), ("q50_enc002", O.Q5_0), ("q6k_rand", O.Q6_K), ("iq3_rand", O.IQ3_XXS), ("q80_rand", O.Q8_0)]


@pytest.mark.parametrize("name,qt", MM)
def test_matmul_bit_exact_vs_reference(oracle, golden, name, qt):
    w = golden[f"mm_{name}_w"]
    for tag in ("1", "4"):
        x = golden[f"mm_x{tag}"]
        y = golden[f"mm_{name}_y{tag}"]
        got = oracle.matmul(qt, w, x, y.shape[1], x.shape[1])
        assert (bits(got) == bits(y)).all(), (name, tag)


WIDE = [("q4k", O.Q4_K, c) for c in (3584, 5120, 17408, 18944)] + \
       [("q6k", O.Q6_K, c) for c in (3584, 17408, 18944)] + \
       [("iq3", O.IQ3_XXS, c) for c in (3584, 17408, 18944)] + [("q80", O.Q8_0, c) for c in (4096, 5120, 17408)]


@pytest.mark.parametrize("name,qt,cols", WIDE)
def test_matmul_bit_exact_vs_reference_at_baseline_widths(oracle, golden, name, qt, cols):
    """At the BASELINE widths (14-74 superblocks, 128-544 Q8_0 blocks) the
    oracle's fp32 cross-block accumulation matches the compiled reference bit
    for bit, for the one-token row path and the 4-token batch path."""
    w = golden[f"mmw_{name}_{cols}_w"]
    x4 = golden[f"mmw_x4_{cols}"]
    for tag, x in (("1", x4[:1]), ("4", x4)):
        y = golden[f"mmw_{name}_{cols}_y{tag}"]
        got = oracle.matmul(qt, w, x, 8, cols)
        assert (bits(got) == bits(y)).all(), (name, cols, tag)


def test_matmul_q80_cols96(oracle, golden):
    got = oracle.matmul(O.Q8_0, golden["mm_q80c96_w"], golden["mm_q80c96_x"], 16, 96)
    assert (bits(got) == bits(golden["mm_q80c96_y"])).all()


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ3_XXS, O.IQ3_S, O.IQ2_S,
                                O.IQ2_XS, O.IQ4_XS, O.IQ4_NL, O.Q5_0])
def test_matmul_close_to_float_dot(oracle, qt):
    """Independent of the reference: the quantized mat-vec approximates the
    float product of the dequantized weights with x (activation quantization
    error only, < 2% of the output scale)."""
    rng = np.random.default_rng(3)
    rows, cols = 32, 1024
    if qt == O.Q4_K:
        w = oracle.encode(qt, rng.standard_normal((rows, cols)).astype(np.float32))
    else:
        w = oracle.encode(qt, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    x = rng.standard_normal((2, cols)).astype(np.float32)
    y = oracle.matmul(qt, w, x, rows, cols)
    deq = oracle.dequant(qt, w, rows, cols)
    ref = x.astype(np.float64) @ deq.T.astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(y - ref).max() < 0.02 * scale


def test_iq3_e0_probe_reference_test(oracle, golden):
    """unit_tests/DequantizeTest.cpp:1216-1270: with x = e0 the fused result
    equals the first dequantized weight of each row within 1e-3."""
    for c in (1536, 2048, 3584):
        w = golden[f"iq3probe_{c}_w"]
        e0 = np.zeros((1, c), np.float32)
        e0[0, 0] = 1.0
        got = oracle.matmul(O.IQ3_XXS, w, e0, 8, c)
        assert (bits(got) == bits(golden[f"iq3probe_{c}_y"])).all()
        deq = oracle.dequant(O.IQ3_XXS, w, 8, c)
        assert np.abs(got[0] - deq[:, 0]).max() < 1e-3


# ---- encoders --------------------------------------------------------------------------

def test_q4k_encoder_matches_reference(oracle, golden):
    got = oracle.encode(O.Q4_K, golden["enc_q4k_x"])
    assert (got.reshape(-1, 144) == golden["enc_q4k_out"]).all()


def test_q4k_encoder_reference_roundtrip_thresholds(oracle):
    """unit_tests/DequantizeTest.cpp:1280-1340: ramp within 0.02, gaussian
    blocks with per-group spread at mean relRms < 9%."""
    ramp = (np.arange(256) % 16 - 7.5).astype(np.float32)[None]
    y = oracle.dequant(O.Q4_K, oracle.encode(O.Q4_K, ramp), 1, 256)
    assert np.abs(y - ramp).max() < 0.02
    rng = np.random.default_rng(20261116)
    xs = []
    for _ in range(256):
        s = rng.uniform(0.5, 2.0, 8)
        off = 0.15 * s * rng.standard_normal(8)
        xs.append((off[:, None] + s[:, None] * rng.standard_normal((8, 32))).ravel())
    x = np.array(xs, np.float32)
    y = oracle.dequant(O.Q4_K, oracle.encode(O.Q4_K, x.reshape(-1, 256)), 256, 256)
    rel = np.sqrt(((y - x) ** 2).sum(1) / (x ** 2).sum(1))
    assert rel.mean() < 0.09


@pytest.mark.parametrize("qt,bound", [(O.Q8_0, 0.01), (O.Q2_K, 0.45), (O.Q3_K, 0.2), (O.Q5_K, 0.08), (O.Q6_K, 0.04),
                                      (O.IQ3_XXS, 0.25), (O.IQ3_S, 0.2), (O.IQ2_S, 0.35),
                                      (O.IQ2_XS, 0.4), (O.IQ4_XS, 0.1), (O.IQ4_NL, 0.1), (O.Q5_0, 0.06)])
def test_own_encoders_roundtrip(oracle, qt, bound):
    """This build's Q8_0 / Q2_K / Q3_K / Q5_K / Q6_K / IQ3_XXS / IQ3_S / IQ2_S / IQ2_XS / IQ4_XS / IQ4_NL / Q5_0 encoders (the reference has none):
    N(0, 0.02) rows round-trip within the format's expected relative RMS."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    y = oracle.dequant(qt, oracle.encode(qt, x), 16, 1024)
    rel = np.sqrt(((y - x) ** 2).sum() / (x ** 2).sum())
    assert rel < bound


def test_iq3_encoder_sign_parity(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    w = oracle.encode(O.IQ3_XXS, x).reshape(4, 98)
    y = oracle.dequant(O.IQ3_XXS, w.ravel(), 4, 256)
    # every 8-group carries an even number of negatives (format rule)
    neg = (y < 0).reshape(4, 32, 8).sum(2)
    assert (neg % 2 == 0).all()


def test_iq3s_grid_tables_match_reference(golden):
    """The committed IQ3_S codebook (oracle/ and the kernels' copy) is the
    reference table (digest written from the compiled reference)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for path in ("oracle/iq3s_grid.inc", "tinycoder-inference_amd/csrc/iq3s_grid.inc"):
        text = open(os.path.join(root, path)).read()
        vals = [int(t, 16) for t in __import__("re").findall(r"0x[0-9a-f]{8}", text)]
        assert len(vals) == 512
        digest = hashlib.sha256(np.array(vals, np.uint32).tobytes()).digest()
        assert digest == golden["iq3s_grid_sha256"].tobytes(), path
        # format facts: odd magnitudes 1..15 in every byte
        b = np.array(vals, np.uint32).view(np.uint8)
        assert ((b % 2 == 1) & (b <= 15)).all()


def test_iq2xs_float_path_and_grid(oracle, golden):
    """IQ2_XS: no integer sums (the reference's CPU path dots unquantized x);
    its codebook tables match the reference digest; every 8-group of an
    encoded block has an even number of negative weights (format rule)."""
    w = golden["mm_iq2xs_rand_w"]
    with pytest.raises(AssertionError):
        oracle.block_isums(O.IQ2_XS, w, golden["mm_x1"], len(w) // 74 // (golden["mm_x1"].shape[1] // 256),
                           golden["mm_x1"].shape[1])
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for path in ("oracle/iq2xs_grid.inc", "tinycoder-inference_amd/csrc/iq2xs_grid.inc"):
        text = open(os.path.join(root, path)).read()
        arr = np.array([int(t, 16) for t in __import__("re").findall(r"0x([0-9a-f]{16})ull", text)], np.uint64)
        assert len(arr) == 512
        assert hashlib.sha256(arr.tobytes()).digest() == golden["iq2xs_grid_sha256"].tobytes(), path
    x = np.random.default_rng(4).standard_normal((4, 256)).astype(np.float32)
    y = oracle.dequant(O.IQ2_XS, oracle.encode(O.IQ2_XS, x), 4, 256)
    assert ((y < 0).reshape(4, 32, 8).sum(2) % 2 == 0).all()


def test_iq2s_grid_tables_match_reference(golden):
    """The committed IQ2_S codebook (oracle/ and the kernels' copy) is the
    reference table; every byte is one of the format's magnitudes 8, 25, 43."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for path in ("oracle/iq2s_grid.inc", "tinycoder-inference_amd/csrc/iq2s_grid.inc"):
        text = open(os.path.join(root, path)).read()
        vals = [int(t, 16) for t in __import__("re").findall(r"0x([0-9a-f]{16})ull", text)]
        assert len(vals) == 1024
        arr = np.array(vals, np.uint64)
        assert hashlib.sha256(arr.tobytes()).digest() == golden["iq2s_grid_sha256"].tobytes(), path
        assert np.isin(arr.view(np.uint8), [8, 25, 43]).all()


# ---- MoE ------------------------------------------------------------------------------

def test_moe_matches_reference_composition(oracle, golden):
    E, K, H, FF, S, seed = [int(v) for v in golden["moe_dims"]]
    wg, wu, wd = moe_weights(lambda x: oracle.encode(O.Q4_K, x), E, H, FF, seed)
    digest = hashlib.sha256(wg.tobytes() + wu.tobytes() + wd.tobytes()).digest()
    assert digest == golden["moe_wsha256"].tobytes()
    got = oracle.moe_ffn(golden["moe_x"], golden["moe_ids"], golden["moe_wts"], wg, wu, wd, E, H, FF)
    ref = golden["moe_y"]
    assert np.allclose(got, ref, rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("name,qt,tb", [("iq4nl", O.IQ4_NL, 18), ("q50", O.Q5_0, 22)])
def test_float_path_types(oracle, golden, name, qt, tb):
    """IQ4_NL and Q5_0: no integer sums (the reference's CPU paths dot fp32
    x); the mat-vec is linear in x (exact for x scaled by a power of two)."""
    w = golden[f"mm_{name}_rand_w"]
    x = golden["mm_x1"]
    cols = x.shape[1]
    rows = len(w) // tb // (cols // 32)
    with pytest.raises(AssertionError):
        oracle.block_isums(qt, w, x, rows, cols)
    y = oracle.matmul(qt, w, x, rows, cols)
    assert (bits(oracle.matmul(qt, w, 4.0 * x, rows, cols)) == bits(4.0 * y)).all()


# ---- MoE router ------------------------------------------------------------------------

def test_router_logits_bit_exact_vs_reference(oracle, golden):
    """The F32 router mat-vec (SIMDMatMulVecAVX2.cpp:2982) in the reference's
    FMA-chain order, with a 4-column tail, for 1 and 16 tokens."""
    w, x = golden["router_w"], golden["router_x"]
    E, H = w.shape
    for tag, xs in (("1", x[:1]), ("16", x)):
        got = oracle.matmul_f32(w, xs, E, H)
        assert (bits(got) == bits(golden[f"router_logits{tag}"])).all(), tag


def test_router_logits_close_to_float64_dot(oracle):
    """What the mathematics fixes: the logits are the dot products up to fp32
    rounding (a dropped column or chain would fail this)."""
    rng = np.random.default_rng(8)
    for H in (7, 40, 520, 2052):
        w = rng.standard_normal((16, H)).astype(np.float32)
        x = rng.standard_normal((3, H)).astype(np.float32)
        got = oracle.matmul_f32(w, x, 16, H).astype(np.float64)
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-4 * np.sqrt(H))


@pytest.mark.parametrize("k", [1, 8, 10])
def test_router_selection_bit_exact_vs_reference(oracle, golden, k):
    """Softmax, top-k (std::partial_sort's order, ties included) and the
    clamped renormalisation of ModelMoE.cpp:387-424: ids and weights bit for
    bit on random and tie-heavy logits."""
    cases = [("sel", golden["router_logits16"]), ("ties", golden["router_ties"])]
    if k == 8:
        cases.append(("wide", golden["router_wide"]))
    for name, lg in cases:
        ids, wts = oracle.moe_route(lg, k)
        assert (ids == golden[f"router_{name}{k}_ids"]).all(), name
        assert (bits(wts) == bits(golden[f"router_{name}{k}_wts"])).all(), name


def test_router_selection_invariants(oracle):
    """Without ties the selection is the k largest probabilities in
    descending order (brute force), the weights are the softmax restricted to
    them and renormalised (they sum to 1), and logits shifted by a constant
    select the same experts."""
    rng = np.random.default_rng(9)
    lg = (rng.standard_normal((64, 128)) * 3.0).astype(np.float32)
    ids, wts = oracle.moe_route(lg, 8)
    for s in range(64):
        p = np.exp(lg[s].astype(np.float64) - lg[s].max())
        p /= p.sum()
        order = np.argsort(-p, kind="stable")[:8]
        assert (ids[s] == order).all()
        assert np.allclose(wts[s], p[order] / p[order].sum(), rtol=1e-5)
        assert abs(float(wts[s].astype(np.float64).sum()) - 1.0) < 1e-5
    ids2, _ = oracle.moe_route(lg + np.float32(0.5), 8)
    assert (ids2 == ids).all()
