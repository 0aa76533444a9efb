"""GPU parity tests of the reference-named C++ interfaces, called with real
buffers through a compiled C++ driver (tests/cpp/iface_driver.cpp):
tinycoder::gpu::int8Gemv / int8Gemm / int8GemvDual* (include/tc_int8gemm.hpp,
the reference's include/Int8Gemm.hpp:42-107) on device buffers, and
tinycoder::matMulVecBatch*_SIMD (include/tc_simd_matmul.hpp, the reference's
include/SIMDMatMulVec.hpp:448-584) on host buffers.

Bar: fp32 outputs within 1e-3 relative / 1e-4 absolute of the oracle; a
refused call returns false and writes nothing.
"""
import ctypes

import numpy as np
import pytest

from qdata import IQ3_XXS, IQ4_NL, IQ4_XS, NAMES, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, close, gaussian, row_bytes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def drv(tc):
    import iface
    return iface.load()


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def H(a):
    return ctypes.c_void_p(a.ctypes.data)


def weights(oracle, qt, rng, rows, cols):
    return oracle.encode(qt, gaussian(rng, (rows, cols), 1.0 if qt == Q4_K else 0.02))


def test_available_and_preferred(drv):
    assert drv.drv_int8GemmAvailable() == 1
    for t in (Q8_0, Q4_K, Q6_K, IQ3_XXS):
        assert drv.drv_int8GemmPreferred(t, 4096, 4096) == 1
    assert drv.drv_int8GemmPreferred(99, 4096, 4096) == 0


@pytest.mark.parametrize("qt", [Q4_K, Q6_K, IQ3_XXS, Q8_0, Q5_K])
@pytest.mark.parametrize("S", [1, 3, 8])
def test_int8Gemv(drv, tc, dev, oracle, qt, S):
    import torch
    rng = np.random.default_rng(qt * 10 + S)
    rows, cols = 300, 3584
    w = weights(oracle, qt, rng, rows, cols)
    x = gaussian(rng, (S, cols))
    out = torch.full((S, rows), 7.0, device=dev)
    drv.drv_int8GemvReserve(cols, S)
    assert drv.drv_int8Gemv(qt, P(to_dev(w, dev)), P(to_dev(x, dev)), P(out), S, rows, cols, tc._stream()) == 1
    ok, worst = close(out.cpu().numpy(), oracle.matmul(qt, w, x, rows, cols))
    assert ok, f"{NAMES[qt]} S={S}: {worst:.3g}"


@pytest.mark.parametrize("qt", [Q4_K, Q8_0, Q6_K, IQ3_XXS])
def test_int8Gemm(drv, tc, dev, oracle, qt):
    import torch
    rng = np.random.default_rng(qt)
    M, rows, cols = 77, 200, 2048
    w = weights(oracle, qt, rng, rows, cols)
    x = gaussian(rng, (M, cols))
    out = torch.empty((M, rows), device=dev)
    bpr = cols // (32 if qt == Q8_0 else 256)
    assert drv.drv_int8Gemm(qt, P(to_dev(w, dev)), P(to_dev(x, dev)), P(out), M, rows, cols, bpr, tc._stream()) == 1
    ok, worst = close(out.cpu().numpy(), oracle.matmul(qt, w, x, rows, cols))
    assert ok, f"{NAMES[qt]}: {worst:.3g}"
    # blocksPerRow that does not match cols: refused, nothing written
    out2 = torch.full((M, rows), 7.0, device=dev)
    assert drv.drv_int8Gemm(qt, P(to_dev(w, dev)), P(to_dev(x, dev)), P(out2), M, rows, cols, bpr + 1,
                            tc._stream()) == 0
    assert (out2.cpu() == 7.0).all()


def test_int8Gemm_q8_disabled(drv, tc, dev, oracle):
    import torch
    rng = np.random.default_rng(5)
    w = weights(oracle, Q8_0, rng, 64, 512)
    x = gaussian(rng, (20, 512))
    out = torch.full((20, 64), 7.0, device=dev)
    drv.drv_int8GemmSetQ8Enabled(0)
    try:
        assert drv.drv_int8Gemm(Q8_0, P(to_dev(w, dev)), P(to_dev(x, dev)), P(out), 20, 64, 512, 16,
                                tc._stream()) == 0
    finally:
        drv.drv_int8GemmSetQ8Enabled(1)
    assert (out.cpu() == 7.0).all()


@pytest.mark.parametrize("which,qt", [(0, Q4_K), (1, IQ3_XXS)])
def test_int8GemvDual(drv, tc, dev, oracle, which, qt):
    import torch
    rng = np.random.default_rng(40 + which)
    rows, cols = 1000, 3584
    wg, wu = weights(oracle, qt, rng, rows, cols), weights(oracle, qt, rng, rows, cols)
    x = gaussian(rng, (1, cols))
    gout = torch.empty((1, rows), device=dev)
    uout = torch.empty((1, rows), device=dev)
    assert drv.drv_int8GemvDual(which, P(to_dev(wg, dev)), P(to_dev(wu, dev)), P(to_dev(x, dev)), P(gout),
                                P(uout), rows, cols, tc._stream()) == 1
    g = oracle.matmul(qt, wg, x, rows, cols).astype(np.float64)
    u = oracle.matmul(qt, wu, x, rows, cols)
    ok, worst = close(uout.cpu().numpy(), u)
    assert ok, worst
    ok, worst = close(gout.cpu().numpy(), g / (1 + np.exp(-g)) * u, 2e-3)
    assert ok, worst


SIMD_TYPES = [Q4_K, Q3_K, Q6_K, Q5_K, IQ4_XS, IQ4_NL, Q8_0, Q2_K]  # Q2_K: matMulVecBatchQ2K_Compact_SIMD


@pytest.mark.parametrize("qt", SIMD_TYPES)
@pytest.mark.parametrize("S", [1, 12])
def test_matMulVecBatch_SIMD_host_pointers(drv, tc, oracle, qt, S):
    """The CPU entry points' signatures on host buffers: decode (S = 1) and the
    prefill GEMM (S = 12), against the oracle."""
    rng = np.random.default_rng(qt + 100 * S)
    rows, cols = 257, 2048
    w = weights(oracle, qt, rng, rows, cols)
    x = gaussian(rng, (S, cols))
    out = np.full((S, rows), 7.0, np.float32)
    assert drv.drv_matMulVecBatch_SIMD(qt, H(w), H(x), S, rows, cols, H(out), None) == 1
    ok, worst = close(out, oracle.matmul(qt, w, x, rows, cols))
    assert ok, f"{NAMES[qt]} S={S}: {worst:.3g}"


@pytest.mark.parametrize("S", [1, 16])
def test_matMulVecBatchF32_SIMD_bits(drv, tc, oracle, S):
    """The router's F32 entry point on host buffers: the reference AVX2
    kernel's FMA order, so the oracle's bits (a width with a 4-column tail)."""
    rng = np.random.default_rng(50 + S)
    rows, cols = 128, 2052
    w = (rng.standard_normal((rows, cols)) * 0.03).astype(np.float32)
    x = rng.standard_normal((S, cols)).astype(np.float32)
    out = np.full((S, rows), 7.0, np.float32)
    assert drv.drv_matMulVecBatchF32_SIMD(H(w), H(x), S, rows, cols, H(out)) == 1
    ref = oracle.matmul_f32(w, x, rows, cols)
    assert (out.view(np.uint32) == np.ascontiguousarray(ref, np.float32).view(np.uint32)).all()


def test_matMulVecBatchQ3K_residual_and_registered_weights(drv, tc, oracle):
    """Q3_K's residual-fused store (out = W.x + residual), and a weight range
    registered once with tc_host_weights_register (read from its device copy,
    with the same result), then unregistered."""
    rng = np.random.default_rng(33)
    rows, cols, S = 300, 3584, 2
    w = weights(oracle, Q3_K, rng, rows, cols)
    x = gaussian(rng, (S, cols))
    res = gaussian(rng, (S, rows))
    ref = oracle.matmul(Q3_K, w, x, rows, cols) + res
    out = np.zeros((S, rows), np.float32)
    assert drv.drv_matMulVecBatch_SIMD(Q3_K, H(w), H(x), S, rows, cols, H(out), H(res)) == 1
    ok, worst = close(out, ref)
    assert ok, worst
    # out and residual the same buffer (the reference's attnO in-place residual,
    # SIMDMatMulVec.hpp:472-476): W.x + residual, the residual read before the
    # output overwrites it
    inplace = res.copy()
    assert drv.drv_matMulVecBatch_SIMD(Q3_K, H(w), H(x), S, rows, cols, H(inplace), H(inplace)) == 1
    ok, worst = close(inplace, ref)
    assert ok, worst
    assert tc.lib.tc_host_weights_register(H(w), w.nbytes) == 0
    try:
        rb = row_bytes(Q3_K, cols)
        # sub-ranges of the registered matrix: rows 100..199 (a 16-byte-aligned
        # start) and rows 1..100 (1540-byte rows: the device copy's address is
        # not 16-byte aligned, so the call stages the range instead)
        for r0, nr in ((100, 100), (1, 100)):
            wsub = w[r0 * rb:(r0 + nr) * rb]
            out3 = np.zeros((S, nr), np.float32)
            assert drv.drv_matMulVecBatch_SIMD(Q3_K, H(wsub), H(x), S, nr, cols, H(out3), None) == 1
            ok, worst = close(out3, (ref - res)[:, r0:r0 + nr])
            assert ok, (r0, worst)
        out2 = np.zeros((S, rows), np.float32)
        assert drv.drv_matMulVecBatch_SIMD(Q3_K, H(w), H(x), S, rows, cols, H(out2), None) == 1
        ok, worst = close(out2, ref - res)
        assert ok, worst
    finally:
        assert tc.lib.tc_host_weights_unregister(H(w)) == 0
    assert tc.lib.tc_host_weights_unregister(H(w)) != 0


def test_matMulVecBatch_SIMD_refuses(drv, tc):
    w = np.zeros(row_bytes(Q4_K, 512) * 2, np.uint8)
    x = np.zeros((1, 500), np.float32)
    out = np.full((1, 2), 7.0, np.float32)
    assert drv.drv_matMulVecBatch_SIMD(Q4_K, H(w), H(x), 1, 2, 500, H(out), None) == 0  # cols % 256
    assert drv.drv_matMulVecBatch_SIMD(99, H(w), H(x), 1, 2, 512, H(out), None) == 0
    assert (out == 7.0).all()
