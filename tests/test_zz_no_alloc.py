"""GPU test of tc_gemm_noalloc, the prefill GEMM entry point that allocates
nothing (its scratch is a fixed per-device array), through the C-ABI: two
calls in a row, the second with a smaller input, each against tc_gemm on the
same inputs (the same kernels on the same data: bit for bit), and a shape
beyond the fixed scratch refused without writing."""
import ctypes

import numpy as np
import pytest

from qdata import IQ2_S, IQ3_S, IQ3_XXS, Q4_K, Q5_K, Q6_K, Q8_0, gaussian

pytestmark = pytest.mark.gpu


def P(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, Q8_0])
def test_gemm_noalloc_matches_gemm(tc, dev, oracle, qt):
    import torch
    from tc_hip import TC_OK
    lib = tc.lib
    lib.tc_gemm_noalloc.restype = ctypes.c_int
    lib.tc_gemm_noalloc.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_uint32] * 4 + [ctypes.c_void_p]
    rng = np.random.default_rng(qt)
    bdiv = 32 if qt == Q8_0 else 256
    for M, N, K in ((300, 1000, 4096), (40, 136, 2048)):  # second call: smaller input
        w = oracle.encode(qt, gaussian(rng, (N, K), 1.0 if qt in (Q4_K, Q5_K) else 0.02))
        x = gaussian(rng, (M, K))
        wd, xd = torch.from_numpy(w).to(dev), torch.from_numpy(x).to(dev)
        ref = tc.gemm(qt, wd, xd, N, K)
        out = torch.full((M, N), 7.0, device=dev)
        rc = lib.tc_gemm_noalloc(qt, P(wd), P(xd), P(out), M, N, K, K // bdiv, tc._stream())
        assert rc == TC_OK, lib.tc_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"M={M} N={N} K={K}: max diff {(out - ref).abs().max().item()}"


def test_gemm_noalloc_refuses_beyond_scratch(tc, dev):
    import torch
    from tc_hip import TC_E_UNSUPPORTED
    lib = tc.lib
    lib.tc_gemm_noalloc.restype = ctypes.c_int
    lib.tc_gemm_noalloc.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_uint32] * 4 + [ctypes.c_void_p]
    lib.tc_gemm_noalloc_scratch_bytes.restype = ctypes.c_size_t
    cap = lib.tc_gemm_noalloc_scratch_bytes()
    M, K, N = 8192, 17408, 64  # ~143 MB of quantized activations
    assert M * K > cap
    w = torch.zeros(N * K // 256 * 144, dtype=torch.uint8, device=dev)
    x = torch.zeros((M, K), device=dev)
    out = torch.full((M, N), 7.0, device=dev)
    assert lib.tc_gemm_noalloc(Q4_K, P(w), P(x), P(out), M, N, K, K // 256, tc._stream()) == TC_E_UNSUPPORTED
    torch.cuda.synchronize()
    assert (out == 7.0).all()
