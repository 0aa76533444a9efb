"""GPU parity tests for the prefill GEMM (tc_gemm, int8 MFMA for Q4_K / Q5_K /
Q6_K / IQ3_XXS / IQ3_S / IQ2_S / Q8_0, the exact batched mat-vec path (IQ2_XS
on fp32 x) for Q2_K / Q3_K / IQ4_XS / IQ4_NL / Q5_0 / IQ2_XS), through the
C-ABI.

Bar: fp32 outputs within 1e-3 relative / 1e-4 absolute of the oracle (the C
restatement of the reference CPU kernels, itself bit-exact with the compiled
reference in tests/test_oracle.py). The activation quantizer the GEMM runs is
the one whose bytes are checked bit-exact in test_gpu_gemv.py.
"""
import numpy as np
import pytest

from qdata import ALL, IQ2_S, IQ2_XS, IQ4_NL, IQ4_XS, Q5_0, IQ3_S, IQ3_XXS, NAMES, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, close, gaussian, oracle_matmul_par, random_blocks, row_bytes, tile_edges

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def enc_weights(oracle, qt, rng, rows, cols):
    # Q4_K from N(0,1): at N(0,0.02) the reference quantizer stores most
    # scales as 0 (its fp16 conversion flushes values below 2^-13).
    return oracle.encode(qt, gaussian(rng, (rows, cols), 1.0 if qt in (Q4_K, Q5_K) else 0.02))


# (M tokens, N rows, K cols): ragged tiles, a K-split case (few output tiles),
# a single token, and a multi-tile case.
# (40, 72, 2304): K-slices of 5 and 4 superblocks (odd and even counts);
# (200, 1000, 4096): Q4_K stream-K with every tile split over 4 workgroups and
# ragged rows and tokens.
# (33, 77, 768) and (5, 129, 256): an odd number of weight units, so the
# last unit of a 2-byte-aligned format (IQ3_XXS, Q6_K, IQ3_S, IQ2_S) starts
# 4-byte aligned and its last dword load ends past the matrix.
SHAPES = [(1, 64, 256), (37, 200, 1024), (128, 256, 5120), (130, 136, 2048), (300, 384, 768), (40, 72, 2304),
          (200, 1000, 4096), (33, 77, 768), (5, 129, 256)]


MFMA_TYPES = [Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, Q8_0]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("qt", MFMA_TYPES)
def test_gemm_vs_oracle(tc, dev, oracle, qt, M, N, K):
    rng = np.random.default_rng(M * 7 + N + K + qt)
    w = enc_weights(oracle, qt, rng, N, K)
    x = gaussian(rng, (M, K))
    got = tc.gemm(qt, to_dev(w, dev), to_dev(x, dev), N, K).cpu().numpy()
    ref = oracle.matmul(qt, w, x, N, K)
    ok, worst = close(got, ref)
    assert ok, f"{NAMES[qt]} M={M} N={N} K={K}: worst err/bound {worst:.3g}"


@pytest.mark.parametrize("M", [8, 40, 64, 100])
@pytest.mark.parametrize("qt", MFMA_TYPES)
def test_gemm_token_tiles(tc, dev, oracle, qt, M):
    """Token counts around the token-tile widths the GEMM picks from M (32,
    64, 128 tokens), with a ragged last row block."""
    rng = np.random.default_rng(M * 3 + qt)
    N, K = 300, 2048
    w = enc_weights(oracle, qt, rng, N, K)
    x = gaussian(rng, (M, K))
    got = tc.gemm(qt, to_dev(w, dev), to_dev(x, dev), N, K).cpu().numpy()
    ok, worst = close(got, oracle.matmul(qt, w, x, N, K))
    assert ok, f"{NAMES[qt]} M={M}: worst err/bound {worst:.3g}"


@pytest.mark.parametrize("qt", MFMA_TYPES)
def test_gemm_random_blocks(tc, dev, oracle, qt):
    """Arbitrary block bytes (all scale/min codes, subnormal fp16 scales)."""
    rng = np.random.default_rng(99 + qt)
    M, N, K = 70, 96, 1536
    w = random_blocks(qt, rng, N, K)
    x = gaussian(rng, (M, K))
    got = tc.gemm(qt, to_dev(w, dev), to_dev(x, dev), N, K).cpu().numpy()
    ref = oracle.matmul(qt, w, x, N, K)
    ok, worst = close(got, ref)
    assert ok, worst


@pytest.mark.parametrize("qt", [Q2_K, Q3_K, IQ2_XS, IQ4_XS, IQ4_NL, Q5_0])
def test_gemm_exact_batched_types(tc, dev, oracle, qt):
    rng = np.random.default_rng(5 + qt)
    M, N, K = 21, 80, 512
    w = enc_weights(oracle, qt, rng, N, K)
    x = gaussian(rng, (M, K))
    got = tc.gemm(qt, to_dev(w, dev), to_dev(x, dev), N, K).cpu().numpy()
    ok, worst = close(got, oracle.matmul(qt, w, x, N, K))
    assert ok, worst


@pytest.mark.parametrize("M", [128, 512, 2048])
@pytest.mark.parametrize("qt,N,K", [(Q4_K, 17408, 5120), (Q4_K, 5120, 17408), (Q8_0, 17408, 5120),
                                    (Q8_0, 5120, 17408)])
def test_gemm_cfg4_full_shape(tc, dev, oracle, qt, N, K, M):
    """BASELINE config 4 at full size: both matrices, both types, M in {128,
    512, 2048}."""
    full_shape_check(tc, dev, oracle, qt, N, K, M)


@pytest.mark.parametrize("M", [128, 512])
@pytest.mark.parametrize("qt,N,K", [(qt, N, K) for qt in (Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S)
                                    for N, K in ((18944, 3584), (3584, 18944))])
def test_gemm_7b_ffn_full_shape(tc, dev, oracle, qt, N, K, M):
    """The 7B FFN shapes (18944 x 3584 up, 3584 x 18944 down) for the other
    MFMA types at prefill batch sizes 128 and 512."""
    full_shape_check(tc, dev, oracle, qt, N, K, M)


def full_shape_check(tc, dev, oracle, qt, N, K, M):
    """Weights from the GPU encoder, x ~ N(0,1). The oracle checks
    the first and last row of every 64-row workgroup tile plus 32 seeded rows,
    against every token for M <= 512, and at M = 2048 the first and last token
    of every 128-token tile, the whole last token tile and 32 seeded tokens
    (tokens and rows are independent of each other, so these entries are
    exactly the full output's)."""
    import torch
    gen = torch.Generator(device=dev).manual_seed(4 + qt + N + M)
    wf = torch.randn((N, K), generator=gen, device=dev) * (1.0 if qt in (Q4_K, Q5_K) else 0.02)
    w = tc.encode(qt, wf)
    del wf
    x = torch.randn((M, K), generator=gen, device=dev)
    got = tc.gemm(qt, w, x, N, K).cpu().numpy()
    assert np.isfinite(got).all()
    rng = np.random.default_rng(M + N)
    rows = tile_edges(N, 64, 32, rng)
    toks = np.arange(M) if M <= 512 else tile_edges(M, 128, 32, rng)
    wh = w.cpu().numpy().reshape(N, row_bytes(qt, K))[rows]
    xh = x.cpu().numpy()[toks]
    ref = oracle_matmul_par(oracle, qt, wh, xh, len(rows), K)
    sub = got[np.ix_(toks, rows)]
    ok, worst = close(sub, ref)
    bad = np.argwhere(~(np.abs(sub - ref) <= 1e-4 + 1e-3 * np.abs(ref)))
    assert ok, (f"{NAMES[qt]} M={M} N={N} K={K}: worst err/bound {worst:.3g}; first bad (token, row) "
                f"{[(int(toks[i]), int(rows[j])) for i, j in bad[:5]]}")


def test_gemm_matches_gemv_small_batch(tc, dev):
    """M <= 8: the MFMA GEMM and the decode kernel agree within tolerance."""
    rng = np.random.default_rng(3)
    N, K = 300, 2048
    w = random_blocks(Q4_K, rng, N, K)
    x = gaussian(rng, (5, K))
    wd, xd = to_dev(w, dev), to_dev(x, dev)
    g = tc.gemm(Q4_K, wd, xd, N, K).cpu().numpy()
    v = tc.gemv(Q4_K, wd, xd, N, K).cpu().numpy()
    ok, worst = close(g, v)
    assert ok, worst


def test_gemm_refuses_bad_shapes(tc, dev):
    import tc_hip
    w = to_dev(np.zeros(row_bytes(Q4_K, 512) * 4, np.uint8), dev)
    x = to_dev(np.zeros((3, 500), np.float32), dev)
    with pytest.raises(tc_hip.TCError):
        tc.gemm(Q4_K, w, x, 4, 500)


def test_q80_minus128_true_product(tc, dev, oracle):
    """Q8_0 weight bytes of -128 (never written by a quantizer: q =
    round(w/d) with d = amax/127 stays in [-127, 127]): the GPU paths compute
    the true product -128 * x. The reference AVX2 kernel's sign trick
    (SIMDMatMulVecAVX2.cpp:4239-4383) cannot negate -128 and gives -128 * |x|
    instead; the oracle mirrors that, so on such rows the two differ. Pins the
    GPU's behaviour (mat-vec, the MFMA GEMM and the host entry point) against
    the exact product from the reference's own activation quantization."""
    rng = np.random.default_rng(128)
    rows, cols = 96, 1024
    w = random_blocks(Q8_0, rng, rows, cols)
    blk = w.reshape(rows, cols // 32, 34)
    q = blk[:, :, 2:].view(np.int8)
    q[rng.random(q.shape) < 0.05] = -128  # some -128 bytes in most blocks
    blk[:, :, :2] = (rng.uniform(0.5, 2.0, (rows, cols // 32, 1)) * 1e-3).astype(np.float16).view(np.uint8)
    dw = blk[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    for S in (1, 4, 40):
        x = gaussian(rng, (S, cols))
        exact = np.zeros((S, rows))
        for s in range(S):
            xq, d8 = oracle.quantize_q8_0_act(x[s])
            isum = (q.astype(np.int64) * xq.reshape(cols // 32, 32).astype(np.int64)[None]).sum(axis=2)
            exact[s] = (isum * dw * d8.astype(np.float64)[None]).sum(axis=1)
        xd, wd = to_dev(x, dev), to_dev(w, dev)
        got = tc.gemv(Q8_0, wd, xd, rows, cols) if S <= 8 else tc.gemm(Q8_0, wd, xd, rows, cols)
        ok, worst = close(got.cpu().numpy(), exact.astype(np.float32))
        assert ok, f"S={S}: worst err/bound {worst:.3g}"
        ref = oracle.matmul(Q8_0, w, x, rows, cols)
        assert not close(ref, exact.astype(np.float32))[0], "the reference quirk should show on these rows"
