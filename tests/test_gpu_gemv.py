"""GPU parity tests for the decode mat-vec path, through the C-ABI.

Bars (stated in the tests): activation quantization bytes and scales and the
per-block int32 dot sums are bit-exact against the oracle; fp32 outputs are
within 1e-3 relative / 1e-4 absolute of the oracle (which is itself bit-exact
with the compiled reference, tests/test_oracle.py) and of the golden outputs.
"""
import numpy as np
import pytest

import oracle as O
from qdata import ALL, INT8_ACT, IQ2_S, IQ2_XS, IQ4_NL, IQ4_XS, Q5_0, IQ3_S, IQ3_XXS, NAMES, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, close, gaussian, oracle_matmul_par, random_blocks, row_bytes

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def f32bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---- activation quantizers ---------------------------------------------------------

def test_quantize_q8k_golden(tc, dev, golden):
    x = golden["q8k_x"]
    qs, d, bs = tc.quantize_act(Q4_K, to_dev(x, dev), x.shape[1])
    assert (qs.cpu().numpy() == golden["q8k_qs"]).all()
    assert (f32bits(d.cpu().numpy()) == f32bits(golden["q8k_d"])).all()
    assert (bs.cpu().numpy() == golden["q8k_bsums"]).all()


@pytest.mark.parametrize("qt", [Q4_K, Q8_0])
@pytest.mark.parametrize("S,cols", [(1, 256), (3, 3584), (8, 18944), (2, 5120), (5, 6711040)])
def test_quantize_act_bit_exact(tc, dev, oracle, qt, S, cols):
    """Bit-exact against the oracle. 5 x 6711040 is 131075 blocks: the
    large-batch quantizer (4 blocks per wave) with a partial last wave."""
    rng = np.random.default_rng(cols + S)
    x = gaussian(rng, (S, cols))
    x[0, :64] = 0.0
    x[-1, 100], x[-1, 101] = -7.0, 7.0  # |x| tie, first wins
    qs, d, bs = tc.quantize_act(qt, to_dev(x, dev), cols)
    for s in range(S):
        if qt == Q8_0:
            rq, rd = oracle.quantize_q8_0_act(x[s])
        else:
            rq, rd, rb = oracle.quantize_q8k(x[s])
            assert (bs[s].cpu().numpy() == rb).all()
        assert (qs[s].cpu().numpy() == rq).all()
        assert (f32bits(d[s].cpu().numpy()) == f32bits(rd)).all()


def test_quantize_act_probe_golden(tc, dev, golden):
    # The Q8_0 activation quantizer of the reference kernel, pinned through
    # its unit-probe outputs (out[i] = d8 * xq[i]).
    x = golden["probe_q80_x"]
    qs, d, _ = tc.quantize_act(Q8_0, to_dev(x, dev), x.shape[1])
    got = np.repeat(d.cpu().numpy(), 32, axis=1) * qs.cpu().numpy().astype(np.float32)
    assert np.array_equal(got, golden["probe_q80_y"])


# ---- per-block integer sums ---------------------------------------------------------

@pytest.mark.parametrize("qt", INT8_ACT)
@pytest.mark.parametrize("S,rows,cols", [(1, 37, 512), (3, 130, 1024), (8, 9, 3584), (1, 5, 18944)])
def test_block_isums_bit_exact(tc, dev, oracle, qt, S, rows, cols):
    rng = np.random.default_rng(rows * 31 + qt)
    w = random_blocks(qt, rng, rows, cols)
    x = gaussian(rng, (S, cols))
    got = tc.block_isums(qt, to_dev(w, dev), to_dev(x, dev), rows, cols).cpu().numpy()
    ref = oracle.block_isums(qt, w, x, rows, cols)
    assert got.shape == ref.shape
    assert (got == ref).all(), f"{NAMES[qt]}: {np.argwhere(got != ref)[:5]}"


# ---- mat-vec outputs ----------------------------------------------------------------------

MM = [("q4k_rand", Q4_K), ("q4k_enc1", Q4_K), ("q4k_enc002", Q4_K),
      ("q5k_rand", Q5_K), ("q5k_enc1", Q5_K), ("q3k_rand", Q3_K), ("q3k_enc002", Q3_K), ("q2k_rand", Q2_K), ("q2k_enc002", Q2_K), ("iq3s_rand", IQ3_S),
      ("iq3s_enc002", IQ3_S), ("iq2s_rand", IQ2_S), ("iq2s_enc002", IQ2_S),
      ("iq2xs_rand", IQ2_XS), ("iq2xs_enc002", IQ2_XS), ("iq4xs_rand", IQ4_XS), ("iq4xs_enc002", IQ4_XS),
      ("iq4nl_rand", IQ4_NL), ("iq4nl_enc002", IQ4_NL), ("q50_rand", Q5_0), ("q50_enc002", Q5_0),
      ("q6k_rand", Q6_K), ("iq3_rand", IQ3_XXS), ("q80_rand", Q8_0)]


@pytest.mark.parametrize("name,qt", MM)
def test_gemv_golden(tc, dev, golden, name, qt):
    w = golden[f"mm_{name}_w"]
    if qt == Q8_0:
        # the golden Q8_0 bytes include -128 (the reference kernel's sign-trick
        # quirk); compare only rows whose weights avoid it
        pass
    for tag in ("1", "4"):
        x = golden[f"mm_x{tag}"]
        y = golden[f"mm_{name}_y{tag}"]
        rows, cols = y.shape[1], x.shape[1]
        got = tc.gemv(qt, to_dev(w, dev), to_dev(x, dev), rows, cols).cpu().numpy()
        if qt == Q8_0:
            wq = w.reshape(rows, cols // 32, 34)[:, :, 2:].view(np.int8)
            ok_rows = ~(wq == -128).any(axis=(1, 2))
            got, y = got[:, ok_rows], y[:, ok_rows]
            assert ok_rows.sum() >= 1
        ok, worst = close(got, y)
        assert ok, f"{name} S={tag}: worst err/bound {worst:.2f}"


WIDE = [("q4k", Q4_K, c) for c in (3584, 5120, 17408, 18944)] + [("q6k", Q6_K, c) for c in (3584, 17408, 18944)] + \
       [("iq3", IQ3_XXS, c) for c in (3584, 17408, 18944)] + [("q80", Q8_0, c) for c in (4096, 5120, 17408)]


@pytest.mark.parametrize("name,qt,cols", WIDE)
def test_gemv_golden_baseline_widths(tc, dev, golden, name, qt, cols):
    """The compiled reference's outputs at the BASELINE widths (8 rows, one
    token and four): decode mat-vec and, for the four tokens, the prefill
    GEMM entry point, both within 1e-3 relative / 1e-4 absolute."""
    w = golden[f"mmw_{name}_{cols}_w"]
    x4 = golden[f"mmw_x4_{cols}"]
    wd = to_dev(w, dev)
    for tag, x in (("1", x4[:1]), ("4", x4)):
        y = golden[f"mmw_{name}_{cols}_y{tag}"]
        got = tc.gemv(qt, wd, to_dev(x, dev), 8, cols).cpu().numpy()
        ok, worst = close(got, y)
        assert ok, f"{name} cols={cols} S={tag}: worst err/bound {worst:.2f}"
    got = tc.gemm(qt, wd, to_dev(x4, dev), 8, cols).cpu().numpy()
    ok, worst = close(got, golden[f"mmw_{name}_{cols}_y4"])
    assert ok, f"{name} cols={cols} gemm: worst err/bound {worst:.2f}"


@pytest.mark.parametrize("qt", ALL)
@pytest.mark.parametrize("S", [1, 3])
def test_gemv_odd_unit_count(tc, dev, oracle, qt, S):
    """77 rows x 768 columns: an odd number of weight units, so the last
    unit of a 2-byte-aligned format ends 2 bytes into a dword past the
    matrix."""
    rng = np.random.default_rng(300 + 10 * qt + S)
    rows, cols = 77, 768
    w = oracle.encode(qt, gaussian(rng, (rows, cols), 1.0 if qt == Q4_K else 0.02))
    x = gaussian(rng, (S, cols))
    got = tc.gemv(qt, to_dev(w, dev), to_dev(x, dev), rows, cols).cpu().numpy()
    ref = oracle.matmul(qt, w, x, rows, cols)
    ok, worst = close(got, ref)
    assert ok, f"{NAMES[qt]} S={S}: worst err/bound {worst:.2f}"


@pytest.mark.parametrize("qt", ALL)
@pytest.mark.parametrize("S", [1, 2, 5, 8])
def test_gemv_vs_oracle(tc, dev, oracle, qt, S):
    """Encoder-made weights (realistic scales). Random-byte blocks, whose
    extreme sub-scales make results cancel far below the size of their terms,
    are covered bit-exactly by the integer-sum tests and by the goldens."""
    rng = np.random.default_rng(100 * qt + S)
    rows, cols = 203, 2048
    w = oracle.encode(qt, gaussian(rng, (rows, cols), 1.0 if qt == Q4_K else 0.02))
    x = gaussian(rng, (S, cols))
    got = tc.gemv(qt, to_dev(w, dev), to_dev(x, dev), rows, cols).cpu().numpy()
    ref = oracle.matmul(qt, w, x, rows, cols)
    ok, worst = close(got, ref)
    assert ok, f"{NAMES[qt]} S={S}: worst err/bound {worst:.2f}"


@pytest.mark.parametrize("qt,rows,cols", [
    (Q4_K, 3584, 3584), (Q4_K, 512, 3584), (Q4_K, 18944, 3584), (Q4_K, 3584, 18944),
    (Q8_0, 4096, 4096), (Q6_K, 152064, 3584), (Q6_K, 3584, 18944), (IQ3_XXS, 18944, 3584),
    (Q5_K, 18944, 3584), (Q3_K, 3584, 18944), (IQ3_S, 18944, 3584), (IQ2_S, 3584, 18944), (Q2_K, 18944, 3584),
    (IQ2_XS, 18944, 3584), (IQ4_XS, 3584, 18944), (IQ4_NL, 18944, 3584), (Q5_0, 3584, 18944), (IQ2_XS, 3584, 18944),
])
def test_gemv_full_shapes(tc, dev, oracle, qt, rows, cols):
    """BASELINE shapes at full size (configs 1-3, the Q6_K LM head included),
    weights from the GPU encoder on N(0,0.02) (Q4_K on N(0,1), where the
    reference quantizer keeps d normal): EVERY output row is compared with the
    oracle, so each workgroup's row range, its boundaries and the last partial
    tile are all checked."""
    import torch
    g = torch.Generator(device=dev).manual_seed(rows + cols + qt)
    std = 1.0 if qt == Q4_K else 0.02
    wf = torch.randn((rows, cols), generator=g, device=dev) * std
    w = tc.encode(qt, wf)
    del wf
    rng = np.random.default_rng(1)
    x = gaussian(rng, (1, cols))
    got = tc.gemv(qt, w, to_dev(x, dev), rows, cols).cpu().numpy()
    ref = oracle_matmul_par(oracle, qt, w.cpu().numpy(), x, rows, cols)
    assert np.isfinite(got).all()
    ok, worst = close(got, ref)
    bad = np.argwhere(~(np.abs(got - ref) <= 1e-4 + 1e-3 * np.abs(ref)))
    assert ok, f"{NAMES[qt]} {rows}x{cols}: worst err/bound {worst:.2f}, first bad rows {bad[:5, 1].tolist()}"


def test_q80_ragged_cols_golden(tc, dev, golden):
    """Q8_0 at cols = 96 (3 blocks; the reference's Q8_0 dispatch takes any
    cols % 32 == 0, QuantizedMatrix.cpp:96-103): the compiled reference's
    outputs through the decode entry point and the GEMM entry point."""
    w, x, y = golden["mm_q80c96_w"], golden["mm_q80c96_x"], golden["mm_q80c96_y"]
    rows, cols = y.shape[1], 96
    wq = w.reshape(rows, 3, 34)[:, :, 2:].view(np.int8)
    ok_rows = ~(wq == -128).any(axis=(1, 2))  # the reference kernel's -128 quirk (see test_gemv_golden)
    assert ok_rows.sum() >= 4
    for got in (tc.gemv(Q8_0, to_dev(w, dev), to_dev(x, dev), rows, cols).cpu().numpy(),
                tc.gemm(Q8_0, to_dev(w, dev), to_dev(x, dev), rows, cols).cpu().numpy()):
        ok, worst = close(got[:, ok_rows], y[:, ok_rows])
        assert ok, worst


@pytest.mark.parametrize("S,rows,cols", [(1, 300, 4000), (3, 77, 800), (8, 130, 32), (2, 64, 18976)])
def test_q80_ragged_cols_vs_oracle(tc, dev, oracle, S, rows, cols):
    """Q8_0 widths that are multiples of 32 but not of 256, through tc_gemv,
    tc_gemm (M = 40 as well) and the gate/up pair, against the oracle; the
    activation bytes and scales of the quantizer entry point bit-exact."""
    import torch
    rng = np.random.default_rng(cols + S)
    wf = gaussian(rng, (rows, cols), 0.02)
    # the Q8_0 encoder works on whole 256-column units: encode the padded
    # matrix and cut each row back to its cols/32 blocks
    cp = (cols + 255) // 256 * 256
    wpad = np.zeros((rows, cp), np.float32)
    wpad[:, :cols] = wf
    w = oracle.encode(Q8_0, wpad).reshape(rows, cp // 32, 34)[:, :cols // 32].copy().ravel()
    x = gaussian(rng, (S, cols))
    ref = oracle.matmul(Q8_0, w, x, rows, cols)
    wd, xd = to_dev(w, dev), to_dev(x, dev)
    for got in (tc.gemv(Q8_0, wd, xd, rows, cols).cpu().numpy(), tc.gemm(Q8_0, wd, xd, rows, cols).cpu().numpy()):
        ok, worst = close(got, ref)
        assert ok, worst
    x40 = gaussian(rng, (40, cols))
    ok, worst = close(tc.gemm(Q8_0, wd, to_dev(x40, dev), rows, cols).cpu().numpy(),
                      oracle.matmul(Q8_0, w, x40, rows, cols))
    assert ok, worst
    # gate/up pair (up = the same matrix) with the SwiGLU epilogue
    gout = torch.empty((1, rows), device=dev)
    uout = torch.empty((1, rows), device=dev)
    from tc_hip import _ptr
    tc._check(tc.lib.tc_gemv_dual(Q8_0, _ptr(wd), _ptr(wd), _ptr(xd[:1].contiguous()), _ptr(gout), _ptr(uout),
                                  rows, cols, tc._stream()))
    u = uout.cpu().numpy()[0]
    ok, worst = close(u, ref[0])
    assert ok, worst
    ok, worst = close(gout.cpu().numpy()[0], ref[0] / (1.0 + np.exp(-ref[0].astype(np.float64))) * ref[0], 2e-3)
    assert ok, worst
    qs, d, _ = tc.quantize_act(Q8_0, xd, cols)
    for s in range(S):
        rq, rd = oracle.quantize_q8_0_act(x[s])
        assert (qs[s].cpu().numpy() == rq).all()
        assert (f32bits(d[s].cpu().numpy()) == f32bits(rd)).all()


def test_gemv_zero_activation(tc, dev):
    import torch
    rng = np.random.default_rng(0)
    for qt in ALL:
        w = random_blocks(qt, rng, 64, 512)
        x = torch.zeros((1, 512), device=dev)
        got = tc.gemv(qt, to_dev(w, dev), x, 64, 512).cpu().numpy()
        assert (got == 0).all()


def test_gemv_refuses_bad_shapes_without_writing(tc, dev):
    import torch
    from tc_hip import TC_E_UNSUPPORTED, TCError
    w = torch.zeros(144 * 4, dtype=torch.uint8, device=dev)
    x = torch.zeros((1, 512), device=dev)
    out = torch.full((1, 2), 7.0, device=dev)
    for args in [(Q4_K, 2, 300), (Q4_K, 0, 512), (9, 2, 512)]:
        qt, rows, cols = args
        with pytest.raises(TCError) as e:
            tc.gemv(qt, w, x, rows, cols, out=out)
        assert e.value.code == TC_E_UNSUPPORTED
    x9 = torch.zeros((9, 512), device=dev)
    with pytest.raises(TCError):
        tc.gemv(Q4_K, w, x9, 2, 512, out=out)
    torch.cuda.synchronize()
    assert (out.cpu() == 7.0).all()


# ---- encoders --------------------------------------------------------------------------------

@pytest.mark.parametrize("qt", ALL)
def test_encoder_bit_exact_vs_oracle(tc, dev, oracle, qt):
    rng = np.random.default_rng(qt)
    x = np.concatenate([gaussian(rng, (8, 512)), gaussian(rng, (8, 512), 0.02),
                        gaussian(rng, (2, 512), 1e-4)])
    x[0, :256] = 0.0
    got = tc.encode(qt, to_dev(x, dev)).cpu().numpy()
    ref = oracle.encode(qt, x)
    assert (got == ref).all(), f"{NAMES[qt]}: first diff {np.argwhere(got != ref)[:4].ravel()}"


def test_q4k_encoder_golden(tc, dev, golden):
    got = tc.encode(Q4_K, to_dev(golden["enc_q4k_x"], dev)).cpu().numpy()
    assert (got.reshape(-1, 144) == golden["enc_q4k_out"]).all()


# ---- multi-matrix launch, gate/up pair, pre-quantized activations -------------------------

def test_gemv_multi_matches_single(tc, dev, oracle):
    """q/k/v-style launch (shared input) plus matrices with their own input and
    width, in ONE launch; every output equals the oracle within tolerance and
    the single-matrix launch bit for bit (same kernel, same block order)."""
    rng = np.random.default_rng(77)
    shapes = [(300, 1024), (64, 1024), (64, 1024), (128, 2048), (40, 512)]
    ws = [random_blocks(Q4_K, rng, r, c) for r, c in shapes]
    x1 = gaussian(rng, (1, 1024))
    xs = [x1, x1, x1, gaussian(rng, (1, 2048)), gaussian(rng, (1, 512))]
    wd = [to_dev(w, dev) for w in ws]
    xd = [to_dev(x, dev) for x in xs]
    outs = tc.gemv_multi(Q4_K, wd, xd, [r for r, _ in shapes], [c for _, c in shapes])
    for i, (r, c) in enumerate(shapes):
        got = outs[i].cpu().numpy()
        single = tc.gemv(Q4_K, wd[i], xd[i], r, c).cpu().numpy()
        assert np.array_equal(got, single), i
        ok, worst = close(got, oracle.matmul(Q4_K, ws[i], xs[i], r, c))
        assert ok, (i, worst)


def test_gemv_multi_eight_jobs(tc, dev, oracle):
    """The largest job list (8 matrices of different heights and widths): every
    workgroup must find its job, the last one included."""
    rng = np.random.default_rng(78)
    shapes = [(96, 512), (200, 1024), (33, 256), (512, 768), (64, 2048), (7, 512), (150, 1280), (301, 512)]
    ws = [random_blocks(Q4_K, rng, r, c) for r, c in shapes]
    xs = [gaussian(rng, (1, c)) for _, c in shapes]
    wd = [to_dev(w, dev) for w in ws]
    xd = [to_dev(x, dev) for x in xs]
    outs = tc.gemv_multi(Q4_K, wd, xd, [r for r, _ in shapes], [c for _, c in shapes])
    for i, (r, c) in enumerate(shapes):
        got = outs[i].cpu().numpy()
        assert np.array_equal(got, tc.gemv(Q4_K, wd[i], xd[i], r, c).cpu().numpy()), i
        ok, worst = close(got, oracle.matmul(Q4_K, ws[i], xs[i], r, c))
        assert ok, (i, worst)


@pytest.mark.parametrize("S", [1, 2])
def test_gemv_multi_full_layer(tc, dev, oracle, S):
    """The 7 matrices of a Qwen2.5-7B layer (q, k, v, o, gate, up, down;
    inputs of 3584 and 18944 columns) in ONE launch, as the benchmark's
    one-launch layer: the workgroup shares differ from the single launches
    (per-job staging cost), so every output is checked against its own
    single-matrix launch bit for bit and against the oracle on every row."""
    import torch
    H, F = 3584, 18944
    shapes = [(H, H), (512, H), (512, H), (H, H), (F, H), (F, H), (H, F)]
    g = torch.Generator(device=dev).manual_seed(90 + S)
    rng = np.random.default_rng(90 + S)
    ws, xs = [], []
    for r, c in shapes:
        ws.append(tc.encode(Q4_K, torch.randn((r, c), generator=g, device=dev)))
    x_attn = gaussian(rng, (S, H))
    xs = [x_attn, x_attn, x_attn, gaussian(rng, (S, H)), *(2 * [gaussian(rng, (S, H))]), gaussian(rng, (S, F))]
    xd = [to_dev(x, dev) for x in xs]
    outs = tc.gemv_multi(Q4_K, ws, xd, [r for r, _ in shapes], [c for _, c in shapes])
    for i, (r, c) in enumerate(shapes):
        got = outs[i].cpu().numpy()
        single = tc.gemv(Q4_K, ws[i], xd[i], r, c).cpu().numpy()
        assert np.array_equal(got, single), (i, r, c)
        ref = oracle_matmul_par(oracle, Q4_K, ws[i].cpu().numpy(), xs[i], r, c)
        ok, worst = close(got, ref)
        assert ok, (i, r, c, worst)


@pytest.mark.parametrize("qt", ALL)
def test_gemv_dual_swiglu(tc, dev, oracle, qt):
    """gate/up pair in one launch: uout = up row sums, gout = silu(gate) * up.
    The gate pre-activation is not an output, so its tolerance is carried
    through silu (|silu'| <= 1.1): |d(silu(g) u)| <= 1.1 |u| dg + |silu(g)| du."""
    rng = np.random.default_rng(5 + qt)
    rows, cols = 517, 1536
    sd = 1.0 if qt == Q4_K else 0.02
    wg = oracle.encode(qt, gaussian(rng, (rows, cols), sd))
    wu = oracle.encode(qt, gaussian(rng, (rows, cols), sd))
    x = gaussian(rng, (1, cols))
    g, u = tc.gemv_dual(qt, to_dev(wg, dev), to_dev(wu, dev), to_dev(x, dev), rows, cols)
    g, u = g.cpu().numpy().astype(np.float64), u.cpu().numpy().astype(np.float64)
    rg = oracle.matmul(qt, wg, x, rows, cols)[0].astype(np.float64)
    ru = oracle.matmul(qt, wu, x, rows, cols)[0].astype(np.float64)
    ok, worst = close(u, ru)
    assert ok, worst
    silu = rg / (1.0 + np.exp(-rg))
    ref = silu * ru
    dg = 1e-4 + 1e-3 * np.abs(rg)
    du = 1e-4 + 1e-3 * np.abs(ru)
    bound = 1.1 * np.abs(ru) * dg + np.abs(silu) * du + 1e-6
    err = np.abs(g - ref)
    assert (err <= bound).all(), float((err / bound).max())


@pytest.mark.parametrize("qt", INT8_ACT)
def test_gemv_prequantized_equals_fused(tc, dev, qt):
    """tc_act_quantize + tc_gemv_q8 (the reference's launchQGemvQ81 shape)
    gives bit-identical results to tc_gemv, which quantizes in-kernel."""
    rng = np.random.default_rng(31 + qt)
    rows, cols, S = 129, 3584, 3
    w = to_dev(random_blocks(qt, rng, rows, cols), dev)
    x = to_dev(gaussian(rng, (S, cols)), dev)
    act = tc.act_buffer(qt, S, cols)
    tc.act_quantize(qt, x, cols, act)
    a = tc.gemv_q8(qt, w, act, S, rows, cols).cpu().numpy()
    b = tc.gemv(qt, w, x, rows, cols).cpu().numpy()
    assert np.array_equal(a, b)


# ---- parity hooks (reference GPUModel::debugQ8KRow / debugQ8_0Row / debugQ8KBlocks /
# debugQ8_0Blocks, include/GPUCompute.hpp:399-460) -----------------------------------------------

@pytest.mark.parametrize("qt", INT8_ACT)
def test_debug_row_hook(tc, dev, oracle, qt):
    rng = np.random.default_rng(400 + qt)
    cols = 2048
    w = random_blocks(qt, rng, 3, cols)
    x = gaussian(rng, (1, cols))
    rb = row_bytes(qt, cols)
    full = tc.gemv(qt, to_dev(w, dev), to_dev(x, dev), 3, cols).cpu().numpy()[0]
    for r in range(3):
        v = tc.debug_row(qt, w[r * rb:(r + 1) * rb], x)
        assert np.float32(v) == full[r]  # same kernel, same order
        ok, worst = close(v, oracle.matmul(qt, w[r * rb:(r + 1) * rb], x, 1, cols)[0, 0])
        assert ok, worst


@pytest.mark.parametrize("qt", INT8_ACT)
def test_debug_blocks_hook(tc, dev, oracle, qt):
    rng = np.random.default_rng(500 + qt)
    cols = 1536
    w = random_blocks(qt, rng, 1, cols)
    x = gaussian(rng, (1, cols))
    blk, q = tc.debug_blocks(qt, w, x)
    bs = O.oc_block_size(qt) if hasattr(O, "oc_block_size") else (32 if qt == Q8_0 else 256)
    nb = cols // bs
    # activation blocks: bit-exact against the oracle's quantizer
    if qt == Q8_0:
        qs, d = oracle.quantize_q8_0_act(x)
        rec = q.reshape(nb, 36)
        assert np.array_equal(rec[:, :4].copy().view(np.float32).ravel().view(np.uint32), d.view(np.uint32))
        assert np.array_equal(rec[:, 4:].copy().view(np.int8).ravel(), qs)
    else:
        qs, d, bsum = oracle.quantize_q8k(x)
        rec = q.reshape(nb, 292)
        assert np.array_equal(rec[:, :4].copy().view(np.float32).ravel().view(np.uint32), d.view(np.uint32))
        assert np.array_equal(rec[:, 4:260].copy().view(np.int8).ravel(), qs)
        assert np.array_equal(rec[:, 260:].copy().view(np.int16).ravel(), bsum)
    # each block's contribution: the oracle on the row with every other block zeroed
    tb = row_bytes(qt, bs)
    for b in range(nb):
        wz = w.copy().reshape(nb, tb)
        for k in range(nb):
            if k == b:
                continue
            if qt in (Q4_K, Q5_K):
                wz[k, :4] = 0
            elif qt == Q6_K:
                wz[k, 208:210] = 0
            elif qt == Q3_K:
                wz[k, 108:110] = 0
            elif qt == Q2_K:
                wz[k, 80:84] = 0
            else:
                wz[k, :2] = 0
        ok, worst = close(blk[b], oracle.matmul(qt, wz.ravel(), x, 1, cols)[0, 0])
        assert ok, (b, worst)


@pytest.mark.parametrize("qt", [IQ2_XS, IQ4_NL, Q5_0])
def test_float_types_refuse_quantized_activation_entry_points(tc, dev, qt):
    """IQ2_XS, IQ4_NL and Q5_0 dot fp32 x (as their reference CPU paths): the entry
    points that hand over quantized activations refuse them without writing."""
    import ctypes
    import torch
    from tc_hip import TC_E_UNSUPPORTED, _ptr
    w = torch.zeros(row_bytes(qt, 256) * 2, dtype=torch.uint8, device=dev)
    x = torch.zeros((1, 256), device=dev)
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    out = torch.full((1, 2), 7.0, device=dev)
    assert tc.lib.tc_act_bytes(qt, 1, 256) == 0
    assert tc.lib.tc_act_quantize(qt, _ptr(x), 1, 256, _ptr(buf), None) == TC_E_UNSUPPORTED
    assert tc.lib.tc_gemv_q8(qt, _ptr(w), _ptr(buf), _ptr(out), 1, 2, 256, None) == TC_E_UNSUPPORTED
    isums = torch.zeros(16, dtype=torch.int32, device=dev)
    assert tc.lib.tc_block_isums(qt, _ptr(w), _ptr(x), _ptr(isums), 1, 2, 256, None) == TC_E_UNSUPPORTED
    # the per-block debug hook (host buffers) refuses them too, writing nothing
    import numpy as np
    w_row = np.zeros(row_bytes(qt, 256), dtype=np.uint8)
    xh = np.ones(256, dtype=np.float32)
    out_blk = np.full(8, 7.0, dtype=np.float32)
    out_q = np.full(292, 0x5A, dtype=np.uint8)
    nbpr = 256 // 32  # IQ4_NL / Q5_0 blocks per row; IQ2_XS has 1
    for bpr in (1, nbpr):
        rc = tc.lib.tc_debug_q8k_blocks(qt, w_row.ctypes.data, bpr, xh.ctypes.data, 256, out_blk.ctypes.data,
                                        out_q.ctypes.data)
        assert rc == TC_E_UNSUPPORTED
    assert (out_blk == 7.0).all() and (out_q == 0x5A).all()
    torch.cuda.synchronize()
    assert (out.cpu() == 7.0).all()
    del ctypes


@pytest.mark.parametrize("qt", [IQ2_XS, IQ4_NL, Q5_0])
def test_float_types_wide_multi_token(tc, dev, oracle, qt):
    """fp32-activation types at cols=18944 with 8 tokens: tc_gemv and tc_gemm
    (which split the tokens over launches when x does not fit one workgroup's
    LDS) match the oracle, and tc_gemv_multi, which must run all tokens in one
    launch, either matches it too or refuses without writing."""
    import torch
    import tc_hip
    rng = np.random.default_rng(77 + qt)
    S, rows, cols = 8, 256, 18944
    w = random_blocks(qt, rng, rows, cols)
    x = gaussian(rng, (S, cols))
    ref = oracle_matmul_par(oracle, qt, w, x, rows, cols)
    wd, xd = torch.from_numpy(w).to(dev), torch.from_numpy(x).to(dev)
    for fn in (tc.gemv, tc.gemm):
        ok, worst = close(fn(qt, wd, xd, rows, cols).cpu().numpy(), ref)
        assert ok, (fn.__name__, worst)
    out = torch.full((S, rows), 7.0, device=dev)
    try:
        tc.gemv_multi(qt, [wd], [xd], [rows], [cols], outs=[out])
    except tc_hip.TCError as e:
        assert e.code == tc_hip.TC_E_UNSUPPORTED
        torch.cuda.synchronize()
        assert (out.cpu() == 7.0).all()
    else:
        ok, worst = close(out.cpu().numpy(), ref)
        assert ok, worst
