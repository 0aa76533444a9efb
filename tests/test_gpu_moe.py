"""GPU parity tests for the MoE expert FFN (tc_moe_ffn), through the C-ABI.

Bar: fp32 outputs within 1e-3 relative / 1e-4 absolute of the oracle's MoE
composition (oracle/oracle.c oc_moe_ffn, which follows ModelMoE.cpp:566-600,
660-672, 990-1002) and of the golden composition computed through the compiled
reference kernels (tests/golden/gen_golden.py).

A composition of three mat-vecs with SwiGLU between them has outputs that
cancel to nearly zero; their difference between two fp32 summation orders is
set by the magnitude of the terms, not of the result. For those outputs only,
the relative part of the bound uses 1e-3 of the token's output RMS instead of
|ref|; the tests assert that at most 0.1% of outputs take that floor. The
grouped-GEMM tests also allow, for at most 1% of the tokens, one int8 step of
the requantized SwiGLU output (close_moe_flips).
"""
import numpy as np
import pytest

from gen_golden import moe_weights
from qdata import Q4_K

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def close_moe(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=1, keepdims=True))
    strict = 1e-4 + 1e-3 * np.abs(ref)
    floored = 1e-4 + 1e-3 * np.maximum(np.abs(ref), 1e-3 * rms)
    err = np.abs(got - ref)
    n_floor = int(((err > strict) & (err <= floored)).sum())
    ok = bool((err <= floored).all()) and n_floor <= max(1, err.size // 1000)
    return ok, f"worst err/bound {float((err / floored).max()):.3g}, {n_floor} of {err.size} on the RMS floor"


def h_step_bound(oracle, x, ids, wts, wg, wu, wd, E, H, FF):
    """Per token, the change of its output that one int8 step of the Q8_K
    quantization of h = silu(gate)*up can cause: sum over its ranks of
    wts * (max|h| / 127) * max|W_down[e]|. The gate/up sums are fp32 in a
    different order on each path, so an h value within rounding of a
    quantization boundary may land on either side; the test allows that
    one-step flip, and only on a few outputs."""
    gb, db = row_bytes_q4k(H) * FF, row_bytes_q4k(FF) * H
    wdmax = [np.abs(oracle.dequant(Q4_K, wd[e * db:(e + 1) * db], H, FF)).max() for e in range(E)]
    S, K = ids.shape
    step = np.zeros((S, 1))
    for t in range(S):
        for r in range(K):
            e = int(ids[t, r])
            if not 0 <= e < E:
                continue
            g = oracle.matmul(Q4_K, wg[e * gb:(e + 1) * gb], x[t:t + 1], FF, H)[0].astype(np.float64)
            u = oracle.matmul(Q4_K, wu[e * gb:(e + 1) * gb], x[t:t + 1], FF, H)[0].astype(np.float64)
            h = g / (1 + np.exp(-g)) * u
            step[t] += abs(wts[t, r]) * np.abs(h).max() / 127 * wdmax[e]
    return step


def row_bytes_q4k(cols):
    return cols // 256 * 144


def close_moe_flips(got, ref, step):
    """close_moe, except that the outputs of at most 1% of the tokens (at
    least 1) may instead be within the bar plus one h quantization step of
    their token (one flipped h element moves every output of its token)."""
    ok, msg = close_moe(got, ref)
    if ok:
        return ok, msg
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=1, keepdims=True))
    floored = 1e-4 + 1e-3 * np.maximum(np.abs(ref), 1e-3 * rms)
    err = np.abs(got - ref)
    over = err > floored
    n_tok = int(over.any(axis=1).sum())
    ok = bool((err <= floored + step).all()) and n_tok <= max(1, err.shape[0] // 100)
    return ok, (f"{msg}; {int(over.sum())} outputs of {n_tok} tokens past the bar, "
                f"worst err/(bar+step) {float((err / (floored + step)).max()):.3g}")


def routing(rng, S, E, K):
    """Top-K ids uniform without replacement, weights softmax of N(0,1) logits
    (the benchmark configuration's routing)."""
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(S)]).astype(np.int32)
    lg = rng.standard_normal((S, K)).astype(np.float32)
    wts = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
    return ids, wts


def test_moe_golden_composition(tc, dev, oracle, golden):
    E, K, H, FF, S, seed = [int(v) for v in golden["moe_dims"]]
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed)
    got = tc.moe_ffn(to_dev(golden["moe_x"], dev), to_dev(golden["moe_ids"], dev), to_dev(golden["moe_wts"], dev),
                     to_dev(wg, dev), to_dev(wu, dev), to_dev(wd, dev), E, H, FF).cpu().numpy()
    ok, worst = close_moe(got, golden["moe_y"])
    assert ok, worst


@pytest.mark.parametrize("S", [1, 5])
def test_moe_vs_oracle(tc, dev, oracle, S):
    E, K, H, FF = 16, 4, 1024, 512
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed=31 + S)
    rng = np.random.default_rng(S)
    ids, wts = routing(rng, S, E, K)
    x = rng.standard_normal((S, H)).astype(np.float32)
    got = tc.moe_ffn(to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), to_dev(wg, dev), to_dev(wu, dev),
                     to_dev(wd, dev), E, H, FF).cpu().numpy()
    ok, worst = close_moe(got, oracle.moe_ffn(x, ids, wts, wg, wu, wd, E, H, FF))
    assert ok, worst


def test_moe_skips_out_of_range_ids(tc, dev, oracle):
    """An id outside [0, n_experts) contributes nothing (the oracle skips it)."""
    E, K, H, FF, S = 8, 3, 512, 256, 2
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed=5)
    rng = np.random.default_rng(9)
    ids, wts = routing(rng, S, E, K)
    ids[0, 1] = -1
    ids[1, 2] = E
    x = rng.standard_normal((S, H)).astype(np.float32)
    got = tc.moe_ffn(to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), to_dev(wg, dev), to_dev(wu, dev),
                     to_dev(wd, dev), E, H, FF).cpu().numpy()
    ok, worst = close_moe(got, oracle.moe_ffn(x, ids, wts, wg, wu, wd, E, H, FF))
    assert ok, worst


@pytest.mark.parametrize("S", [1, 16])
def test_moe_full_config(tc, dev, oracle, S):
    """qwen35moe-style experts at full size: 128 experts, top-8, hidden 2048,
    ff 768, Q4_K weights N(0,1) from the GPU encoder (the reference Q4_K
    quantizer, bit-exact port)."""
    import torch
    E, K, H, FF = 128, 8, 2048, 768
    gen = torch.Generator(device=dev).manual_seed(100 + S)

    def enc(rows, cols):
        return tc.encode(Q4_K, torch.randn((rows, cols), generator=gen, device=dev))

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    rng = np.random.default_rng(200 + S)
    ids, wts = routing(rng, S, E, K)
    x = rng.standard_normal((S, H)).astype(np.float32)
    got = tc.moe_ffn(to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), wg, wu, wd, E, H, FF).cpu().numpy()
    ref = oracle.moe_ffn(x, ids, wts, wg.cpu().numpy(), wu.cpu().numpy(), wd.cpu().numpy(), E, H, FF)
    ok, worst = close_moe(got, ref)
    assert ok, worst


def moe_counts(got, ref, step):
    """(outputs past the strict 1e-3 relative / 1e-4 absolute bar, outputs
    past the token-RMS floor, tokens with an output past the floor, outputs
    past floor + one h quantization step)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=1, keepdims=True))
    err = np.abs(got - ref)
    strict = 1e-4 + 1e-3 * np.abs(ref)
    floored = 1e-4 + 1e-3 * np.maximum(np.abs(ref), 1e-3 * rms)
    over = err > floored
    return (int((err > strict).sum()), int(over.sum()), int(over.any(axis=1).sum()),
            int((err > floored + step).sum()))


@pytest.mark.parametrize("S", [1, 16])
@pytest.mark.parametrize("path", ["pairs", "grouped"])
def test_moe_cfg5_relaxation_counts(tc, dev, oracle, S, path):
    """Config 5 at full size on both paths, with the relaxations of the bar
    counted and bounded per run: at most 0.1% of outputs past the strict bar
    (all of them within the token-RMS floor), and at most one token whose
    outputs move by a one-step flip of the requantized h (0 on the per-pair
    path, which quantizes h with the reference rule from the same fp32 sums
    layout)."""
    import torch
    E, K, H, FF = 128, 8, 2048, 768
    gen = torch.Generator(device=dev).manual_seed(300 + S)

    def enc(rows, cols):
        return tc.encode(Q4_K, torch.randn((rows, cols), generator=gen, device=dev))

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    rng = np.random.default_rng(400 + S)
    ids, wts = routing(rng, S, E, K)
    x = rng.standard_normal((S, H)).astype(np.float32)
    args = [to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), wg, wu, wd, E, H, FF]
    got = run_path(tc, args, 0 if path == "grouped" else 1 << 30)
    wgh, wuh, wdh = wg.cpu().numpy(), wu.cpu().numpy(), wd.cpu().numpy()
    ref = oracle.moe_ffn(x, ids, wts, wgh, wuh, wdh, E, H, FF)
    step = h_step_bound(oracle, x, ids, wts, wgh, wuh, wdh, E, H, FF)
    n_strict, n_floor, n_tok, n_step = moe_counts(got, ref, step)
    msg = (f"{path} S={S}: {n_strict} of {got.size} outputs past the strict bar, {n_floor} past the RMS floor "
           f"({n_tok} tokens), {n_step} past floor + one h step")
    print(msg)
    assert n_strict <= max(1, got.size // 1000), msg
    assert n_step == 0, msg
    assert n_tok <= 1, msg
    if path == "pairs":
        assert n_floor == 0, msg


# ---- grouped path: device-side routing + one grouped MFMA GEMM per matrix ----------

GEMM_MIN = 40  # the library's default


@pytest.fixture
def grouped(tc):
    """Force the grouped-GEMM path for every token count; restore afterwards."""
    tc.lib.tc_moe_set_gemm_min_tokens(0)
    yield
    tc.lib.tc_moe_set_gemm_min_tokens(GEMM_MIN)


def run_path(tc, args, gemm_min):
    tc.lib.tc_moe_set_gemm_min_tokens(gemm_min)
    try:
        return tc.moe_ffn(*args).cpu().numpy()
    finally:
        tc.lib.tc_moe_set_gemm_min_tokens(GEMM_MIN)


@pytest.mark.parametrize("S", [1, 3, 40, 150])
def test_moe_grouped_vs_oracle(tc, dev, oracle, grouped, S):
    """Expert-sorted rows; invalid ids (-1, E) skipped; segments of every size
    (1 row up to several 128-row tiles per expert)."""
    E, K, H, FF = 16, 4, 1024, 512
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed=61 + S)
    rng = np.random.default_rng(70 + S)
    ids, wts = routing(rng, S, E, K)
    ids[0, 0] = -1
    if S > 1:
        ids[1, K - 1] = E
    x = rng.standard_normal((S, H)).astype(np.float32)
    args = [to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), to_dev(wg, dev), to_dev(wu, dev), to_dev(wd, dev),
            E, H, FF]
    got = tc.moe_ffn(*args).cpu().numpy()
    ok, worst = close_moe_flips(got, oracle.moe_ffn(x, ids, wts, wg, wu, wd, E, H, FF),
                                h_step_bound(oracle, x, ids, wts, wg, wu, wd, E, H, FF))
    assert ok, worst
    again = tc.moe_ffn(*args).cpu().numpy()
    assert np.array_equal(got, again)  # an expert's rows take pair order: repeated calls agree bit for bit


def test_moe_grouped_deterministic_many_tiles(tc, dev, grouped):
    """Config-5 experts at 1024 tokens (~64 rows per expert, so experts span
    two 64-row tiles whose K ranges split differently): a row's tile decides
    the rounding of its sums, so the rows of an expert must land in a fixed
    order. Three calls agree bit for bit."""
    import torch
    E, K, H, FF, S = 128, 8, 2048, 768, 1024
    gen = torch.Generator(device=dev).manual_seed(777)

    def enc(rows, cols):
        return tc.encode(Q4_K, torch.randn((rows, cols), generator=gen, device=dev) * 0.02)

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    ids, wts = routing(np.random.default_rng(778), S, E, K)
    x = torch.randn((S, H), generator=gen, device=dev)
    args = [x, to_dev(ids, dev), to_dev(wts, dev), wg, wu, wd, E, H, FF]
    first = tc.moe_ffn(*args).cpu().numpy()
    for _ in range(2):
        assert np.array_equal(first, tc.moe_ffn(*args).cpu().numpy())


def test_moe_grouped_large_routing(tc, dev):
    """2100 tokens x top-8 over 128 experts: more pairs than the router keeps
    in LDS (ids read from memory) and token bitmaps too large for LDS (the
    counting fallback). Checked against the per-pair mat-vec path (itself held
    to the oracle): every row routed, in a fixed order."""
    import torch
    E, K, H, FF, S = 128, 8, 256, 256, 2100
    gen = torch.Generator(device=dev).manual_seed(555)

    def enc(rows, cols):
        return tc.encode(Q4_K, torch.randn((rows, cols), generator=gen, device=dev) * 0.02)

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    ids, wts = routing(np.random.default_rng(556), S, E, K)
    x = torch.randn((S, H), generator=gen, device=dev)
    args = [x, to_dev(ids, dev), to_dev(wts, dev), wg, wu, wd, E, H, FF]
    got = run_path(tc, args, 0)
    assert np.array_equal(got, run_path(tc, args, 0))
    ref = run_path(tc, args, 1 << 30)
    # per token: the grouped path differs from the per-pair one only by the
    # rounding of its sums and rare one-step flips of h's requantization
    err = np.abs(got - ref).max(axis=1) / (np.sqrt((ref ** 2).mean(axis=1)) + 1e-30)
    assert np.median(err) < 1e-3 and err.max() < 0.1, (np.median(err), err.max())


def test_moe_grouped_repeated_expert(tc, dev, oracle, grouped):
    """An expert named twice for one token (the router never does this; the
    kernel's fallback row assignment): both pairs computed, as the oracle
    does, and repeated calls agree."""
    E, K, H, FF, S = 8, 4, 512, 256, 40
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed=91)
    rng = np.random.default_rng(92)
    ids, wts = routing(rng, S, E, K)
    ids[0, 1] = ids[0, 0]
    ids[7, 3] = ids[7, 2]
    x = rng.standard_normal((S, H)).astype(np.float32)
    args = [to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), to_dev(wg, dev), to_dev(wu, dev), to_dev(wd, dev),
            E, H, FF]
    got = tc.moe_ffn(*args).cpu().numpy()
    ok, worst = close_moe_flips(got, oracle.moe_ffn(x, ids, wts, wg, wu, wd, E, H, FF),
                                h_step_bound(oracle, x, ids, wts, wg, wu, wd, E, H, FF))
    assert ok, worst
    assert np.array_equal(got, tc.moe_ffn(*args).cpu().numpy())


def test_moe_grouped_all_ids_invalid(tc, dev, oracle, grouped):
    E, K, H, FF, S = 4, 2, 512, 256, 5
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed=3)
    ids = np.full((S, K), E, np.int32)
    ids[2, 1] = -7
    wts = np.full((S, K), 0.5, np.float32)
    x = np.random.default_rng(1).standard_normal((S, H)).astype(np.float32)
    got = tc.moe_ffn(to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), to_dev(wg, dev), to_dev(wu, dev),
                     to_dev(wd, dev), E, H, FF).cpu().numpy()
    assert (got == 0).all()


def test_moe_grouped_full_config(tc, dev, oracle):
    """128 experts, top-8, hidden 2048, ff 768 at 96 tokens (768 rows): the
    grouped GEMM checked against the oracle and, with the per-pair mat-vec
    path, both against it."""
    import torch
    E, K, H, FF, S = 128, 8, 2048, 768, 96
    gen = torch.Generator(device=dev).manual_seed(4242)

    def enc(rows, cols):
        return tc.encode(Q4_K, torch.randn((rows, cols), generator=gen, device=dev))

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    rng = np.random.default_rng(4243)
    ids, wts = routing(rng, S, E, K)
    x = rng.standard_normal((S, H)).astype(np.float32)
    args = [to_dev(x, dev), to_dev(ids, dev), to_dev(wts, dev), wg, wu, wd, E, H, FF]
    got = run_path(tc, args, 0)
    wgh, wuh, wdh = wg.cpu().numpy(), wu.cpu().numpy(), wd.cpu().numpy()
    ref = oracle.moe_ffn(x, ids, wts, wgh, wuh, wdh, E, H, FF)
    step = h_step_bound(oracle, x, ids, wts, wgh, wuh, wdh, E, H, FF)
    ok, worst = close_moe_flips(got, ref, step)
    assert ok, worst
    pairs = run_path(tc, args, 1 << 30)
    ok, worst = close_moe_flips(pairs, ref, step)
    assert ok, worst


# ---- the router (ModelMoE.cpp:341-425) --------------------------------------------------
# Bar: logits, expert ids and weights bit-exact (integer/index work, the
# CPU's own FMA order, and the same IEEE divisions of the same values).

def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_router_golden(tc, dev, golden):
    """The compiled reference's logits (its F32 AVX2 kernel, a width with a
    4-column tail) and its selection on them, for 1 and 16 tokens, k = 1, 8
    and 10."""
    w, x = golden["router_w"], golden["router_x"]
    wd = to_dev(w, dev)
    for tag, xs in (("1", x[:1]), ("16", x)):
        for k in (1, 8, 10):
            lg, ids, wts = tc.moe_router(wd, to_dev(xs, dev), k)
            assert (_bits(lg.cpu().numpy()) == _bits(golden[f"router_logits{tag}"])).all(), tag
            n = xs.shape[0]
            assert (ids.cpu().numpy() == golden[f"router_sel{k}_ids"][:n]).all(), (tag, k)
            assert (_bits(wts.cpu().numpy()) == _bits(golden[f"router_sel{k}_wts"][:n])).all(), (tag, k)


@pytest.mark.parametrize("k", [1, 8, 10])
def test_router_selection_ties_golden(tc, dev, golden, k):
    """Tie-heavy logits (multiples of 1/4): equal probabilities come out in
    std::partial_sort's order, exactly as the reference's selection."""
    cases = [("ties", golden["router_ties"])] + ([("wide", golden["router_wide"])] if k == 8 else [])
    for name, lg in cases:
        ids, wts = tc.moe_select(to_dev(lg, dev), k)
        assert (ids.cpu().numpy() == golden[f"router_{name}{k}_ids"]).all(), name
        assert (_bits(wts.cpu().numpy()) == _bits(golden[f"router_{name}{k}_wts"])).all(), name


@pytest.mark.parametrize("S", [1, 16, 300])
def test_router_cfg5_vs_oracle(tc, dev, oracle, S):
    """Config 5's router shape (128 experts, hidden 2048, top 8) against the
    oracle: logits, ids and weights bit for bit."""
    rng = np.random.default_rng(S)
    E, H, K = 128, 2048, 8
    w = (rng.standard_normal((E, H)) * 0.03).astype(np.float32)
    x = rng.standard_normal((S, H)).astype(np.float32)
    lg, ids, wts = tc.moe_router(to_dev(w, dev), to_dev(x, dev), K)
    rl = oracle.matmul_f32(w, x, E, H)
    assert (_bits(lg.cpu().numpy()) == _bits(rl)).all()
    rids, rwts = oracle.moe_route(rl, K)
    assert (ids.cpu().numpy() == rids).all()
    assert (_bits(wts.cpu().numpy()) == _bits(rwts)).all()


def test_router_feeds_moe_ffn(tc, dev, oracle):
    """Router on the device feeding the expert FFN with no host round trip:
    the ids and weights the FFN consumes are the oracle router's, and the
    output is the oracle composition's within the MoE bar."""
    E, K, H, FF, S = 16, 4, 1024, 512, 6
    rng = np.random.default_rng(77)
    wg, wu, wd = moe_weights(lambda x: oracle.encode(Q4_K, x), E, H, FF, seed=77)
    wr = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    x = rng.standard_normal((S, H)).astype(np.float32)
    xd = to_dev(x, dev)
    _, ids, wts = tc.moe_router(to_dev(wr, dev), xd, K)
    got = tc.moe_ffn(xd, ids, wts, to_dev(wg, dev), to_dev(wu, dev), to_dev(wd, dev), E, H, FF).cpu().numpy()
    rids, rwts = oracle.moe_route(oracle.matmul_f32(wr, x, E, H), K)
    assert (ids.cpu().numpy() == rids).all()
    ref = oracle.moe_ffn(x, rids, rwts, wg, wu, wd, E, H, FF)
    ok, msg = close_moe(got, ref)
    assert ok, msg


def test_router_refuses_bad_arguments(tc, dev):
    import torch
    from tc_hip import TC_E_ARG, _ptr
    lg = torch.zeros((2, 8), device=dev)
    ids = torch.full((2, 9), -7, dtype=torch.int32, device=dev)
    wts = torch.zeros((2, 9), device=dev)
    assert tc.lib.tc_moe_select(_ptr(lg), 2, 8, 9, _ptr(ids), _ptr(wts), None) == TC_E_ARG  # top_k > n_experts
    assert tc.lib.tc_moe_select(_ptr(lg), 2, 8, 0, _ptr(ids), _ptr(wts), None) == TC_E_ARG
    torch.cuda.synchronize()
    assert (ids.cpu() == -7).all()
