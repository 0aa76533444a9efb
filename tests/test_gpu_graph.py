"""HIP graph capture of the entry points (after one eager call has sized the
scratch, as tc_gemv_reserve documents): every replay, with eager work and
synchronizations between replays, must reproduce the eager results bit for
bit."""
import numpy as np
import pytest

from qdata import Q4_K, Q8_0, gaussian, random_blocks

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_graph_replays_match_eager(tc, dev):
    import torch
    import tc_hip
    rng = np.random.default_rng(21)
    rows, cols, M = 700, 2048, 40
    w4 = to_dev(random_blocks(Q4_K, rng, rows, cols), dev)
    wu = to_dev(random_blocks(Q4_K, rng, rows, cols), dev)
    w8 = to_dev(random_blocks(Q8_0, rng, rows, cols), dev)
    x1 = to_dev(gaussian(rng, (1, cols)), dev)
    xm = to_dev(gaussian(rng, (M, cols)), dev)
    outs = {k: torch.empty(shape, device=dev) for k, shape in
            (("gemv", (1, rows)), ("g", (1, rows)), ("u", (1, rows)), ("q8", (1, rows)), ("gemm", (M, rows)),
             ("gemm8", (M, rows)))}

    def work():
        tc.gemv(Q4_K, w4, x1, rows, cols, out=outs["gemv"])
        tc._check(tc.lib.tc_gemv_dual(Q4_K, tc_hip._ptr(w4), tc_hip._ptr(wu), tc_hip._ptr(x1), tc_hip._ptr(outs["g"]),
                                      tc_hip._ptr(outs["u"]), rows, cols, tc._stream()))
        tc.gemv(Q8_0, w8, x1, rows, cols, out=outs["q8"])
        tc.gemm(Q4_K, w4, xm, rows, cols, out=outs["gemm"])
        tc.gemm(Q8_0, w8, xm, rows, cols, out=outs["gemm8"])

    work()  # sizes the scratch
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in outs.items()}
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            work()
    torch.cuda.synchronize()
    for rep in range(3):
        for v in outs.values():
            v.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in outs:
            assert torch.equal(outs[k], ref[k]), (rep, k)
