"""Benchmark of the quantized mat-vec hot path on one MI355X.

Default workload (BASELINE config #2): one Qwen2.5-7B-shaped decoder layer of
Q4_K decode mat-vecs at batch 1 -- q 3584x3584, k/v 512x3584, o 3584x3584,
gate/up 18944x3584, down 3584x18944 -- with weights drawn from N(0, 0.02)
and quantized by the reference's own Q4_K quantizer (bit-exact GPU port),
activations N(0, 1). A step is one pass over the layer in decode order, as 4
launches: q/k/v in one launch on the shared input, o, gate/up as a pair with
the SwiGLU epilogue, down (each launch quantizes its input in-kernel), issued
as HIP graph replays of 8 steps (the eager 4-launch sequence is timed
beside it). The weights of 8 identical layer copies are rotated step by
step (1.05 GB working set) so that the 256 MB Infinity Cache cannot serve them.

Prints one JSON line. `value` is whole-step weight+activation bytes per
second (GB/s); `roofline` is the step's largest launch (the gate/up pair),
its average duration timed with HIP events around back-to-back launches on the
stream it runs on, its HBM traffic read from the committed rocprofv3 summary; `cpu_baseline` is the reference's own AVX2
kernel (compiled from its sources, oracle/_ref) on the host cores.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tinycoder-inference_amd"))

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K decode GEMV GB/s (% HBM peak) at batch 1; int8 prefill GEMM TOPS"
LAYER = [("q", 3584, 3584), ("k", 512, 3584), ("v", 512, 3584), ("o", 3584, 3584),
         ("gate", 18944, 3584), ("up", 18944, 3584), ("down", 3584, 18944)]
# activation groups: matrices that read the same input vector
GROUPS = [("attn", 3584, ["q", "k", "v"]), ("o_in", 3584, ["o"]), ("ffn", 3584, ["gate", "up"]),
          ("down_in", 18944, ["down"])]
N_COPIES = 8


def algorithmic_bytes(rows, cols, row_bytes):
    # weights + fp32 activation read + fp32 output write, per mat-vec
    return rows * row_bytes + 4 * cols + 4 * rows


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gate_up_pair_18944x3584_pmc.md")


def measured_traffic():
    """HBM bytes per gate/up launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-kernel calibrated), or None if absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def host_cpu_info():
    """CPU model, SIMD level and the CPUs this process may run on (`nproc`), read
    from /proc/cpuinfo and the scheduler affinity (lscpu reads the same)."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    simd = ("avx512f+avx512bw" if {"avx512f", "avx512bw"} <= flags else "avx2" if "avx2" in flags else "sse")
    if "amx_int8" in flags:
        simd += "+amx"
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()
            if q != "max":
                quota = round(int(q) / int(per), 2)
    except (OSError, ValueError):
        pass
    return model, simd, nproc, quota


def cpu_baseline(weights_host, xs_host, row_bytes):
    """The reference's CPU kernel (matMulVecBatchQ4K_Q8K_AVX2 through its
    ThreadPool, compiled from its sources; the C port if that build is absent)
    over full layer passes for a bounded ~8 s sample. Threads: TINYCODER_THREADS
    if set, else `nproc` (the reference's ThreadPool::recommendedThreadCount,
    ThreadPool.cpp:68-94, counts the online CPUs; `nproc` counts the ones this
    process may use). The pass rotates over N_COPIES copies of the layer's
    weights (1.05 GB), so the host's last-level cache cannot serve them."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    model, simd, nproc, quota = host_cpu_info()
    env = os.environ.get("TINYCODER_THREADS", "")
    threads = int(env) if env.isdigit() and int(env) > 0 else nproc
    try:
        impl = O.Reference(threads=threads)
        kind = "reference"
        threads = impl.threads
    except (FileNotFoundError, OSError):
        impl = O.Oracle()
        kind = "port"
        threads = 1
    copies = [{n: weights_host[n].copy() for n in weights_host} for _ in range(N_COPIES)]
    outs = {n: np.zeros((1, r), np.float32) for n, r, _ in LAYER}
    xmap = {}
    for g, _, names in GROUPS:
        for n in names:
            xmap[n] = xs_host[g]

    def one_pass(i):
        w = copies[i % N_COPIES]
        for n, r, c in LAYER:
            if kind == "reference":
                impl.matmul(12, w[n], xmap[n], r, c, out=outs[n])
            else:
                outs[n][:] = impl.matmul(12, w[n], xmap[n], r, c)

    for i in range(N_COPIES):
        one_pass(i)
    t0 = time.perf_counter()
    reps = 0
    while True:
        one_pass(reps)
        reps += 1
        el = time.perf_counter() - t0
        if (el > 8.0 and reps >= N_COPIES) or reps >= 4000:
            break
    per_pass = sum(algorithmic_bytes(r, c, row_bytes(12, c)) for _, r, c in LAYER)
    impl_name = ("reference AVX2 matMulVecBatchQ4K_Q8K_AVX2 + ThreadPool" if kind == "reference"
                 else "C port, 1 thread")
    return {"value": round(per_pass * reps / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "cpu_model": model, "simd": simd, "nproc": nproc, "cgroup_cpu_quota": quota,
            "sample": f"{reps} full-layer passes (7 Q4_K mat-vecs, {per_pass / 1e6:.1f} MB each) over "
                      f"{N_COPIES} rotating weight copies in {el:.1f} s, {impl_name}, {threads} threads"}


GEMM_SHAPES = [(17408, 5120), (5120, 17408)]   # (rows N, cols K), out x in
GEMM_TOKENS = [128, 512, 2048]
GEMM_7B_SHAPES = [(18944, 3584), (3584, 18944)]   # qwen2.5-7b FFN up and down
INT8_PEAK_TOPS = 5000.0


def gemm_time(torch, tc, qt, N, K, Ms, gen, dev, reps):
    """Per-call time in us of tc_gemm (activation quantization + int8 MFMA GEMM
    [+ split-K reduce]) for each M in Ms: weights N(0,0.02) through the GPU
    encoder, rotating copies of at least 600 MB in all (beyond the 256 MB
    Infinity Cache); x ~ N(0,1)."""
    wf = torch.randn((N, K), generator=gen, device=dev) * 0.02
    w0 = tc.encode(qt, wf)
    del wf
    ncopy = max(4, -(-600_000_000 // (w0.numel())))
    ws = [w0] + [w0.clone() for _ in range(ncopy - 1)]
    times = []
    for M in Ms:
        x = torch.randn((M, K), generator=gen, device=dev)
        out = torch.empty((M, N), device=dev)
        for i in range(3):
            tc.gemm(qt, ws[i % ncopy], x, N, K, out=out)
        torch.cuda.synchronize()
        n = max(3, reps if M < 2048 else reps // 4)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(n):
            tc.gemm(qt, ws[i % ncopy], x, N, K, out=out)
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) * 1e3 / n)
    del ws, w0
    torch.cuda.empty_cache()
    return times


def gemm_bench(torch, tc, tc_hip, dev, reps):
    """Prefill GEMM at every M x shape x type. Returns one record per config."""
    gen = torch.Generator(device=dev).manual_seed(7)
    res = []
    legs = [(tc_hip.Q4_K, "Q4_K", GEMM_SHAPES), (tc_hip.Q8_0, "Q8_0", GEMM_SHAPES),
            (tc_hip.Q5_K, "Q5_K", GEMM_7B_SHAPES), (tc_hip.Q6_K, "Q6_K", GEMM_7B_SHAPES),
            (tc_hip.IQ3_XXS, "IQ3_XXS", GEMM_7B_SHAPES), (tc_hip.IQ3_S, "IQ3_S", GEMM_7B_SHAPES),
            (tc_hip.IQ2_S, "IQ2_S", GEMM_7B_SHAPES)]
    for qt, tname, shapes in legs:
        for N, K in shapes:
            for M, us in zip(GEMM_TOKENS, gemm_time(torch, tc, qt, N, K, GEMM_TOKENS, gen, dev, reps)):
                tops = 2.0 * M * N * K / us / 1e6
                res.append({"type": tname, "N": N, "K": K, "M": M, "us": round(us, 1), "TOPS": round(tops, 1),
                            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)})
    return res


# The only per-shape GEMM times the reference publishes (source comments,
# RTX 2080 Ti, seq 512): GemmDispatch.cu:522 (IQ3_XXS) and :533-536 (Q4_K).
REF_GEMM_POINTS = [("Q4_K", 18944, 3584, 1389.0), ("Q4_K", 3584, 18944, 1604.0), ("Q4_K", 3584, 3584, 341.0),
                   ("Q4_K", 512, 3584, 102.0), ("IQ3_XXS", 18944, 3584, 1724.0)]


def gemm_reference_points(torch, tc, tc_hip, dev, reps):
    """The reference's published int8 GEMM shapes at seq 512, timed here the
    same way, beside the reference's own figures (other hardware: a side
    comparison, not the headline vs_baseline)."""
    gen = torch.Generator(device=dev).manual_seed(11)
    out = []
    for tname, N, K, ref_us in REF_GEMM_POINTS:
        us = gemm_time(torch, tc, getattr(tc_hip, tname), N, K, [512], gen, dev, reps)[0]
        out.append({"type": tname, "N": N, "K": K, "M": 512, "us": round(us, 1),
                    "reference_us_rtx2080ti": ref_us, "speedup": round(ref_us / us, 1)})
    return out


def head_start(torch):
    """Keep the GPU busy for a bounded time (~25 ms) while the host queues the
    timed launches, so that events measure back-to-back GPU execution and not
    the Python launch rate."""
    try:
        torch.cuda._sleep(int(60e6))
    except (AttributeError, RuntimeError):
        pass


def timed(torch, fn, n):
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    fn(0)
    torch.cuda.synchronize()
    head_start(torch)
    a.record()
    for i in range(n):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / n


def roof_probes(torch, tc, tc_hip, dev):
    """What this part sustains, measured in the same run: the int8 MFMA rate
    from registers (tc_probe_mfma_i8), and the HBM read rate of a plain
    streaming kernel (tc_probe_read: non-temporal 16-byte loads, one
    contiguous chunk per workgroup, no decode work) over 2 GiB and at the
    byte counts of the decode launches (rotating buffers, back-to-back
    launches): the ceiling a single launch of that size can reach."""
    sink = torch.empty(tc.lib.tc_probe_sink_bytes(), dtype=torch.uint8, device=dev)
    st = tc._stream()
    wgs, iters = 2048, 2000
    mf = timed(torch, lambda i: tc._check(tc.lib.tc_probe_mfma_i8(wgs, iters, tc_hip._ptr(sink), st)), 5)
    mfma_tops = wgs * 4 * 4 * iters * 65536 / mf / 1e6
    read = {}
    for name, nbytes, nbuf in (("2GiB", 2 << 30, 1), ("gate_up", 76562432, 12), ("down", 38281216, 16),
                               ("o", 7254016, 32)):
        nbytes = nbytes // 16384 * 16384
        bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        best = 0.0
        for nwg in (256, 512, 1024):
            us = timed(torch, lambda i: tc._check(tc.lib.tc_probe_read(tc_hip._ptr(bufs[i % nbuf]), nbytes, nwg,
                                                                       tc_hip._ptr(sink), st)), 5 if nbuf == 1 else 60)
            best = max(best, nbytes / us / 1e3)
        read[name] = {"GB/s": round(best, 1), "frac": round(best / HBM_PEAK_GBS, 4)}
        del bufs
        torch.cuda.empty_cache()
    del sink
    return {"int8_mfma_TOPS": round(mfma_tops, 1), "hbm_read": read,
            "note": "tc_probe_mfma_i8: v_mfma_i32_32x32x32_i8 from registers, 4 chains x 2 waves per SIMD; "
                    "tc_probe_read: each buffer read once per launch, best of 256/512/1024 workgroups"}


def other_decode_bench(torch, tc, tc_hip, dev, reps):
    """BASELINE configs #1 and #3 (batch-1 decode mat-vecs of other formats), and
    Q5_K, Q3_K, Q2_K, IQ3_S, IQ2_S, IQ2_XS, IQ4_XS, IQ4_NL and Q5_0 at the 7B FFN shape:
    weights N(0,0.02) through the GPU encoders, rotating copies so that every
    working set exceeds the 256 MB Infinity Cache."""
    gen = torch.Generator(device=dev).manual_seed(11)
    rb = tc_hip.row_bytes
    cases = [("cfg1 Q8_0 4096x4096", tc_hip.Q8_0, 4096, 4096, False, 16),
             ("cfg3 Q6_K LM head 152064x3584", tc_hip.Q6_K, 152064, 3584, False, 1),
             ("cfg3 Q6_K down 3584x18944", tc_hip.Q6_K, 3584, 18944, False, 6),
             ("cfg3 IQ3_XXS gate/up pair 18944x3584 (SwiGLU)", tc_hip.IQ3_XXS, 18944, 3584, True, 6),
             ("Q5_K gate/up pair 18944x3584 (SwiGLU; format beyond the BASELINE configs)", tc_hip.Q5_K, 18944,
              3584, True, 6),
             ("Q3_K gate/up pair 18944x3584 (SwiGLU; format beyond the BASELINE configs)", tc_hip.Q3_K, 18944,
              3584, True, 8),
             ("IQ3_S gate/up pair 18944x3584 (SwiGLU; format beyond the BASELINE configs)", tc_hip.IQ3_S, 18944,
              3584, True, 8),
             ("IQ2_S gate/up pair 18944x3584 (SwiGLU; format beyond the BASELINE configs)", tc_hip.IQ2_S, 18944,
              3584, True, 8),
             ("Q2_K gate/up pair 18944x3584 (SwiGLU; format beyond the BASELINE configs)", tc_hip.Q2_K, 18944,
              3584, True, 8),
             ("IQ2_XS gate/up pair 18944x3584 (SwiGLU, fp32 x: int8GemvDualIQ2XS)", tc_hip.IQ2_XS, 18944,
              3584, True, 8),
             ("IQ4_XS gate/up pair 18944x3584 (SwiGLU; format beyond the BASELINE configs)", tc_hip.IQ4_XS, 18944,
              3584, True, 6),
             ("IQ4_NL gate/up pair 18944x3584 (SwiGLU, fp32 x; format beyond the BASELINE configs)", tc_hip.IQ4_NL,
              18944, 3584, True, 6),
             ("Q5_0 gate/up pair 18944x3584 (SwiGLU, fp32 x; format beyond the BASELINE configs)", tc_hip.Q5_0,
              18944, 3584, True, 6)]
    res = []
    for name, qt, rows, cols, dual, ncopy in cases:
        mats = 2 if dual else 1
        ws = []
        for _ in range(mats):
            wf = torch.randn((rows, cols), generator=gen, device=dev) * 0.02
            ws.append(tc.encode(qt, wf))
            del wf
        copies = [[w if c == 0 else w.clone() for w in ws] for c in range(ncopy)]
        x = torch.randn((1, cols), generator=gen, device=dev)
        out = torch.empty((1, rows), device=dev)
        out2 = torch.empty((1, rows), device=dev)

        def fn(i):
            c = copies[i % ncopy]
            if dual:
                tc.lib.tc_gemv_dual(qt, tc_hip._ptr(c[0]), tc_hip._ptr(c[1]), tc_hip._ptr(x), tc_hip._ptr(out),
                                    tc_hip._ptr(out2), rows, cols, tc._stream())
            else:
                tc.gemv(qt, c[0], x, rows, cols, out=out)

        us = timed(torch, fn, reps)
        by = mats * rows * rb(qt, cols) + 4 * cols + 4 * rows * mats
        res.append({"config": name, "us": round(us, 2), "bytes": by, "GB/s": round(by / us / 1e3, 1),
                    "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4)})
        del copies, ws
        torch.cuda.empty_cache()
    return res


def moe_bench(torch, tc, tc_hip, dev, reps):
    """BASELINE config #5: 128 Q4_K experts (gate/up 768x2048, down 2048x768,
    W ~ N(0,0.02) through the reference Q4_K quantizer), top-8 routing uniform
    without replacement, softmax(N(0,1)) weights, batch 1 and 16. A fresh
    routing per repetition (so a repeated expert set cannot sit in the
    Infinity Cache); bytes = distinct experts of that routing x 2,654,208."""
    E, K, H, FF = 128, 8, 2048, 768
    gen = torch.Generator(device=dev).manual_seed(13)

    def enc(r, c):
        return tc.encode(tc_hip.Q4_K, torch.randn((r, c), generator=gen, device=dev) * 0.02)

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    per_expert = 3 * FF * (H // 256) * 144
    rng = np.random.default_rng(17)
    res = []
    for T in (1, 16):
        ids_l, wts_l, nbytes = [], [], []
        for _ in range(reps):
            ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
            lg = rng.standard_normal((T, K)).astype(np.float32)
            w = np.exp(lg) / np.exp(lg).sum(1, keepdims=True)
            ids_l.append(torch.from_numpy(ids).to(dev))
            wts_l.append(torch.from_numpy(w.astype(np.float32)).to(dev))
            nbytes.append(len(np.unique(ids)) * per_expert)
        x = torch.randn((T, H), generator=gen, device=dev)
        out = torch.empty((T, H), device=dev)

        def fn(i):
            tc.moe_ffn(x, ids_l[i % reps], wts_l[i % reps], wg, wu, wd, E, H, FF, out=out)

        us = timed(torch, fn, reps)
        by = float(np.mean(nbytes)) + 4 * T * H * 2
        res.append({"batch": T, "us": round(us, 2), "bytes": int(by), "GB/s": round(by / us / 1e3, 1),
                    "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4), "launches": 2})
    del wg, wu, wd
    torch.cuda.empty_cache()
    return res


def moe_prefill_bench(torch, tc, tc_hip, dev, reps):
    """MoE prefill (the reference's moeBatchExperts case, MoeBatch.cu:37-197)
    at the config-5 expert shapes: T tokens x top-8, routed on the device,
    each matrix one grouped int8 MFMA GEMM over all experts ("gemm"); beside
    it the per-(token, rank) mat-vec path ("pairs") on the same inputs (the
    library takes the GEMM from 40 tokens). TOPS = 2 * T * 8 *
    3 * 768 * 2048 int8 ops / time (the whole FFN, router and combine
    included)."""
    E, K, H, FF = 128, 8, 2048, 768
    gen = torch.Generator(device=dev).manual_seed(19)

    def enc(r, c):
        return tc.encode(tc_hip.Q4_K, torch.randn((r, c), generator=gen, device=dev) * 0.02)

    wg, wu, wd = enc(E * FF, H), enc(E * FF, H), enc(E * H, FF)
    rng = np.random.default_rng(23)
    res = []
    for T in (16, 64, 256, 1024):
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        lg = rng.standard_normal((T, K)).astype(np.float32)
        w = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
        idd, wd_ = torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)
        x = torch.randn((T, H), generator=gen, device=dev)
        out = torch.empty((T, H), device=dev)
        ops = 2.0 * T * K * 3 * FF * H
        row = {"tokens": T}
        for name, thr in (("gemm", 0), ("pairs", 1 << 30)):
            tc.lib.tc_moe_set_gemm_min_tokens(thr)
            us = timed(torch, lambda i: tc.moe_ffn(x, idd, wd_, wg, wu, wd, E, H, FF, out=out), reps)
            row[name] = {"us": round(us, 1), "TOPS": round(ops / us / 1e6, 1)}
        tc.lib.tc_moe_set_gemm_min_tokens(40)
        res.append(row)
    del wg, wu, wd
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM leg")
    ap.add_argument("--no-other", action="store_true", help="skip the other-format decode and MoE legs")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="counter-collection run: a 256 MiB device copy (the calibration kernel of known "
                         "traffic), then --steps passes over the layer's launches; prints nothing else")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported by this build "
              "(the hot path runs on one GPU: each GPU of a sharded deployment would run this same "
              "single-GPU launch on its own shard of the weight rows)", file=sys.stderr)
        sys.exit(2)

    import torch
    import tc_hip

    dev = torch.device("cuda:0")
    tc = tc_hip.Library()
    Q4K = tc_hip.Q4_K
    gen = torch.Generator(device=dev).manual_seed(20261201)

    # ---- weights: encode once, replicate into rotating copies --------------------
    base = {}
    for n, r, c in LAYER:
        wf = torch.randn((r, c), generator=gen, device=dev) * 0.02
        base[n] = tc.encode(Q4K, wf)
        del wf
    copies = [{n: base[n].clone() for n in base} for _ in range(N_COPIES)]
    xs = {g: torch.randn((1, c), generator=gen, device=dev) for g, c, _ in GROUPS}
    outs = {n: torch.empty((1, r), device=dev) for n, r, _ in LAYER}
    dims = {n: (r, c) for n, r, c in LAYER}
    torch.cuda.synchronize()

    h_out = torch.empty((1, 18944), device=dev)
    u_out = torch.empty((1, 18944), device=dev)
    LAUNCHES = [("qkv", ["q", "k", "v"]), ("o", ["o"]), ("gate_up", ["gate", "up"]), ("down", ["down"])]

    def launch(name, ws):
        if name == "qkv":
            tc.gemv_multi(Q4K, [ws["q"], ws["k"], ws["v"]], [xs["attn"]] * 3, [3584, 512, 512], [3584] * 3,
                          outs=[outs["q"], outs["k"], outs["v"]])
        elif name == "o":
            tc.gemv(Q4K, ws["o"], xs["o_in"], 3584, 3584, out=outs["o"])
        elif name == "gate_up":
            tc.lib.tc_gemv_dual(Q4K, tc_hip._ptr(ws["gate"]), tc_hip._ptr(ws["up"]), tc_hip._ptr(xs["ffn"]),
                                tc_hip._ptr(h_out), tc_hip._ptr(u_out), 18944, 3584, tc._stream())
        else:
            tc.gemv(Q4K, ws["down"], xs["down_in"], 3584, 18944, out=outs["down"])

    def step(i):
        ws = copies[i % N_COPIES]
        for name, _ in LAUNCHES:
            launch(name, ws)

    def step_one_launch(i):
        ws = copies[i % N_COPIES]
        names = [n for n, _, _ in LAYER]
        xin = {"q": "attn", "k": "attn", "v": "attn", "o": "o_in", "gate": "ffn", "up": "ffn", "down": "down_in"}
        tc.gemv_multi(Q4K, [ws[n] for n in names], [xs[xin[n]] for n in names], [dims[n][0] for n in names],
                      [dims[n][1] for n in names], outs=[outs[n] for n in names])

    for i in range(args.warmup):
        step(i)
        step_one_launch(i)
    torch.cuda.synchronize()

    if args.pmc_probe:
        # Calibration: one copy kernel that reads and writes exactly 256 MiB.
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        for i in range(args.steps):
            step(i)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": True, "copy_bytes": 2 * src.numel() * 4, "steps": args.steps}), flush=True)
        return

    # ---- the steps as HIP graphs -----------------------------------------------------
    # One graph holds N_COPIES consecutive steps (one per weight copy, 4
    # launches each), captured after the warm-up (which sized every scratch
    # buffer, so nothing allocates under capture); K steps are K // N_COPIES
    # replays of it plus single-step graphs for the remainder. This is how a
    # serving loop issues decode steps; the eager launch sequence is timed
    # beside it.
    cap_stream = torch.cuda.Stream()
    cap_stream.wait_stream(torch.cuda.current_stream())
    one = []
    with torch.cuda.stream(cap_stream):
        block = torch.cuda.CUDAGraph()
        with torch.cuda.graph(block, stream=cap_stream):
            for c in range(N_COPIES):
                step(c)
        for c in range(N_COPIES):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap_stream):
                step(c)
            one.append(g)
    torch.cuda.current_stream().wait_stream(cap_stream)
    torch.cuda.synchronize()
    block.replay()
    for g in one:
        g.replay()
    torch.cuda.synchronize()

    def graph_steps(k):
        for _ in range(k // N_COPIES):
            block.replay()
        for c in range(k % N_COPIES):
            one[c].replay()

    # ---- timed region: K steps ------------------------------------------------------
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    head_start(torch)
    t_start.record()
    graph_steps(args.steps)
    t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)

    # the same K steps issued eagerly (4 launches each from the host)
    e_start = torch.cuda.Event(enable_timing=True)
    e_end = torch.cuda.Event(enable_timing=True)
    head_start(torch)
    e_start.record()
    for i in range(args.steps):
        step(i)
    e_end.record()
    torch.cuda.synchronize()
    eager_ms_per_step = e_start.elapsed_time(e_end) / args.steps

    # the same layer as one launch (7 independent mat-vecs, one kernel)
    t1s = torch.cuda.Event(enable_timing=True)
    t1e = torch.cuda.Event(enable_timing=True)
    head_start(torch)
    t1s.record()
    for i in range(args.steps):
        step_one_launch(i)
    t1e.record()
    torch.cuda.synchronize()
    one_launch_ms = t1s.elapsed_time(t1e) / args.steps

    # ---- per-launch kernel durations ----------------------------------------------------
    # Each launch kind alone, K back-to-back launches over the rotating copies
    # between two events on the launch stream (the kernels run back to back,
    # so total / K is the kernel's average duration).
    rb = tc_hip.row_bytes
    per_launch = {}
    stream = torch.cuda.current_stream()
    for name, mats in LAUNCHES:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        head_start(torch)
        a.record(stream)
        for i in range(args.steps):
            launch(name, copies[i % N_COPIES])
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / args.steps
        by = sum(algorithmic_bytes(dims[m][0], dims[m][1], rb(Q4K, dims[m][1])) for m in mats)
        per_launch[name] = {"mats": mats, "bytes": by, "us": round(us, 2), "GB/s": round(by / us / 1e3, 1),
                            "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 3)}
    dom = per_launch["gate_up"]
    achieved = dom["bytes"] / dom["us"] / 1e3

    step_bytes = sum(algorithmic_bytes(r, c, rb(Q4K, c)) for _, r, c in LAYER)
    ms_per_step = total_ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    one_launch_gbs = step_bytes / (one_launch_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: W ~ N(0,0.02) -> reference Q4_K quantizer, x ~ N(0,1)",
        "config": {"workload": "qwen2.5-7b layer, Q4_K decode mat-vec, batch 1 (q,k,v,o,gate,up,down)",
                   "batch": 1, "weight_bytes_per_step": int(sum(r * rb(Q4K, c) for _, r, c in LAYER)),
                   "rotating_copies": N_COPIES, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "k_gemv_t<Q4_K,1,CfgBig> gate/up pair 2x18944x3584 with SwiGLU epilogue "
                               "(the step's largest launch); bytes = weights + x + both outputs per launch"},
        "step_issue": {"timed": f"HIP graph replays of {N_COPIES} steps (4 launches each), remainder as 1-step graphs",
                       "eager_ms_per_step": round(eager_ms_per_step, 4),
                       "eager_GB/s": round(step_bytes / (eager_ms_per_step * 1e-3) / 1e9, 1)},
        "per_launch": per_launch,
        "layer_one_launch": {"us": round(one_launch_ms * 1e3, 2), "GB/s": round(one_launch_gbs, 1),
                             "frac": round(one_launch_gbs / HBM_PEAK_GBS, 4)},
    }
    if not args.no_other:
        line["decode_other_formats"] = other_decode_bench(torch, tc, tc_hip, dev, max(20, args.steps // 2))
        line["moe"] = moe_bench(torch, tc, tc_hip, dev, max(20, args.steps // 2))
        line["moe_prefill"] = moe_prefill_bench(torch, tc, tc_hip, dev, 10)
    if not args.no_gemm:
        del copies
        torch.cuda.empty_cache()
        greps = max(10, args.steps // 4)
        g = gemm_bench(torch, tc, tc_hip, dev, greps)
        best = max(g, key=lambda r: r["TOPS"])
        line["prefill_gemm"] = {"unit": "TOPS (2*M*N*K / time, int8 MFMA; includes the activation quantizer)",
                                "peak_TOPS": INT8_PEAK_TOPS, "best": best, "configs": g,
                                "reference_shapes_seq512": gemm_reference_points(torch, tc, tc_hip, dev, greps)}
    line["roof_probes"] = roof_probes(torch, tc, tc_hip, dev)
    if not args.no_cpu:
        wh = {n: base[n].cpu().numpy() for n in base}
        xh = {g: xs[g].cpu().numpy() for g in xs}
        line["cpu_baseline"] = cpu_baseline(wh, xh, rb)
    # Compact per-config evidence as the line's last key, so that the tail of
    # stdout a driver keeps (a few KB) holds every BASELINE config.
    line["summary"] = summarize(line)
    print(json.dumps(line), flush=True)


def summarize(line):
    """Each BASELINE config's figures in short form: the decode step and its
    launches against the same-size read probes (cfg 2), the other decode
    formats (cfg 1, 3), the MoE expert FFN (cfg 5), and the prefill GEMM
    table (cfg 4: TOPS and us per type, shape and M)."""
    sm = {"cfg2_step": {"GB/s": line["value"], "frac": line["config"]["frac_of_hbm_peak"],
                        "us": round(line["ms_per_step"] * 1e3, 1)},
          "cfg2_per_launch_frac": {k: v["frac"] for k, v in line["per_launch"].items()},
          "cfg2_per_launch_us": {k: v["us"] for k, v in line["per_launch"].items()},
          "cfg2_layer_one_launch_frac": line["layer_one_launch"]["frac"]}
    rp = line.get("roof_probes")
    if rp:
        sm["read_probe_frac"] = {k: v["frac"] for k, v in rp["hbm_read"].items()}
        sm["mfma_probe_TOPS"] = rp["int8_mfma_TOPS"]
    if "decode_other_formats" in line:
        sm["cfg1_cfg3_frac"] = {r["config"].split(" (")[0]: r["frac"] for r in line["decode_other_formats"]
                                if r["config"].startswith("cfg")}
        sm["cfg5_moe_decode_frac"] = {f"batch{r['batch']}": r["frac"] for r in line["moe"]}
        sm["cfg5_moe_prefill_us"] = {f"T{r['tokens']}": [r["gemm"]["us"], r["pairs"]["us"]]
                                     for r in line["moe_prefill"]}
    if "prefill_gemm" in line:
        sm["cfg4_TOPS_us"] = {f"{r['type']} {r['N']}x{r['K']} M{r['M']}": [r["TOPS"], r["us"]]
                              for r in line["prefill_gemm"]["configs"] if r["type"] in ("Q4_K", "Q8_0")}
    if "cpu_baseline" in line:
        sm["cpu_baseline_GB/s"] = line["cpu_baseline"]["value"]
    return sm


if __name__ == "__main__":
    main()
