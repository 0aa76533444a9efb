"""GPU test of the GGUF reader feeding the kernels: tensors written to a GGUF
file (tests/gguf_write.py), read back with tc_gguf_open, uploaded with
tc_gguf_upload and multiplied with tc_gemv. The result must equal the same
kernel on the writer's bytes bit for bit, and the oracle within the fp32 bar
(1e-3 relative / 1e-4 absolute)."""
import numpy as np
import pytest

import gguf_write as W
from qdata import IQ3_XXS, Q4_K, Q5_K, Q6_K, Q8_0, close, gaussian

pytestmark = pytest.mark.gpu


def test_gguf_tensors_through_gemv(tc, dev, oracle, tmp_path):
    import tc_hip
    import torch
    rng = np.random.default_rng(808)
    cols = 1024
    specs = [("blk.0.attn_q.weight", Q4_K, 96), ("blk.0.attn_k.weight", Q5_K, 40),
             ("blk.0.ffn_down.weight", Q6_K, 72), ("blk.0.attn_v.weight", Q8_0, 24),
             ("blk.0.ffn_gate.weight", IQ3_XXS, 48)]
    tensors, host = [], {}
    for name, qt, rows in specs:
        w = oracle.encode(qt, gaussian(rng, (rows, cols), 1.0 if qt == Q4_K else 0.02))
        host[name] = w
        tensors.append((name, qt, (cols, rows), w))
    path = str(tmp_path / "m.gguf")
    W.write_gguf(path, [("general.architecture", W.STRING, "qwen2")], tensors)
    g = tc_hip.GGUFLoader(tc.lib)
    assert g.load(path), g.last_error
    x = gaussian(rng, (2, cols))
    xd = torch.from_numpy(x).to(dev)
    for name, qt, rows in specs:
        rec = g.getTensorInfo(name)
        assert rec.bytes == rows * tc.lib.tc_row_bytes(qt, cols)
        wd = g.upload(name, dev)
        got = tc.gemv(qt, wd, xd, rows, cols).cpu().numpy()
        same = tc.gemv(qt, torch.from_numpy(host[name]).to(dev), xd, rows, cols).cpu().numpy()
        assert np.array_equal(got, same), name
        ok, worst = close(got, oracle.matmul(qt, g.getTensor(name), x, rows, cols))
        assert ok, (name, worst)
    small = torch.empty(8, dtype=torch.uint8, device=dev)
    import ctypes
    rc = tc.lib.tc_gguf_upload(g.h, 0, ctypes.c_void_p(small.data_ptr()), 8, None)
    assert rc == tc_hip.TC_E_ARG
    g.close()
