"""CPU tests of the C-ABI boundary: the built library loads and exports every
function that include/*.h declares (no compute call without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(tc_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("tc_gemv", "tc_gemm", "tc_gemv_dual", "tc_moe_ffn", "tc_quantize_act", "tc_block_isums"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import tc_hip
    lib = tc_hip.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(tc_hip.SIGNATURES)


def test_no_device_is_reported_cleanly():
    import tc_hip
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = tc_hip.load_library()
    assert lib.tc_available() == 0
    rc = lib.tc_gemv(12, None, None, None, 1, 1, 256, None)
    assert rc == tc_hip.TC_E_UNSUPPORTED
    assert b"gfx950" in lib.tc_last_error()


def test_row_bytes():
    import tc_hip
    lib = tc_hip.load_library()
    assert lib.tc_row_bytes(12, 3584) == 14 * 144
    assert lib.tc_row_bytes(8, 4096) == 128 * 34
    assert lib.tc_row_bytes(14, 18944) == 74 * 210
    assert lib.tc_row_bytes(18, 3584) == 14 * 98
    assert lib.tc_row_bytes(11, 256) == 110
    assert lib.tc_row_bytes(10, 256) == 84
    assert lib.tc_row_bytes(9, 256) == 0  # Q8_1: not a weight type here


def test_type_ids_and_block_geometry():
    """The header's TC_* type ids are the binding's, and each type's row size
    is its GGUF block geometry as the GGUF reader's own table gives it (that
    table is checked against the reference loader in test_gguf.py). IQ2_XXS
    (16) and the reference's own formats are not weight types here."""
    import tc_hip
    lib = tc_hip.load_library()
    text = open(os.path.join(ROOT, "include", "tc_qmatmul.h")).read()
    enum = dict((m.group(1), int(m.group(2))) for m in re.finditer(r"\bTC_([A-Z0-9_]+) = (\d+)", text)
                if not m.group(1).startswith("E_") and m.group(1) != "OK")
    assert {k: v for k, v in enum.items() if k in tc_hip.TYPES} == tc_hip.TYPES
    assert set(tc_hip.TYPES) <= set(enum)
    for name, t in tc_hip.TYPES.items():
        bs, ts = lib.tc_gguf_block_size(t), lib.tc_gguf_type_size(t)
        assert (bs, ts) == (tc_hip.BLOCK_SIZE[t], tc_hip.TYPE_SIZE[t]), name
        assert lib.tc_row_bytes(t, 18944) == 18944 // bs * ts, name
        assert lib.tc_row_bytes(t, 3584) == 3584 // bs * ts, name
    for t in (0, 1, 16, 142, 143, 200):
        assert lib.tc_row_bytes(t, 256) == 0, t


def test_reference_interface_header_compiles_and_links(tmp_path):
    """include/tc_int8gemm.hpp (the reference's tinycoder::gpu interface over
    the C ABI) compiles as C++17, links against the library, and reports no
    device and refuses calls cleanly on a machine without a GPU."""
    import shutil
    import subprocess
    import tc_hip
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    lib = tc_hip.load_library()
    so = lib._name
    src = tmp_path / "iface.cpp"
    src.write_text(
        '#include "tc_int8gemm.hpp"\n'
        "int main() {\n"
        "  namespace g = tinycoder::gpu;\n"
        "  if (g::int8GemmAvailable()) return 2;\n"
        "  if (g::int8Gemv(12, nullptr, nullptr, nullptr, 1, 1, 256, nullptr)) return 3;\n"
        "  if (g::int8Gemm(12, nullptr, nullptr, nullptr, 16, 1, 256, 1, nullptr)) return 4;\n"
        "  if (g::int8GemvDualIQ2XS(nullptr, nullptr, nullptr, nullptr, nullptr, 1, 256, nullptr)) return 5;\n"
        "  return 0;\n"
        "}\n")
    exe = tmp_path / "iface"
    subprocess.run([gxx, "-std=c++17", "-I", os.path.join(ROOT, "include"), str(src), so,
                    "-Wl,-rpath," + os.path.dirname(so), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, timeout=60)
    assert r.returncode == 0, (r.returncode, r.stderr)


def test_cpp_interface_driver_without_gpu():
    """The C++ interface driver (tests/cpp, built from include/tc_int8gemm.hpp
    and include/tc_simd_matmul.hpp against the library) loads, and without a
    GPU every call reports false and writes nothing."""
    import numpy as np
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import iface
    d = iface.load()
    assert d.drv_int8GemmAvailable() == 0
    assert d.drv_int8Gemv(12, None, None, None, 1, 1, 256, None) == 0
    assert d.drv_int8Gemm(12, None, None, None, 16, 1, 256, 1, None) == 0
    w = np.zeros(144, np.uint8)
    x = np.zeros(256, np.float32)
    out = np.full(1, 7.0, np.float32)
    for t in (12, 11, 14, 13, 23, 20, 8):
        assert d.drv_matMulVecBatch_SIMD(t, w.ctypes.data, x.ctypes.data, 1, 1, 256, out.ctypes.data, None) == 0
    assert out[0] == 7.0
