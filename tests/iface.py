"""Loads tests/cpp/libiface_driver.so: the reference-named C++ interfaces
(include/tc_int8gemm.hpp, include/tc_simd_matmul.hpp) compiled into a small
driver whose exported C functions call them as a reference call site does."""
import ctypes
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tests", "cpp", "libiface_driver.so")
_P, _U32, _I = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
SIGS = {
    "drv_int8GemmAvailable": (_I, []),
    "drv_int8GemmPreferred": (_I, [_U32, _U32, _U32]),
    "drv_int8GemvReserve": (None, [_U32, _U32]),
    "drv_int8GemmSetQ8Enabled": (None, [_I]),
    "drv_int8Gemv": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _P]),
    "drv_int8Gemm": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "drv_int8GemvDual": (_I, [_I, _P, _P, _P, _P, _P, _U32, _U32, _P]),
    "drv_matMulVecBatch_SIMD": (_I, [_I, _P, _P, _U32, _U32, _U32, _P, _P]),
    "drv_matMulVecBatchF32_SIMD": (_I, [_P, _P, _U32, _U32, _U32, _P]),
}


def load():
    import tc_hip
    tc_hip.load_library()  # torch's HIP runtime first, then the library the driver links
    if not os.path.exists(DRIVER):
        raise FileNotFoundError(f"{DRIVER} is not built: run __graft_entry__.build() (make -C tests/cpp)")
    d = ctypes.CDLL(DRIVER)
    for n, (r, a) in SIGS.items():
        f = getattr(d, n)
        f.restype, f.argtypes = r, a
    return d
