"""Writes oracle/iq2s_grid.inc and tinycoder-inference_amd/csrc/iq2s_grid.inc:
the IQ2_S codebook (1024 entries of 8 magnitude bytes; GGUF format data,
include/GGMLDequantize.hpp:807) read from the compiled reference (oracle/_ref,
built by oracle/Makefile). Run once where the reference tree exists; the tables
are committed."""
import ctypes
import hashlib
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def main():
    lib = ctypes.CDLL(os.path.join(HERE, "_ref", "libtcref.so"))
    g = np.zeros(1024, np.uint64)
    lib.ref_iq2s_grid(ctypes.c_void_p(g.ctypes.data))
    head = ("/* IQ2_S codebook: 1024 entries, 8 unsigned magnitudes per entry (one per byte,\n"
            " * little-endian), values 8, 25, 43. The GGUF format fixes these values; they are\n"
            " * the reference table include/GGMLDequantize.hpp:807 (GGMLDequantize::IQ2S_GRID),\n"
            " * written by oracle/gen_iq2s_grid.py from the compiled reference. */\n")
    body = "".join("    " + ", ".join(f"0x{int(v):016x}ull" for v in g[i:i + 4]) + ",\n" for i in range(0, 1024, 4))
    for path in (os.path.join(HERE, "iq2s_grid.inc"), os.path.join(ROOT, "tinycoder-inference_amd", "csrc", "iq2s_grid.inc")):
        with open(path, "w") as f:
            f.write(head + body)
    print("sha256", hashlib.sha256(g.tobytes()).hexdigest())


if __name__ == "__main__":
    main()
