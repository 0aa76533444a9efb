"""Writes oracle/iq3s_grid.inc and tinycoder-inference_amd/csrc/iq3s_grid.inc:
the IQ3_S codebook (512 words; GGUF format data, include/GGMLDequantize.hpp:815)
read from the compiled reference (oracle/_ref, built by oracle/Makefile).
Run once where the reference tree exists; the tables are committed."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def main():
    lib = ctypes.CDLL(os.path.join(HERE, "_ref", "libtcref.so"))
    g = np.zeros(512, np.uint32)
    lib.ref_iq3s_grid(ctypes.c_void_p(g.ctypes.data))
    head = ("/* IQ3_S codebook: 512 entries, 4 unsigned magnitudes per entry (one per byte,\n"
            " * little-endian), odd values 1..15. The GGUF format fixes these values; they\n"
            " * are the reference table include/GGMLDequantize.hpp:815 (GGMLDequantize::IQ3S_GRID),\n"
            " * written by oracle/gen_iq3s_grid.py from the compiled reference. */\n")
    body = "".join("    " + ", ".join(f"0x{v:08x}" for v in g[i:i + 8]) + ",\n" for i in range(0, 512, 8))
    for path in (os.path.join(HERE, "iq3s_grid.inc"), os.path.join(ROOT, "tinycoder-inference_amd", "csrc", "iq3s_grid.inc")):
        with open(path, "w") as f:
            f.write(head + body)
    print("sha256", __import__("hashlib").sha256(g.tobytes()).hexdigest())


if __name__ == "__main__":
    main()
