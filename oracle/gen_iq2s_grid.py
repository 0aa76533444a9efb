"""Writes iq2s_grid.inc and iq2xs_grid.inc into oracle/ and
tinycoder-inference_amd/csrc/: the IQ2_S codebook (1024 entries of 8 magnitude
bytes, include/GGMLDequantize.hpp:807) and the IQ2_XS codebook (512 entries,
:821) -- GGUF format data -- read from the compiled reference (oracle/_ref,
built by oracle/Makefile). Run once where the reference tree exists; the tables
are committed."""
import ctypes
import hashlib
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def write(name, n, fn, head):
    lib = ctypes.CDLL(os.path.join(HERE, "_ref", "libtcref.so"))
    g = np.zeros(n, np.uint64)
    getattr(lib, fn)(ctypes.c_void_p(g.ctypes.data))
    body = "".join("    " + ", ".join(f"0x{int(v):016x}ull" for v in g[i:i + 4]) + ",\n" for i in range(0, n, 4))
    for path in (os.path.join(HERE, name), os.path.join(ROOT, "tinycoder-inference_amd", "csrc", name)):
        with open(path, "w") as f:
            f.write(head + body)
    print(name, "sha256", hashlib.sha256(g.tobytes()).hexdigest())


def main():
    write("iq2s_grid.inc", 1024, "ref_iq2s_grid",
          "/* IQ2_S codebook: 1024 entries, 8 unsigned magnitudes per entry (one per byte,\n"
          " * little-endian), values 8, 25, 43. The GGUF format fixes these values; they are\n"
          " * the reference table include/GGMLDequantize.hpp:807 (GGMLDequantize::IQ2S_GRID),\n"
          " * written by oracle/gen_iq2s_grid.py from the compiled reference. */\n")
    write("iq2xs_grid.inc", 512, "ref_iq2xs_grid",
          "/* IQ2_XS codebook: 512 entries, 8 unsigned magnitudes per entry (one per byte,\n"
          " * little-endian), values 8, 25, 43. The GGUF format fixes these values; they are\n"
          " * the reference table include/GGMLDequantize.hpp:821 (GGMLDequantize::iq2xs_grid),\n"
          " * written by oracle/gen_iq2s_grid.py from the compiled reference. */\n")


if __name__ == "__main__":
    main()
