"""ctypes bindings for the CPU oracle (liboracle.so) and, where it was built,
the compiled reference (oracle/_ref/libtcref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline. The
product never imports this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtcref.so")

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ4_NL, Q5_0 = 8, 10, 11, 12, 13, 14, 17, 18, 21, 22, 23, 20, 6
TYPE_SIZE = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ2_XS: 74, IQ4_XS: 136, IQ4_NL: 18, Q5_0: 22}
BLOCK_SIZE = {Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256, IQ2_XS: 256, IQ4_XS: 256, IQ4_NL: 32, Q5_0: 32}

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def row_bytes(qtype, cols):
    return cols // BLOCK_SIZE[qtype] * TYPE_SIZE[qtype]


class _Lib:
    def __init__(self, path, prefix):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run make -C oracle)")
        self.lib = ctypes.CDLL(path)
        self.prefix = prefix


class Oracle(_Lib):
    """The C restatement (oracle.c)."""

    def __init__(self):
        super().__init__(ORACLE_SO, "oc_")
        L = self.lib
        L.oc_half_to_float.restype = ctypes.c_float
        L.oc_half_to_float.argtypes = [ctypes.c_uint16]
        L.oc_float_to_half.restype = ctypes.c_uint16
        L.oc_float_to_half.argtypes = [ctypes.c_float]
        for name in ("oc_quantize_q8k",):
            getattr(L, name).argtypes = [_P, _U32, _P, _P, _P]
        L.oc_quantize_q8_0_act.argtypes = [_P, _U32, _P, _P]
        L.oc_dequant_row.argtypes = [ctypes.c_int, _P, _U32, _P]
        L.oc_block_isums.argtypes = [ctypes.c_int, _P, _P, _U32, _U32, _U32, _P]
        L.oc_matmul.argtypes = [ctypes.c_int, _P, _P, _U32, _U32, _U32, _P]
        L.oc_encode_rows.argtypes = [ctypes.c_int, _P, _U32, _U32, _P]
        L.oc_moe_ffn.argtypes = [_P, _P, _P, _U32, _U32, _P, _P, _P, _U32, _U32, _U32, _P]
        L.oc_matmul_f32.argtypes = [_P, _P, _U32, _U32, _U32, _P]
        L.oc_moe_route.argtypes = [_P, _U32, _U32, _U32, _P, _P]

    def half_to_float(self, h):
        return self.lib.oc_half_to_float(int(h))

    def float_to_half(self, f):
        return self.lib.oc_float_to_half(float(f))

    def quantize_q8k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        n = x.size
        qs = np.zeros(n, np.int8)
        d = np.zeros(n // 256, np.float32)
        bs = np.zeros(n // 16, np.int16)
        self.lib.oc_quantize_q8k(_ptr(x), n, _ptr(qs), _ptr(d), _ptr(bs))
        return qs, d, bs

    def quantize_q8_0_act(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        n = x.size
        qs = np.zeros(n, np.int8)
        d = np.zeros(n // 32, np.float32)
        self.lib.oc_quantize_q8_0_act(_ptr(x), n, _ptr(qs), _ptr(d))
        return qs, d

    def dequant(self, qtype, w, rows, cols):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        out = np.zeros((rows, cols), np.float32)
        rb = row_bytes(qtype, cols)
        for r in range(rows):
            rc = self.lib.oc_dequant_row(qtype, ctypes.c_void_p(w.ctypes.data + r * rb), cols,
                                         ctypes.c_void_p(out.ctypes.data + r * cols * 4))
            assert rc == 0
        return out

    def block_isums(self, qtype, w, x, rows, cols):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
        S = x.shape[0]
        nb = cols // BLOCK_SIZE[qtype]
        k = 8 if qtype in (Q4_K, Q5_K) else 2 if qtype == Q2_K else 1
        out = np.zeros((S, rows, nb, k), np.int32)
        rc = self.lib.oc_block_isums(qtype, _ptr(w), _ptr(x), S, rows, cols, _ptr(out))
        assert rc == 0
        return out

    def matmul(self, qtype, w, x, rows, cols):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
        S = x.shape[0]
        out = np.zeros((S, rows), np.float32)
        rc = self.lib.oc_matmul(qtype, _ptr(w), _ptr(x), S, rows, cols, _ptr(out))
        assert rc == 0
        return out

    def encode(self, qtype, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, cols = x.shape
        out = np.zeros(rows * row_bytes(qtype, cols), np.uint8)
        rc = self.lib.oc_encode_rows(qtype, _ptr(x), rows, cols, _ptr(out))
        assert rc == 0
        return out

    def matmul_f32(self, w, x, rows, cols):
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
        out = np.zeros((x.shape[0], rows), np.float32)
        self.lib.oc_matmul_f32(_ptr(w), _ptr(x), x.shape[0], rows, cols, _ptr(out))
        return out

    def moe_route(self, logits, k):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        S, E = logits.shape
        ids = np.zeros((S, k), np.int32)
        wts = np.zeros((S, k), np.float32)
        rc = self.lib.oc_moe_route(_ptr(logits), S, E, k, _ptr(ids), _ptr(wts))
        assert rc == 0
        return ids, wts

    def moe_ffn(self, x, ids, wts, wg, wu, wd, E, H, FF):
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        wts = np.ascontiguousarray(wts, dtype=np.float32)
        S, K = ids.shape
        out = np.zeros((S, H), np.float32)
        rc = self.lib.oc_moe_ffn(_ptr(x), _ptr(ids), _ptr(wts), S, K, _ptr(wg), _ptr(wu), _ptr(wd),
                                 E, H, FF, _ptr(out))
        assert rc == 0
        return out


class Reference(_Lib):
    """The reference's own CPU functions, compiled from its sources."""

    def __init__(self, threads=1):
        super().__init__(REF_SO, "ref_")
        L = self.lib
        L.ref_init_threads.restype = ctypes.c_int
        L.ref_init_threads.argtypes = [ctypes.c_int]
        L.ref_half_to_float.restype = ctypes.c_float
        L.ref_half_to_float.argtypes = [ctypes.c_uint16]
        L.ref_float_to_half.restype = ctypes.c_uint16
        L.ref_float_to_half.argtypes = [ctypes.c_float]
        L.ref_quantize_q8k.argtypes = [_P, _U32, _P, _P, _P]
        L.ref_dequant_block.argtypes = [ctypes.c_int, _P, _P]
        L.ref_quantize_q4k_block.argtypes = [_P, _P]
        L.ref_dot_iq3xxs_q8k.restype = ctypes.c_float
        L.ref_dot_iq3xxs_q8k.argtypes = [_P, _P]
        L.ref_matmul.argtypes = [ctypes.c_int, _P, _P, _U32, _U32, _U32, _P]
        L.ref_matmul_f32.argtypes = [_P, _P, _U32, _U32, _U32, _P]
        L.ref_moe_select.argtypes = [_P, _U32, _U32, _U32, _P, _P]
        L.ref_gguf_open.restype = _P
        L.ref_gguf_open.argtypes = [ctypes.c_char_p, ctypes.c_int]
        L.ref_gguf_close.argtypes = [_P]
        L.ref_gguf_count.restype = ctypes.c_uint64
        L.ref_gguf_count.argtypes = [_P]
        L.ref_gguf_record.argtypes = [_P, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_uint64, _P, _P, _P, _P]
        L.ref_gguf_tensor.restype = _P
        L.ref_gguf_tensor.argtypes = [_P, ctypes.c_char_p]
        L.ref_gguf_config.argtypes = [_P, _P, _P, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_uint64]
        L.ref_ggml_type_size.restype = _U32
        L.ref_ggml_type_size.argtypes = [_U32]
        L.ref_ggml_block_size.restype = _U32
        L.ref_ggml_block_size.argtypes = [_U32]
        self.threads = L.ref_init_threads(threads)

    def quantize_q8k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        n = x.size
        qs = np.zeros(n, np.int8)
        d = np.zeros(n // 256, np.float32)
        bs = np.zeros(n // 16, np.int16)
        self.lib.ref_quantize_q8k(_ptr(x), n, _ptr(qs), _ptr(d), _ptr(bs))
        return qs, d, bs

    def dequant(self, qtype, w, rows, cols):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        bs, ts = BLOCK_SIZE[qtype], TYPE_SIZE[qtype]
        nblk = rows * cols // bs
        out = np.zeros(nblk * bs, np.float32)
        for i in range(nblk):
            self.lib.ref_dequant_block(qtype, ctypes.c_void_p(w.ctypes.data + i * ts),
                                       ctypes.c_void_p(out.ctypes.data + i * bs * 4))
        return out.reshape(rows, cols)

    def encode_q4k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        nblk = x.size // 256
        out = np.zeros(nblk * 144, np.uint8)
        for i in range(nblk):
            self.lib.ref_quantize_q4k_block(ctypes.c_void_p(x.ctypes.data + i * 1024),
                                            ctypes.c_void_p(out.ctypes.data + i * 144))
        return out

    def matmul_f32(self, w, x, rows, cols):
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
        out = np.zeros((x.shape[0], rows), np.float32)
        self.lib.ref_matmul_f32(_ptr(w), _ptr(x), x.shape[0], rows, cols, _ptr(out))
        return out

    def moe_select(self, logits, k):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        S, E = logits.shape
        ids = np.zeros((S, k), np.int32)
        wts = np.zeros((S, k), np.float32)
        self.lib.ref_moe_select(_ptr(logits), S, E, k, _ptr(ids), _ptr(wts))
        return ids, wts

    def matmul(self, qtype, w, x, rows, cols, out=None):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
        S = x.shape[0]
        if out is None:
            out = np.zeros((S, rows), np.float32)
        rc = self.lib.ref_matmul(qtype, _ptr(w), _ptr(x), S, rows, cols, _ptr(out))
        assert rc == 0
        return out


class RefGGUF:
    """The reference's own GGUFLoader (compiled from its sources) on one file:
    records, tensor bytes and the parsed config."""

    def __init__(self, ref, path, metadata_only=False):
        self.ref, self.L = ref, ref.lib
        self.h = self.L.ref_gguf_open(os.fsencode(path), int(metadata_only))

    @property
    def ok(self):
        return bool(self.h)

    def close(self):
        if self.h:
            self.L.ref_gguf_close(self.h)
            self.h = None

    def records(self):
        out = []
        for i in range(self.L.ref_gguf_count(self.h)):
            name = ctypes.create_string_buffer(4096)
            t, nd = np.zeros(1, np.uint32), np.zeros(1, np.uint32)
            dims, off = np.zeros(4, np.uint32), np.zeros(1, np.uint64)
            assert self.L.ref_gguf_record(self.h, i, name, 4096, _ptr(t), _ptr(nd), _ptr(dims), _ptr(off)) == 0
            out.append((name.value.decode(), int(t[0]), tuple(int(d) for d in dims[:nd[0]]), int(off[0])))
        return out

    def tensor(self, name, nbytes):
        p = self.L.ref_gguf_tensor(self.h, name.encode())
        return None if not p else np.frombuffer((ctypes.c_uint8 * nbytes).from_address(p), np.uint8).copy()

    def config(self):
        u, f = np.zeros(16, np.uint32), np.zeros(2, np.float32)
        arch, name = ctypes.create_string_buffer(256), ctypes.create_string_buffer(256)
        self.L.ref_gguf_config(self.h, _ptr(u), _ptr(f), arch, name, 256)
        keys = ["numLayers", "maxSeqLen", "hiddenSize", "intermediateSize", "numAttentionHeads", "numKVHeads",
                "vocabSize", "expertCount", "expertUsedCount", "expertFeedForwardLength", "ropeDimensionCount",
                "sec0", "sec1", "sec2", "sec3", "headDim"]
        c = {k: int(v) for k, v in zip(keys, u)}
        c["ropeTheta"], c["finalLogitSoftcapping"] = float(f[0]), float(f[1])
        c["architecture"], c["modelName"] = arch.value.decode(), name.value.decode()
        return c


def available_reference():
    return os.path.exists(REF_SO)
