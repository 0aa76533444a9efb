"""Python binding of libtc_hip.so (the C-ABI in include/tc_qmatmul.h).

The library is the product; this module only passes device pointers, sizes
and the current HIP stream through ctypes, and raises when a call fails.
PyTorch supplies device memory and streams. There is no CPU fallback: if the
library is missing or a call is refused, the call raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtc_hip.so")

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ4_NL, Q5_0 = 8, 10, 11, 12, 13, 14, 17, 18, 21, 22, 23, 20, 6
TYPES = {"Q8_0": Q8_0, "Q2_K": Q2_K, "Q3_K": Q3_K, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K, "IQ3_XXS": IQ3_XXS, "IQ3_S": IQ3_S, "IQ2_S": IQ2_S, "IQ2_XS": IQ2_XS, "IQ4_XS": IQ4_XS, "IQ4_NL": IQ4_NL, "Q5_0": Q5_0}
TYPE_SIZE = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ2_XS: 74, IQ4_XS: 136, IQ4_NL: 18, Q5_0: 22}
BLOCK_SIZE = {Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256, IQ2_XS: 256, IQ4_XS: 256, IQ4_NL: 32, Q5_0: 32}

TC_OK, TC_E_UNSUPPORTED, TC_E_LAUNCH, TC_E_ARG = 0, -1, -2, -3

# Every function the C header declares, with its ctypes signature.
_P, _U32, _I = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
SIGNATURES = {
    "tc_available": (_I, []),
    "tc_gemv": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _P]),
    "tc_gemv_reserve": (_I, [_U32, _U32]),
    "tc_gemv_multi": (_I, [_I, _U32, _P, _P, _P, _P, _P, _U32, _P]),
    "tc_act_bytes": (ctypes.c_size_t, [_I, _U32, _U32]),
    "tc_act_quantize": (_I, [_I, _P, _U32, _U32, _P, _P]),
    "tc_gemv_q8": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _P]),
    "tc_gemv_dual": (_I, [_I, _P, _P, _P, _P, _P, _U32, _U32, _P]),
    "tc_gemm": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "tc_gemm_preferred": (_I, [_U32, _U32, _U32]),
    "tc_gemm_set_q8_enabled": (None, [_I]),
    "tc_quantize_act": (_I, [_I, _P, _U32, _U32, _P, _P, _P, _P]),
    "tc_block_isums": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _P]),
    "tc_encode": (_I, [_I, _P, _P, _U32, _U32, _P]),
    "tc_row_bytes": (ctypes.c_size_t, [_I, _U32]),
    "tc_moe_ffn": (_I, [_P, _P, _P, _U32, _U32, _P, _P, _P, _U32, _U32, _U32, _P, _P]),
    "tc_debug_q8k_row": (_I, [_I, _P, _U32, _P, _U32, _P]),
    "tc_debug_q8_0_row": (_I, [_P, _U32, _P, _U32, _P]),
    "tc_debug_q8k_blocks": (_I, [_I, _P, _U32, _P, _U32, _P, _P]),
    "tc_debug_q8_0_blocks": (_I, [_P, _U32, _P, _U32, _P, _P]),
    "tc_last_error": (ctypes.c_char_p, []),
    "tc_probe_sink_bytes": (ctypes.c_size_t, []),
    "tc_probe_mfma_i8": (_I, [_U32, _U32, _P, _P]),
    "tc_probe_read": (_I, [_P, ctypes.c_size_t, _U32, _P, _P]),
    "tc_moe_set_gemm_min_tokens": (None, [_U32]),
    "tc_moe_router": (_I, [_P, _P, _U32, _U32, _U32, _U32, _P, _P, _P, _P]),
    "tc_moe_select": (_I, [_P, _U32, _U32, _U32, _P, _P, _P]),
    "tc_host_matmul": (_I, [_I, _P, _P, _U32, _U32, _U32, _P, _P]),
    "tc_host_matmul_f32": (_I, [_P, _P, _U32, _U32, _U32, _P]),
    "tc_gemm_noalloc": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "tc_gemm_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "tc_host_weights_register": (_I, [_P, ctypes.c_size_t]),
    "tc_host_weights_unregister": (_I, [_P]),
    "tc_gguf_open": (_P, [ctypes.c_char_p]),
    "tc_gguf_open_metadata": (_P, [ctypes.c_char_p]),
    "tc_gguf_close": (None, [_P]),
    "tc_gguf_version": (_U32, [_P]),
    "tc_gguf_tensor_count": (ctypes.c_uint64, [_P]),
    "tc_gguf_metadata_count": (ctypes.c_uint64, [_P]),
    "tc_gguf_data_offset": (ctypes.c_uint64, [_P]),
    "tc_gguf_find_tensor": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "tc_gguf_tensor_info": (_I, [_P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U32),
                                 ctypes.POINTER(_U32), ctypes.POINTER(ctypes.c_uint64),
                                 ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "tc_gguf_tensor_data": (_P, [_P, ctypes.c_uint64]),
    "tc_gguf_upload": (_I, [_P, ctypes.c_uint64, _P, ctypes.c_uint64, _P]),
    "tc_gguf_meta": (ctypes.c_char_p, [_P, ctypes.c_char_p]),
    "tc_gguf_type_size": (_U32, [_U32]),
    "tc_gguf_block_size": (_U32, [_U32]),
}


class TCError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libtc_hip error {code}: {msg}")
        self.code = code


def row_bytes(qtype, cols):
    return cols // BLOCK_SIZE[qtype] * TYPE_SIZE[qtype]


def load_library(path=LIB_PATH):
    # torch ships its own libamdhip64.so.7; it must be the HIP runtime this
    # library binds to, or the streams and memory torch hands over belong to
    # another runtime instance. Importing torch first makes the loader reuse it.
    import torch  # noqa: F401
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() "
                                "(make -C tinycoder-inference_amd)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Library:
    """Thin callable wrapper; tensors are torch CUDA tensors."""

    def __init__(self, path=LIB_PATH):
        self.lib = load_library(path)
        self.path = path

    # -- helpers ---------------------------------------------------------------
    def _stream(self):
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def _check(self, rc):
        if rc != TC_OK:
            raise TCError(rc, self.lib.tc_last_error().decode())
        return rc

    def available(self):
        return bool(self.lib.tc_available())

    # -- entry points -------------------------------------------------------------
    def gemv(self, qtype, w, x, rows, cols, out=None):
        import torch
        S = x.numel() // cols
        if out is None:
            out = torch.empty((S, rows), dtype=torch.float32, device=x.device)
        self._check(self.lib.tc_gemv(qtype, _ptr(w), _ptr(x), _ptr(out), S, rows, cols, self._stream()))
        return out

    def gemv_multi(self, qtype, ws, xs, rows, cols, outs=None):
        """One launch over several matrices; xs[i] is [S][cols[i]]."""
        import torch
        n = len(ws)
        S = xs[0].numel() // cols[0]
        if outs is None:
            outs = [torch.empty((S, rows[i]), dtype=torch.float32, device=xs[0].device) for i in range(n)]
        arr = ctypes.c_void_p * n
        u32 = ctypes.c_uint32 * n
        self._check(self.lib.tc_gemv_multi(qtype, n, arr(*[w.data_ptr() for w in ws]),
                                           arr(*[x.data_ptr() for x in xs]), arr(*[o.data_ptr() for o in outs]),
                                           u32(*rows), u32(*cols), S, self._stream()))
        return outs

    def act_buffer(self, qtype, seq_len, cols, device="cuda"):
        import torch
        n = self.lib.tc_act_bytes(qtype, seq_len, cols)
        if n == 0:
            raise TCError(TC_E_UNSUPPORTED, f"no activation layout for type {qtype}, cols {cols}")
        return torch.empty(n, dtype=torch.uint8, device=device)

    def act_quantize(self, qtype, x, cols, act):
        S = x.numel() // cols
        self._check(self.lib.tc_act_quantize(qtype, _ptr(x), S, cols, _ptr(act), self._stream()))
        return act

    def gemv_q8(self, qtype, w, act, seq_len, rows, cols, out=None):
        import torch
        if out is None:
            out = torch.empty((seq_len, rows), dtype=torch.float32, device=act.device)
        self._check(self.lib.tc_gemv_q8(qtype, _ptr(w), _ptr(act), _ptr(out), seq_len, rows, cols,
                                        self._stream()))
        return out

    def gemm(self, qtype, w, x, rows, cols, out=None):
        import torch
        S = x.numel() // cols
        if out is None:
            out = torch.empty((S, rows), dtype=torch.float32, device=x.device)
        self._check(self.lib.tc_gemm(qtype, _ptr(w), _ptr(x), _ptr(out), S, rows, cols,
                                     cols // BLOCK_SIZE[qtype], self._stream()))
        return out

    def gemv_dual(self, qtype, wg, wu, x, rows, cols):
        import torch
        g = torch.empty(rows, dtype=torch.float32, device=x.device)
        u = torch.empty(rows, dtype=torch.float32, device=x.device)
        self._check(self.lib.tc_gemv_dual(qtype, _ptr(wg), _ptr(wu), _ptr(x), _ptr(g), _ptr(u), rows,
                                          cols, self._stream()))
        return g, u

    def quantize_act(self, qtype, x, cols):
        import torch
        S = x.numel() // cols
        blk = 32 if qtype == Q8_0 else 256
        qs = torch.empty((S, cols), dtype=torch.int8, device=x.device)
        d = torch.empty((S, cols // blk), dtype=torch.float32, device=x.device)
        bs = None if qtype == Q8_0 else torch.empty((S, cols // 16), dtype=torch.int16, device=x.device)
        self._check(self.lib.tc_quantize_act(qtype, _ptr(x), S, cols, _ptr(qs), _ptr(d), _ptr(bs),
                                             self._stream()))
        return qs, d, bs

    def block_isums(self, qtype, w, x, rows, cols):
        import torch
        S = x.numel() // cols
        nb = cols // BLOCK_SIZE[qtype]
        k = 8 if qtype in (Q4_K, Q5_K) else 2 if qtype == Q2_K else 1
        out = torch.empty((S, rows, nb, k), dtype=torch.int32, device=x.device)
        self._check(self.lib.tc_block_isums(qtype, _ptr(w), _ptr(x), _ptr(out), S, rows, cols,
                                            self._stream()))
        return out

    def encode(self, qtype, x):
        import torch
        rows, cols = x.shape
        out = torch.empty(rows * row_bytes(qtype, cols), dtype=torch.uint8, device=x.device)
        self._check(self.lib.tc_encode(qtype, _ptr(x), _ptr(out), rows, cols, self._stream()))
        return out

    def debug_row(self, qtype, w_row, x):
        """Host numpy row + host x -> the decode kernel's row result."""
        import numpy as np
        w_row = np.ascontiguousarray(w_row, np.uint8)
        x = np.ascontiguousarray(x, np.float32).ravel()
        res = np.zeros(1, np.float32)
        cols = x.size
        if qtype == Q8_0:
            self._check(self.lib.tc_debug_q8_0_row(w_row.ctypes.data, cols // 32, x.ctypes.data, cols,
                                                   res.ctypes.data))
        else:
            self._check(self.lib.tc_debug_q8k_row(qtype, w_row.ctypes.data, cols // 256, x.ctypes.data, cols,
                                                  res.ctypes.data))
        return float(res[0])

    def debug_blocks(self, qtype, w_row, x):
        """-> (per-block float contributions, quantized activation block bytes)."""
        import numpy as np
        w_row = np.ascontiguousarray(w_row, np.uint8)
        x = np.ascontiguousarray(x, np.float32).ravel()
        cols = x.size
        if qtype == Q8_0:
            nb = cols // 32
            blk, q = np.zeros(nb, np.float32), np.zeros(nb * 36, np.uint8)
            self._check(self.lib.tc_debug_q8_0_blocks(w_row.ctypes.data, nb, x.ctypes.data, cols, blk.ctypes.data,
                                                      q.ctypes.data))
        else:
            nb = cols // 256
            blk, q = np.zeros(nb, np.float32), np.zeros(nb * 292, np.uint8)
            self._check(self.lib.tc_debug_q8k_blocks(qtype, w_row.ctypes.data, nb, x.ctypes.data, cols,
                                                     blk.ctypes.data, q.ctypes.data))
        return blk, q

    def moe_ffn(self, x, ids, wts, wg, wu, wd, n_experts, hidden, ff, out=None):
        import torch
        S, K = ids.shape
        if out is None:
            out = torch.empty((S, hidden), dtype=torch.float32, device=x.device)
        self._check(self.lib.tc_moe_ffn(_ptr(x), _ptr(ids), _ptr(wts), S, K, _ptr(wg), _ptr(wu), _ptr(wd),
                                        n_experts, hidden, ff, _ptr(out), self._stream()))
        return out

    def moe_router(self, w_router, x, top_k):
        """Router logits, expert ids and weights for x [S][hidden] against the
        fp32 router matrix [n_experts][hidden]."""
        import torch
        E, H = w_router.shape
        S = x.numel() // H
        logits = torch.empty((S, E), dtype=torch.float32, device=x.device)
        ids = torch.empty((S, top_k), dtype=torch.int32, device=x.device)
        wts = torch.empty((S, top_k), dtype=torch.float32, device=x.device)
        self._check(self.lib.tc_moe_router(_ptr(w_router), _ptr(x), S, E, H, top_k, _ptr(logits), _ptr(ids),
                                           _ptr(wts), self._stream()))
        return logits, ids, wts

    def moe_select(self, logits, top_k):
        import torch
        S, E = logits.shape
        ids = torch.empty((S, top_k), dtype=torch.int32, device=logits.device)
        wts = torch.empty((S, top_k), dtype=torch.float32, device=logits.device)
        self._check(self.lib.tc_moe_select(_ptr(logits), S, E, top_k, _ptr(ids), _ptr(wts), self._stream()))
        return ids, wts


class TensorRecord:
    """One GGUF tensor record (the reference's TensorInfo, IModelLoader.hpp:145:
    name, offset into the data section, shape in file order, GGML type), plus
    its byte size."""

    __slots__ = ("index", "name", "type", "shape", "offset", "bytes")

    def __init__(self, index, name, type_, shape, offset, nbytes):
        self.index, self.name, self.type, self.shape = index, name, type_, shape
        self.offset, self.bytes = offset, nbytes

    def __repr__(self):
        return f"TensorRecord({self.name!r}, type={self.type}, shape={self.shape}, bytes={self.bytes})"


class GGUFLoader:
    """GGUF v3 reader over the C-ABI (tc_gguf_*), shaped like the reference's
    tinycoder::GGUFLoader (include/GGUFLoader.hpp:48): load / loadMetadata,
    getTensor (host bytes, a read-only numpy view of the mapping),
    getTensorInfo, tensorRecords, and upload() to put a tensor's raw blocks in
    device memory for the mat-vec / GEMM entry points. load() returns False on
    failure like the reference; the reason is in last_error."""

    def __init__(self, lib=None):
        self.lib = lib if lib is not None else load_library()
        self.h = None
        self.last_error = ""

    def _open(self, path, fn):
        self.close()
        h = fn(os.fsencode(path))
        if not h:
            self.last_error = self.lib.tc_last_error().decode()
            return False
        self.h = h
        return True

    def load(self, path):
        return self._open(path, self.lib.tc_gguf_open)

    def loadMetadata(self, path):  # noqa: N802 (the reference's name)
        return self._open(path, self.lib.tc_gguf_open_metadata)

    def close(self):
        if self.h:
            self.lib.tc_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self):
        return self.lib.tc_gguf_version(self.h)

    @property
    def data_offset(self):
        return self.lib.tc_gguf_data_offset(self.h)

    def metadata(self, key):
        v = self.lib.tc_gguf_meta(self.h, key.encode())
        return None if v is None else v.decode("utf-8", "surrogateescape")

    def _record(self, i):
        name = ctypes.c_char_p()
        t, nd = ctypes.c_uint32(), ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        rc = self.lib.tc_gguf_tensor_info(self.h, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd),
                                          dims, ctypes.byref(off), ctypes.byref(nb))
        if rc != TC_OK:
            raise TCError(rc, self.lib.tc_last_error().decode())
        return TensorRecord(i, name.value.decode("utf-8", "surrogateescape"), t.value,
                            tuple(dims[k] for k in range(nd.value)), off.value, nb.value)

    def tensorRecords(self):  # noqa: N802
        return [self._record(i) for i in range(self.lib.tc_gguf_tensor_count(self.h))]

    def getTensorInfo(self, name):  # noqa: N802
        i = self.lib.tc_gguf_find_tensor(self.h, name.encode())
        return None if i < 0 else self._record(i)

    def getTensor(self, name):  # noqa: N802
        import numpy as np
        rec = self.getTensorInfo(name)
        if rec is None:
            return None
        p = self.lib.tc_gguf_tensor_data(self.h, rec.index)
        if not p:
            return None
        buf = (ctypes.c_uint8 * rec.bytes).from_address(p)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def upload(self, name, device="cuda"):
        """Raw block bytes of tensor `name` as a uint8 device tensor."""
        import torch
        rec = self.getTensorInfo(name)
        if rec is None:
            raise KeyError(name)
        out = torch.empty(rec.bytes, dtype=torch.uint8, device=device)
        rc = self.lib.tc_gguf_upload(self.h, rec.index, _ptr(out), rec.bytes,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != TC_OK:
            raise TCError(rc, self.lib.tc_last_error().decode())
        return out
