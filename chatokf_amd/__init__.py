"""chatokf_amd -- MI355X (gfx950) quantized weight x activation path.

The product is the C-ABI library ``libokf_quant.so`` (declared in
``include/okf_quant.h``, built by ``chatokf_amd.build``).  This module is the
Python binding of that ABI, shaped like the reference's dispatch surface
``MetalEnc`` (``LLM/Base/MetalEnc.swift``): ``gemv`` (:84-93), ``gemm``
(:241-289), ``gemm_tile`` (:326-352) and ``dequant_row`` (:402-459).  Torch
tensors are only device-memory plumbing; every computation runs in the HIP
library.  There is no fallback: if the library is missing, importing the
binding raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

from .formats import (Q8_0, Q4_K, IQ2_XXS, Q2_0, Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S, IQ3_XXS,  # noqa
                      IQ3_S, IQ1_S, IQ1_M, F32, F16, BF16, Q2_K, Q3_K, NAMES, BY_NAME, block_elems, row_bytes)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("OKF_LIB") or os.path.join(HERE, "libokf_quant.so")

(OKF_OK, OKF_E_TYPE, OKF_E_SHAPE, OKF_E_HIP, OKF_E_INJECTED, OKF_E_ARG, OKF_E_NODEV, OKF_E_IO,
 OKF_E_FORMAT, OKF_E_NOTFOUND, OKF_E_TIMEOUT) = range(11)

# Every symbol include/okf_quant.h declares.
EXPORTS = (
    "okf_ctx_create", "okf_ctx_destroy", "okf_ctx_stream", "okf_ctx_reserve", "okf_row_bytes",
    "okf_gemv", "okf_gemv_silu", "okf_gemv_gate_up", "okf_ffn", "okf_silu_mul", "okf_gemm", "okf_gemm_tile", "okf_dequant_row",
    "okf_embed_batch", "okf_add_rmsnorm_batch", "okf_argmax_rows", "okf_argmax_rows_noalloc",
    "okf_stream_read", "okf_parallel_begin",
    "okf_parallel_end", "okf_sync", "okf_set_fault_rate", "okf_last_hip_error", "okf_strerror",
    "okf_gguf_open", "okf_gguf_close", "okf_gguf_tensor_count", "okf_gguf_tensor_at", "okf_gguf_find",
    "okf_gguf_kv_int", "okf_gguf_kv_double", "okf_gguf_kv_string", "okf_gguf_data", "okf_gguf_upload",
    "okf_gguf_free_device",
)


class OkfGGUFTensor(ctypes.Structure):
    """``okf_gguf_tensor`` of include/okf_quant.h."""
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("n_dims", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * 4),
        ("ggml_type", ctypes.c_int32),
        ("offset", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
    ]


class OkfWeight(ctypes.Structure):
    """``okf_weight`` of include/okf_quant.h."""
    _fields_ = [
        ("base", ctypes.c_void_p),
        ("off", ctypes.c_uint64),
        ("K", ctypes.c_uint32),
        ("M", ctypes.c_uint32),
        ("ggml_type", ctypes.c_int32),
    ]


class OkfError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {_lib().okf_strerror(status).decode()} ({status})")


_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m chatokf_amd.build` "
                "(there is no non-HIP fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32
        W = ctypes.POINTER(OkfWeight)
        sig = {
            "okf_ctx_create": [ctypes.c_int, ctypes.POINTER(vp)],
            "okf_ctx_destroy": [vp],
            "okf_ctx_stream": [vp, ctypes.POINTER(vp)],
            "okf_ctx_reserve": [vp, u64, u32, u32],
            "okf_row_bytes": [i32, u64, ctypes.POINTER(u64)],
            "okf_gemv": [vp, W, vp, vp],
            "okf_gemv_silu": [vp, W, vp, vp, vp],
            "okf_ffn": [vp, W, W, W, vp, vp, vp, vp],
            "okf_gemv_gate_up": [vp, W, W, vp, vp, vp],
            "okf_silu_mul": [vp, vp, vp, u32],
            "okf_gemm": [vp, W, vp, u32, vp],
            "okf_gemm_tile": [vp, W, vp, u32, vp],
            "okf_dequant_row": [vp, W, u32, vp],
            "okf_embed_batch": [vp, W, vp, u32, vp],
            "okf_add_rmsnorm_batch": [vp, vp, vp, vp, vp, u32, u32, ctypes.c_float],
            "okf_argmax_rows": [vp, vp, u32, u32, vp],
            "okf_argmax_rows_noalloc": [vp, vp, u32, u32, vp],
            "okf_stream_read": [vp, vp, ctypes.c_uint64, vp],
            "okf_parallel_begin": [vp],
            "okf_parallel_end": [vp],
            "okf_sync": [vp],
            "okf_set_fault_rate": [vp, ctypes.c_double, u64],
            "okf_last_hip_error": [vp],
            "okf_gguf_open": [ctypes.c_char_p, ctypes.POINTER(vp)],
            "okf_gguf_close": [vp],
            "okf_gguf_tensor_count": [vp, ctypes.POINTER(u64)],
            "okf_gguf_tensor_at": [vp, u64, ctypes.POINTER(OkfGGUFTensor)],
            "okf_gguf_find": [vp, ctypes.c_char_p, ctypes.POINTER(OkfGGUFTensor)],
            "okf_gguf_kv_int": [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)],
            "okf_gguf_kv_double": [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)],
            "okf_gguf_kv_string": [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(u64)],
            "okf_gguf_data": [vp, ctypes.POINTER(vp), ctypes.POINTER(u64)],
            "okf_gguf_upload": [vp, vp, ctypes.POINTER(vp)],
            "okf_gguf_free_device": [vp, vp],
        }
        for name, args in sig.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        lib.okf_strerror.argtypes = [ctypes.c_int]
        lib.okf_strerror.restype = ctypes.c_char_p
        _LIB = lib
    return _LIB


def lib():
    """The loaded ctypes library (raises if it was never built)."""
    return _lib()


def _ptr(t) -> int:
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return t.data_ptr()


class QuantTensor:
    """A GGUF-quantized matrix in device memory: M rows of K weights.

    Replaces GGUFTensor + WeightRef (``LLM/Base/GGUF.swift:49-57``,
    ``LLM/Base/MetalContext.swift:4-11``).  ``data`` is a device byte buffer
    (a torch uint8 tensor or a raw pointer), ``off`` a byte offset into it.
    """

    def __init__(self, data, K: int, M: int, ggml_type: int, off: int = 0):
        self.data, self.K, self.M, self.type, self.off = data, int(K), int(M), int(ggml_type), int(off)

    @property
    def row_bytes(self) -> int:
        return row_bytes(self.type, self.K)

    def c(self) -> OkfWeight:
        return OkfWeight(_ptr(self.data), self.off, self.K, self.M, self.type)


class Enc:
    """The MetalEnc-shaped encoder over one okf context (one device, one stream)."""

    def __init__(self, device: int = 0):
        self._lib = _lib()
        h = ctypes.c_void_p()
        st = self._lib.okf_ctx_create(int(device), ctypes.byref(h))
        if st != OKF_OK:
            raise OkfError(st, f"okf_ctx_create({device})")
        self.h = h
        self.device = device

    # -- lifetime
    def close(self):
        if getattr(self, "h", None):
            self._lib.okf_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int, what: str):
        if st != OKF_OK:
            raise OkfError(st, what)

    # -- calls
    @property
    def stream(self) -> int:
        s = ctypes.c_void_p()
        self._check(self._lib.okf_ctx_stream(self.h, ctypes.byref(s)), "okf_ctx_stream")
        return s.value or 0

    def gemv(self, w: QuantTensor, x, out):
        wc = w.c()
        self._check(self._lib.okf_gemv(self.h, ctypes.byref(wc), _ptr(x), _ptr(out)), "okf_gemv")

    def gemv_silu(self, w: QuantTensor, gate, up, out):
        """y = W (silu(gate) * up): MetalEnc.siluMul then gemv, one launch."""
        wc = w.c()
        self._check(self._lib.okf_gemv_silu(self.h, ctypes.byref(wc), _ptr(gate), _ptr(up), _ptr(out)),
                    "okf_gemv_silu")

    def ffn(self, gate: QuantTensor, up: QuantTensor, down: QuantTensor, x, g, u, y):
        """okf_ffn: u = W_up x, g = silu(W_gate x) * u (in place, as the reference's
        siluMul), y = W_down g."""
        gc, uc, dc = gate.c(), up.c(), down.c()
        self._check(self._lib.okf_ffn(self.h, ctypes.byref(gc), ctypes.byref(uc), ctypes.byref(dc), _ptr(x),
                                      _ptr(g), _ptr(u), _ptr(y)), "okf_ffn")

    def gemv_gate_up(self, gate: QuantTensor, up: QuantTensor, x, g, u):
        """okf_gemv_gate_up: u = W_up x, g = silu(W_gate x) * u."""
        gc, uc = gate.c(), up.c()
        self._check(self._lib.okf_gemv_gate_up(self.h, ctypes.byref(gc), ctypes.byref(uc), _ptr(x), _ptr(g),
                                               _ptr(u)), "okf_gemv_gate_up")

    def raw_ffn(self, gc: OkfWeight, uc: OkfWeight, dc: OkfWeight, x: int, g: int, u: int, y: int):
        """okf_ffn on prebuilt descriptors and raw device pointers."""
        rc = self._lib.okf_ffn(self.h, ctypes.byref(gc), ctypes.byref(uc), ctypes.byref(dc), x, g, u, y)
        if rc:
            self._check(rc, "okf_ffn")

    def silu_mul(self, a, b, n: int):
        """a[:n] = silu(a) * b (MetalEnc.siluMul)."""
        self._check(self._lib.okf_silu_mul(self.h, _ptr(a), _ptr(b), int(n)), "okf_silu_mul")

    def gemm(self, w: QuantTensor, X, out, N: int):
        wc = w.c()
        self._check(self._lib.okf_gemm(self.h, ctypes.byref(wc), _ptr(X), int(N), _ptr(out)), "okf_gemm")

    def raw_gemv(self, wc: OkfWeight, x: int, out: int):
        """okf_gemv on a prebuilt descriptor and raw device pointers (no
        per-call Python object construction; for launch-rate-bound callers)."""
        rc = self._lib.okf_gemv(self.h, ctypes.byref(wc), x, out)
        if rc:
            self._check(rc, "okf_gemv")

    def raw_gemv_silu(self, wc: OkfWeight, gate: int, up: int, out: int):
        """okf_gemv_silu on a prebuilt descriptor and raw device pointers."""
        rc = self._lib.okf_gemv_silu(self.h, ctypes.byref(wc), gate, up, out)
        if rc:
            self._check(rc, "okf_gemv_silu")

    def raw_gemm(self, wc: OkfWeight, X: int, N: int, out: int):
        """okf_gemm on a prebuilt descriptor and raw device pointers."""
        rc = self._lib.okf_gemm(self.h, ctypes.byref(wc), X, N, out)
        if rc:
            self._check(rc, "okf_gemm")

    def gemm_tile(self, w: QuantTensor, X, out, N: int):
        wc = w.c()
        self._check(self._lib.okf_gemm_tile(self.h, ctypes.byref(wc), _ptr(X), int(N), _ptr(out)),
                    "okf_gemm_tile")

    def dequant_row(self, w: QuantTensor, out, n: int):
        wc = w.c()
        self._check(self._lib.okf_dequant_row(self.h, ctypes.byref(wc), int(n), _ptr(out)),
                    "okf_dequant_row")

    @contextlib.contextmanager
    def parallel(self):
        """MetalEnc.parallel (``LLM/Base/MetalEnc.swift:42-47``): the matvecs
        issued inside carry no order among themselves and launch together."""
        self._check(self._lib.okf_parallel_begin(self.h), "okf_parallel_begin")
        try:
            yield self
        finally:
            self._check(self._lib.okf_parallel_end(self.h), "okf_parallel_end")

    def embed_batch(self, w: QuantTensor, ids, N: int, out):
        """out[n] = dequantized row ids[n] of w (MetalEnc.embedBatch)."""
        wc = w.c()
        self._check(self._lib.okf_embed_batch(self.h, ctypes.byref(wc), _ptr(ids), int(N), _ptr(out)),
                    "okf_embed_batch")

    def add_rmsnorm(self, x, r, w, y, n: int, rows: int, eps: float):
        """x += r; y = rmsnorm(x) * w per row (MetalEnc.addRmsnormBatch);
        r = None is MetalEnc.rmsnormBatch."""
        self._check(self._lib.okf_add_rmsnorm_batch(self.h, _ptr(x), _ptr(r), _ptr(w), _ptr(y), int(n),
                                                    int(rows), float(eps)), "okf_add_rmsnorm_batch")

    def argmax_rows(self, x, n: int, rows: int, out):
        """out[row] = argmax of row (MetalEnc.argmaxRows)."""
        self._check(self._lib.okf_argmax_rows(self.h, _ptr(x), int(n), int(rows), _ptr(out)),
                    "okf_argmax_rows")

    def argmax_rows_noalloc(self, x, n: int, rows: int, out):
        """okf_argmax_rows on the library's fixed device scratch (allocates nothing)."""
        self._check(self._lib.okf_argmax_rows_noalloc(self.h, _ptr(x), int(n), int(rows), _ptr(out)),
                    "okf_argmax_rows_noalloc")

    def stream_read(self, p, nbytes: int, out):
        """okf_stream_read: out[0] ^= xor of the nbytes at p (a measurement kernel)."""
        self._check(self._lib.okf_stream_read(self.h, _ptr(p), int(nbytes), _ptr(out)), "okf_stream_read")

    def reserve(self, gemm_nk: int, argmax_n: int, argmax_rows: int):
        """okf_ctx_reserve: allocate the scratch now; later calls allocate nothing."""
        self._check(self._lib.okf_ctx_reserve(self.h, int(gemm_nk), int(argmax_n), int(argmax_rows)),
                    "okf_ctx_reserve")

    def sync(self):
        self._check(self._lib.okf_sync(self.h), "okf_sync")

    def set_fault_rate(self, rate: float, seed: int):
        self._check(self._lib.okf_set_fault_rate(self.h, float(rate), int(seed)), "okf_set_fault_rate")


class GGUF:
    """A GGUF file mapped and parsed by the library (okf_gguf_open), the
    counterpart of GGUF(path:) (``LLM/Base/GGUF.swift:99-151``)."""

    def __init__(self, path: str):
        self._lib = _lib()
        h = ctypes.c_void_p()
        rc = self._lib.okf_gguf_open(os.fsencode(path), ctypes.byref(h))
        if rc:
            raise OkfError(rc, "okf_gguf_open")
        self.h = h

    def close(self):
        if self.h:
            self._lib.okf_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _info(t: "OkfGGUFTensor") -> dict:
        return {"name": t.name.decode(), "dims": [int(t.dims[d]) for d in range(t.n_dims)],
                "type": int(t.ggml_type), "offset": int(t.offset), "bytes": int(t.bytes)}

    def tensors(self) -> list:
        n = ctypes.c_uint64()
        self._lib.okf_gguf_tensor_count(self.h, ctypes.byref(n))
        out = []
        for i in range(n.value):
            t = OkfGGUFTensor()
            self._lib.okf_gguf_tensor_at(self.h, i, ctypes.byref(t))
            out.append(self._info(t))
        return out

    def find(self, name: str):
        t = OkfGGUFTensor()
        rc = self._lib.okf_gguf_find(self.h, name.encode(), ctypes.byref(t))
        if rc == OKF_E_NOTFOUND:
            return None
        if rc:
            raise OkfError(rc, "okf_gguf_find")
        return self._info(t)

    def int(self, key: str):
        v = ctypes.c_int64()
        return v.value if self._lib.okf_gguf_kv_int(self.h, key.encode(), ctypes.byref(v)) == 0 else None

    def double(self, key: str):
        v = ctypes.c_double()
        return v.value if self._lib.okf_gguf_kv_double(self.h, key.encode(), ctypes.byref(v)) == 0 else None

    def string(self, key: str):
        p, n = ctypes.c_char_p(), ctypes.c_uint64()
        if self._lib.okf_gguf_kv_string(self.h, key.encode(), ctypes.byref(p), ctypes.byref(n)):
            return None
        return ctypes.string_at(p, n.value).decode()

    def data(self) -> bytes:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        self._lib.okf_gguf_data(self.h, ctypes.byref(p), ctypes.byref(n))
        return ctypes.string_at(p, n.value)

    def upload(self, enc: "Enc") -> int:
        """Device copy of the data region; returns its device address."""
        d = ctypes.c_void_p()
        rc = self._lib.okf_gguf_upload(enc.h, self.h, ctypes.byref(d))
        if rc:
            raise OkfError(rc, "okf_gguf_upload")
        return d.value

    def weight(self, name: str, device_base: int) -> "QuantTensor":
        """The okf_weight of a 2-D (or higher) tensor in an uploaded copy."""
        t = self.find(name)
        if t is None:
            raise KeyError(name)
        K = t["dims"][0]
        M = 1
        for d in t["dims"][1:]:
            M *= d
        return QuantTensor(device_base, K, M, t["type"], off=t["offset"])


__all__ = [
    "Q8_0", "Q4_K", "IQ2_XXS", "Q2_0", "Q4_0", "IQ4_NL", "Q5_K", "Q6_K", "IQ4_XS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S",
    "IQ1_S", "IQ1_M", "F32", "F16", "BF16", "Q2_K", "Q3_K", "NAMES", "BY_NAME", "block_elems", "row_bytes",
    "QuantTensor", "Enc", "OkfError", "OkfWeight", "OkfGGUFTensor", "GGUF", "lib", "EXPORTS", "LIB_PATH",
]
