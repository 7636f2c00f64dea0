"""ctypes binding of oracle/liboracle.so -- the CPU golden models.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, to check results against (and, in the bench, the timed CPU baseline).  Nothing in
the product imports it.  Function-by-function citations of the reference lines it restates
are in golden.h / golden.c.
"""
from __future__ import annotations

import ctypes as ct
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")


class QwenCfg(ct.Structure):
    _fields_ = [("V", ct.c_int), ("C", ct.c_int), ("NL", ct.c_int), ("NH", ct.c_int), ("NKV", ct.c_int),
                ("HD", ct.c_int), ("FC", ct.c_int), ("CTX", ct.c_int), ("eps", ct.c_float), ("theta", ct.c_float)]


class Gpt2Cfg(ct.Structure):
    _fields_ = [("V", ct.c_int), ("C", ct.c_int), ("NL", ct.c_int), ("NH", ct.c_int), ("HD", ct.c_int),
                ("FC", ct.c_int), ("CTX", ct.c_int), ("eps", ct.c_float)]


_P, _I, _F, _S = ct.c_void_p, ct.c_int, ct.c_float, ct.c_size_t
_SIGS = {
    "og_h2f": (_F, [ct.c_uint16]),
    "og_sgemm": (None, [_P, _P, _P, _I, _I, _I]),
    "og_sgemm_rows": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "og_sgemm_verdict_bad": (_I, [_P, _P, _I, _I]),
    "og_gemv": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "og_gemv_h": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "og_gemv_h_fbias": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "og_gemv_hh": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "og_gemv_multi": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "og_rms": (None, [_P, _P, _P, _I, _F]),
    "og_qwen_file_bytes": (_S, [ct.POINTER(QwenCfg)]),
    "og_rope_tables": (None, [_I, _I, ct.c_double, _P, _P]),
    "og_qwen_forward": (_I, [ct.POINTER(QwenCfg), _P, _P, _P, _I, _I, _I, _P, _P, _I]),
    "og_argmax": (_I, [_P, _I]),
    "og_gpt2_file_floats": (_S, [ct.POINTER(Gpt2Cfg)]),
    "og_layernorm": (None, [_P, _P, _P, _P, _I, _F]),
    "og_gpt2_forward": (_I, [ct.POINTER(Gpt2Cfg), _P, _P, _P, _I, _I, _I, _P, _P, _I]),
}

_lib = None


def lib() -> ct.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run make -C oracle")
        L = ct.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def h2f(h: int) -> float:
    return lib().og_h2f(h)


def h2f_array(h: np.ndarray) -> np.ndarray:
    """og_h2f over an array (through a 65,536-entry table built from og_h2f itself)."""
    table = np.array([lib().og_h2f(i) for i in range(65536)], np.float32)
    return table[np.asarray(h, np.uint16)]


def sgemm(A, B, M, N, K):
    A, B = _f32(A), _f32(B)
    C = np.empty(M * N, np.float32)
    lib().og_sgemm(A.ctypes.data, B.ctypes.data, C.ctypes.data, M, N, K)
    return C.reshape(M, N)


def sgemm_rows(A, B, M, N, K, row0, row1, nthreads=1):
    """Rows [row0, row1) of C (the other rows are left as NaN)."""
    A, B = _f32(A), _f32(B)
    C = np.full(M * N, np.nan, np.float32)
    lib().og_sgemm_rows(A.ctypes.data, B.ctypes.data, C.ctypes.data, M, N, K, row0, row1, nthreads)
    return C.reshape(M, N)


def sgemm_verdict_bad(got, ref, M, N) -> int:
    got, ref = _f32(got), _f32(ref)
    return lib().og_sgemm_verdict_bad(got.ctypes.data, ref.ctypes.data, M, N)


def gemv(W, x, bias, K, N, nthreads=1):
    W, x = _f32(W), _f32(x)
    b = _f32(bias) if bias is not None else None
    y = np.empty(N, np.float32)
    lib().og_gemv(W.ctypes.data, x.ctypes.data, b.ctypes.data if b is not None else None, y.ctypes.data, K, N, nthreads)
    return y


def gemv_h(W16, x, bias16, K, N, nthreads=1):
    W16 = np.ascontiguousarray(W16, np.uint16)
    x = _f32(x)
    b = np.ascontiguousarray(bias16, np.uint16) if bias16 is not None else None
    y = np.empty(N, np.float32)
    lib().og_gemv_h(W16.ctypes.data, x.ctypes.data, b.ctypes.data if b is not None else None, y.ctypes.data, K, N,
                    nthreads)
    return y


def gemv_h_fbias(W16, x, bias, K, N, nthreads=1):
    W16 = np.ascontiguousarray(W16, np.uint16)
    x = _f32(x)
    b = _f32(bias) if bias is not None else None
    y = np.empty(N, np.float32)
    lib().og_gemv_h_fbias(W16.ctypes.data, x.ctypes.data, b.ctypes.data if b is not None else None, y.ctypes.data,
                          K, N, nthreads)
    return y


def gemv_hh(W16, x16, bias, K, N, nthreads=1):
    W16 = np.ascontiguousarray(W16, np.uint16)
    x16 = np.ascontiguousarray(x16, np.uint16)
    b = _f32(bias) if bias is not None else None
    y = np.empty(N, np.float32)
    lib().og_gemv_hh(W16.ctypes.data, x16.ctypes.data, b.ctypes.data if b is not None else None, y.ctypes.data,
                     K, N, nthreads)
    return y


def gemv_multi(W, X, bias, K, N, T, nthreads=1):
    W, X = _f32(W), _f32(X)
    b = _f32(bias) if bias is not None else None
    Y = np.empty(T * N, np.float32)
    lib().og_gemv_multi(W.ctypes.data, X.ctypes.data, b.ctypes.data if b is not None else None, Y.ctypes.data,
                        K, N, T, nthreads)
    return Y.reshape(T, N)


def rms(x, w16, eps):
    x = _f32(x)
    w16 = np.ascontiguousarray(w16, np.uint16)
    y = np.empty_like(x)
    lib().og_rms(x.ctypes.data, w16.ctypes.data, y.ctypes.data, x.size, eps)
    return y


def rope_tables(ctx, hd, theta):
    c = np.empty(ctx * (hd // 2), np.float32)
    s = np.empty_like(c)
    lib().og_rope_tables(ctx, hd, theta, c.ctypes.data, s.ctypes.data)
    return c.reshape(ctx, hd // 2), s.reshape(ctx, hd // 2)


def argmax(v) -> int:
    v = _f32(v)
    return lib().og_argmax(v.ctypes.data, v.size)


def qwen_cfg(V, C, NL, NH, NKV, HD, FC, CTX, eps=1e-6, theta=1e6) -> QwenCfg:
    return QwenCfg(V, C, NL, NH, NKV, HD, FC, CTX, eps, theta)


def qwen_file_bytes(cfg: QwenCfg) -> int:
    return lib().og_qwen_file_bytes(ct.byref(cfg))


class QwenGolden:
    """cpu_forward with its own fp32 KV cache."""

    def __init__(self, cfg: QwenCfg, blob: np.ndarray, nthreads: int = 1):
        self.cfg, self.blob, self.nthreads = cfg, np.ascontiguousarray(blob), nthreads
        kvd = cfg.NKV * cfg.HD
        self.kc = np.zeros(cfg.NL * cfg.CTX * kvd, np.float32)
        self.vc = np.zeros_like(self.kc)
        self.logits = np.empty(cfg.V, np.float32)

    def forward(self, token, pos, want_logits=True, trace=None):
        tr = trace.ctypes.data if trace is not None else None
        rc = lib().og_qwen_forward(ct.byref(self.cfg), self.blob.ctypes.data, self.kc.ctypes.data,
                                   self.vc.ctypes.data, token, pos, int(want_logits),
                                   self.logits.ctypes.data if want_logits else None, tr, self.nthreads)
        if rc != 0:
            raise ValueError("og_qwen_forward rejected its arguments")
        return self.logits.copy() if want_logits else None


def layernorm(x, w, b, eps=1e-5):
    x, w, b = _f32(x), _f32(w), _f32(b)
    y = np.empty_like(x)
    lib().og_layernorm(x.ctypes.data, w.ctypes.data, b.ctypes.data, y.ctypes.data, x.size, eps)
    return y


def gpt2_cfg(V=50257, C=768, NL=12, NH=12, HD=64, FC=3072, CTX=1024, eps=1e-5) -> Gpt2Cfg:
    return Gpt2Cfg(V, C, NL, NH, HD, FC, CTX, eps)


def gpt2_file_floats(cfg: Gpt2Cfg) -> int:
    return lib().og_gpt2_file_floats(ct.byref(cfg))


class Gpt2Golden:
    """GPT-2 cpu_forward with its own fp32 KV cache."""

    def __init__(self, cfg: Gpt2Cfg, weights: np.ndarray, nthreads: int = 1):
        self.cfg, self.w, self.nthreads = cfg, _f32(weights), nthreads
        self.kc = np.zeros(cfg.NL * cfg.CTX * cfg.C, np.float32)
        self.vc = np.zeros_like(self.kc)
        self.logits = np.empty(cfg.V, np.float32)

    def forward(self, token, pos, want_logits=True, trace=None):
        tr = trace.ctypes.data if trace is not None else None
        rc = lib().og_gpt2_forward(ct.byref(self.cfg), self.w.ctypes.data, self.kc.ctypes.data, self.vc.ctypes.data,
                                   token, pos, int(want_logits), self.logits.ctypes.data if want_logits else None,
                                   tr, self.nthreads)
        if rc != 0:
            raise ValueError("og_gpt2_forward rejected its arguments")
        return self.logits.copy() if want_logits else None
