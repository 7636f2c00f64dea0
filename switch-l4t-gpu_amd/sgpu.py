"""ctypes binding of libswitchgpu.so (include/switch_gpu.h) for Python callers.

The library is the product: every function here is a thin typed wrapper over one C-ABI
entry point, plus numpy conveniences (DeviceArray).  Loading fails loudly if the built
library is missing; there is no fallback path.
"""
from __future__ import annotations

import ctypes as ct
import os
import re

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libswitchgpu.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "switch_gpu.h")

SGPU_OK = 0
SGPU_ERR_INVALID_ARG = -1
SGPU_ERR_NOT_INITIALIZED = -2
SGPU_ERR_NO_KERNEL = -3
SGPU_ERR_NO_DEVICE = -4
SGPU_ERR_HOST_ALLOC = -5
SGPU_ERR_NO_WORKSPACE = -6
SGPU_ERR_SCRATCH_LIMIT = -7


class SgpuError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: status {status} ({error_string(status)})")


class DeviceProps(ct.Structure):
    _fields_ = [("name", ct.c_char * 256), ("arch", ct.c_char * 64), ("compute_units", ct.c_int),
                ("clock_khz", ct.c_int), ("memory_clock_khz", ct.c_int), ("memory_bus_width", ct.c_int),
                ("total_mem", ct.c_size_t), ("lds_per_block", ct.c_size_t), ("l2_bytes", ct.c_int),
                ("warp_size", ct.c_int)]


class QwenCfg(ct.Structure):
    _fields_ = [("V", ct.c_int), ("C", ct.c_int), ("NL", ct.c_int), ("NH", ct.c_int), ("NKV", ct.c_int),
                ("HD", ct.c_int), ("FC", ct.c_int), ("CTX", ct.c_int), ("eps", ct.c_float), ("theta", ct.c_float)]


class Gpt2Cfg(ct.Structure):
    _fields_ = [("V", ct.c_int), ("C", ct.c_int), ("NL", ct.c_int), ("NH", ct.c_int), ("HD", ct.c_int),
                ("FC", ct.c_int), ("CTX", ct.c_int), ("eps", ct.c_float)]


_P, _I, _F, _S = ct.c_void_p, ct.c_int, ct.c_float, ct.c_size_t
_SIGS = {
    "sgpu_error_string": (ct.c_char_p, [_I]),
    "sgpu_init": (_I, [_I]),
    "sgpu_device_count": (_I, [ct.POINTER(_I)]),
    "sgpu_get_device_props": (_I, [_I, ct.POINTER(DeviceProps)]),
    "sgpu_malloc": (_I, [ct.POINTER(_P), _S]),
    "sgpu_free": (_I, [_P]),
    "sgpu_memcpy_htod": (_I, [_P, _P, _S]),
    "sgpu_memcpy_dtoh": (_I, [_P, _P, _S]),
    "sgpu_memcpy_dtod": (_I, [_P, _P, _S]),
    "sgpu_memcpy_dtod_async": (_I, [_P, _P, _S, _P]),
    "sgpu_memset_d8": (_I, [_P, _I, _S]),
    "sgpu_synchronize": (_I, []),
    "sgpu_stream_synchronize": (_I, [_P]),
    "sgpu_event_create": (_I, [ct.POINTER(_P)]),
    "sgpu_event_destroy": (_I, [_P]),
    "sgpu_event_record": (_I, [_P, _P]),
    "sgpu_event_elapsed_ms": (_I, [ct.POINTER(_F), _P, _P]),
    "sgpu_code_object": (_P, [ct.c_char_p, ct.POINTER(_S)]),
    "sgpu_kernel_geometry": (_I, [ct.c_char_p, _I, _I, _I, ct.POINTER(ct.c_uint), ct.POINTER(ct.c_uint)]),
    "sgpu_sgemm_tiled": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_tiled4": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_opt": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_opt_plan": (ct.c_char_p, [_I, _I, _I, _I, ct.POINTER(_I)]),
    "sgpu_sgemm_opt256": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_kwave": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_kwave_edge": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_kwave128": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_sgemm_splitk": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "sgpu_sgemm_splitk_noalloc": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "sgpu_sgemm_small": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "sgpu_sgemm_naive": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "sgpu_membw_read4": (_I, [_P, _P, _I, _I, ct.POINTER(_I), _P]),
    "sgpu_stream_create": (_I, [_P]),
    "sgpu_stream_destroy": (_I, [_P]),
    "sgpu_graph_begin": (_I, [_P]),
    "sgpu_graph_end": (_I, [_P, _P]),
    "sgpu_graph_launch": (_I, [_P, _P]),
    "sgpu_graph_destroy": (_I, [_P]),
    "sgpu_gemv": (_I, [_P, _P, _P, _I, _I, _P]),
    "sgpu_gemv4": (_I, [_P, _P, _P, _I, _I, _P]),
    "sgpu_gemv_warp": (_I, [_P, _P, _P, _I, _I, _P]),
    "sgpu_gemv_warp_b": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "sgpu_gemv_multi": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "sgpu_gemv_h": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "sgpu_gemv_hh": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "sgpu_rmsnorm": (_I, [_P, _P, _P, _I, _F, _I, _P]),
    "sgpu_rope": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "sgpu_swiglu": (_I, [_P, _P, _P, _I, _P]),
    "sgpu_attn_scores_gqa": (_I, [_P, _P, _P, _I, _F, _I, _I, _I, _P]),
    "sgpu_attn_softmax": (_I, [_P, _P, _I, _I, _P]),
    "sgpu_attn_mix_gqa": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "sgpu_add2": (_I, [_P, _P, _P, _I, _P]),
    "sgpu_layernorm": (_I, [_P, _P, _P, _P, _I, _F, _I, _P]),
    "sgpu_gelu": (_I, [_P, _P, _I, _P]),
    "sgpu_add_bias": (_I, [_P, _P, _I, _P]),
    "sgpu_gpt2_attn_scores": (_I, [_P, _P, _P, _I, _F, _P]),
    "sgpu_gpt2_attn_softmax": (_I, [_P, _P, _I, _P]),
    "sgpu_gpt2_attn_mix": (_I, [_P, _P, _P, _I, _P]),
    "sgpu_gpt2_default_cfg": (None, [ct.POINTER(Gpt2Cfg)]),
    "sgpu_gpt2_file_floats": (_S, [ct.POINTER(Gpt2Cfg)]),
    "sgpu_gpt2_fill_random": (_I, [_P, ct.POINTER(Gpt2Cfg), ct.c_uint64, _F]),
    "sgpu_gpt2_create": (_I, [ct.POINTER(_P), ct.POINTER(Gpt2Cfg), _P]),
    "sgpu_gpt2_destroy": (None, [_P]),
    "sgpu_gpt2_forward": (_I, [_P, _I, _I, _I, _P, _I]),
    "sgpu_gpt2_forward_trace": (_I, [_P, _I, _I, _P, _P, _I]),
    "sgpu_gpt2_forward_stages": (_I, [_P, _I, _I, _P, _I, _P, _P]),
    "sgpu_gpt2_prefill": (_I, [_P, _P, _I, _P]),
    "sgpu_gpt2_set_path": (_I, [_P, _I]),
    "sgpu_gpt2_generate": (_I, [_P, _P, _I, _I, _P]),
    "sgpu_qwen_default_cfg": (None, [ct.POINTER(QwenCfg)]),
    "sgpu_qwen_file_bytes": (_S, [ct.POINTER(QwenCfg)]),
    "sgpu_qwen_fill_random": (_I, [_P, ct.POINTER(QwenCfg), ct.c_uint64, _F]),
    "sgpu_qwen_create": (_I, [ct.POINTER(_P), ct.POINTER(QwenCfg), _P]),
    "sgpu_qwen_destroy": (None, [_P]),
    "sgpu_qwen_forward": (_I, [_P, _I, _I, _I, _P]),
    "sgpu_qwen_forward_trace": (_I, [_P, _I, _I, _P, _P]),
    "sgpu_qwen_device_logits": (_P, [_P]),
    "sgpu_qwen_set_path": (_I, [_P, _I]),
    "sgpu_qwen_generate": (_I, [_P, _P, _I, _I, _P]),
    "sgpu_qwen_phase_times": (_I, [_P, _I, _I, _P]),
    "sgpu_qwen_forward_stages": (_I, [_P, _I, _I, _P, _P, _P]),
    "sgpu_qwen_prefill": (_I, [_P, _P, _I, _P]),
    "sgpu_gen_sgemm_inputs": (None, [_P, _P, _S, ct.c_uint]),
    "sgpu_frand": (_F, [ct.POINTER(ct.c_uint64)]),
    "sgpu_gen_uniform": (None, [_P, _S, ct.POINTER(ct.c_uint64), _F]),
    "sgpu_gen_normal": (None, [_P, _S, ct.POINTER(ct.c_uint64), _F, _F]),
    "sgpu_f32_to_f16": (None, [_P, _P, _S]),
    "sgpu_h2f_host": (_F, [ct.c_uint16]),
}

_lib = None


def lib() -> ct.CDLL:
    """Load libswitchgpu.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (__graft_entry__.build() or make -C)")
        L = ct.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of every function declared in include/switch_gpu.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sgpu_\w+)\s*\(", text)))


def error_string(status: int) -> str:
    return lib().sgpu_error_string(status).decode()


def check(status: int, where: str = "sgpu") -> None:
    if status != SGPU_OK:
        raise SgpuError(status, where)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def init(device: int = 0) -> None:
    call("sgpu_init", device)


def device_props(device: int = 0) -> DeviceProps:
    p = DeviceProps()
    call("sgpu_get_device_props", device, ct.byref(p))
    return p


def synchronize() -> None:
    call("sgpu_synchronize")


class DeviceArray:
    """A device allocation with a numpy dtype and shape (freed on close/GC)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ct.c_void_p()
        call("sgpu_malloc", ct.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_host(cls, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.shape, arr.dtype)
        if arr.nbytes:
            call("sgpu_memcpy_htod", d.ptr, arr.ctypes.data, arr.nbytes)
        return d

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("sgpu_memcpy_dtoh", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def fill_bytes(self, value: int) -> None:
        call("sgpu_memset_d8", self.ptr, value, self.nbytes)

    def offset(self, elems: int) -> int:
        """Device address of element `elems` (a byte offset, as the reference's sub-buffers)."""
        return self.ptr + elems * self.dtype.itemsize

    def close(self) -> None:
        if getattr(self, "ptr", None):
            lib().sgpu_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    """A HIP stream at the default priority (sgpu_stream_create)."""

    def __init__(self):
        h = ct.c_void_p()
        call("sgpu_stream_create", ct.byref(h))
        self.h = h.value

    def synchronize(self):
        call("sgpu_stream_synchronize", self.h)

    def close(self):
        if getattr(self, "h", None):
            lib().sgpu_stream_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """Launches recorded on a Stream and replayed as one graph launch:

        with Graph(stream) as g:
            call("sgpu_gemv_h", ..., stream.h)     # recorded, not run
        g.launch()
    """

    def __init__(self, stream: Stream):
        self.stream, self.h = stream, None

    def __enter__(self):
        call("sgpu_graph_begin", self.stream.h)
        return self

    def __exit__(self, exc_type, exc, tb):
        h = ct.c_void_p()
        rc = lib().sgpu_graph_end(self.stream.h, ct.byref(h))
        if exc_type is None:
            check(rc, "sgpu_graph_end")
        self.h = h.value
        return False

    def launch(self):
        call("sgpu_graph_launch", self.h, self.stream.h)

    def close(self):
        if getattr(self, "h", None):
            lib().sgpu_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Events:
    """A pair of HIP events for timing work on one stream."""

    def __init__(self):
        a, b = ct.c_void_p(), ct.c_void_p()
        call("sgpu_event_create", ct.byref(a))
        call("sgpu_event_create", ct.byref(b))
        self.start, self.stop = a.value, b.value

    def record_start(self, stream=None):
        call("sgpu_event_record", self.start, stream)

    def record_stop(self, stream=None):
        call("sgpu_event_record", self.stop, stream)

    def elapsed_ms(self) -> float:
        ms = ct.c_float()
        call("sgpu_event_elapsed_ms", ct.byref(ms), self.start, self.stop)
        return ms.value

    def __del__(self):
        try:
            lib().sgpu_event_destroy(self.start)
            lib().sgpu_event_destroy(self.stop)
        except Exception:
            pass


# ---- host-side generators (no device needed) ----
def gen_sgemm_inputs(count: int, seed: int = 42):
    A = np.empty(count, np.float32)
    B = np.empty(count, np.float32)
    lib().sgpu_gen_sgemm_inputs(A.ctypes.data, B.ctypes.data, count, seed)
    return A, B


def gen_uniform(n: int, state: int, offset: float = 0.0):
    out = np.empty(n, np.float32)
    s = ct.c_uint64(state)
    lib().sgpu_gen_uniform(out.ctypes.data, n, ct.byref(s), offset)
    return out, s.value


def gen_normal(n: int, state: int, mean: float = 0.0, std: float = 1.0):
    out = np.empty(n, np.float32)
    s = ct.c_uint64(state)
    lib().sgpu_gen_normal(out.ctypes.data, n, ct.byref(s), mean, std)
    return out, s.value


def frand(state: int):
    s = ct.c_uint64(state)
    v = lib().sgpu_frand(ct.byref(s))
    return v, s.value


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().sgpu_f32_to_f16(a.ctypes.data, out.ctypes.data, a.size)
    return out


def qwen_default_cfg() -> QwenCfg:
    c = QwenCfg()
    lib().sgpu_qwen_default_cfg(ct.byref(c))
    return c


def qwen_cfg(**kw) -> QwenCfg:
    c = qwen_default_cfg()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def qwen_random_blob(cfg: QwenCfg, seed: int, std: float = 0.02) -> np.ndarray:
    n = lib().sgpu_qwen_file_bytes(ct.byref(cfg))
    if n == 0:
        raise SgpuError(SGPU_ERR_INVALID_ARG, "sgpu_qwen_file_bytes")
    blob = np.empty(n, np.uint8)
    call("sgpu_qwen_fill_random", blob.ctypes.data, ct.byref(cfg), seed, std)
    return blob


STAGE_FN = ct.CFUNCTYPE(None, ct.c_void_p, ct.c_char_p, ct.POINTER(ct.c_float), ct.c_int)


def _stage_collector():
    """A stage callback for the *_forward_stages entry points and the ordered list it fills
    with (stage, copy of the vector)."""
    got = []

    def fn(ctx, tag, v, n):
        got.append((tag.decode(), np.ctypeslib.as_array(v, (n,)).copy()))

    return STAGE_FN(fn), got


QWEN_PATH_REFERENCE, QWEN_PATH_FUSED, QWEN_PATH_GRAPH = 0, 1, 2
QWEN_PHASES = ("qkv", "attention", "o", "gate_up", "down", "lm_head", "argmax_embed")


class QwenEngine:
    """sgpu_qwen_* engine: weights resident on the device, one forward per position."""

    def __init__(self, cfg: QwenCfg, blob: np.ndarray, path: int = QWEN_PATH_REFERENCE):
        self.cfg = cfg
        h = ct.c_void_p()
        call("sgpu_qwen_create", ct.byref(h), ct.byref(cfg), np.ascontiguousarray(blob).ctypes.data)
        self.h = h.value
        self.logits = np.empty(cfg.V, np.float32)
        call("sgpu_qwen_set_path", self.h, path)

    def set_path(self, path: int) -> None:
        call("sgpu_qwen_set_path", self.h, path)

    def generate(self, prompt, n_gen: int) -> np.ndarray:
        """Greedy ids: the argmax after the prompt and after each of n_gen generated positions."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen + 1, np.int32)
        call("sgpu_qwen_generate", self.h, p.ctypes.data, p.size, n_gen, out.ctypes.data)
        return out

    def forward(self, token: int, pos: int, want_logits: bool = True):
        call("sgpu_qwen_forward", self.h, token, pos, int(want_logits),
             self.logits.ctypes.data if want_logits else None)
        return self.logits if want_logits else None

    def forward_trace(self, token: int, pos: int):
        """The reference launch sequence for one position: (logits, residual after each layer)."""
        trace = np.empty((self.cfg.NL, self.cfg.C), np.float32)
        call("sgpu_qwen_forward_trace", self.h, token, pos, self.logits.ctypes.data, trace.ctypes.data)
        return self.logits, trace

    def forward_stages(self, token: int, pos: int):
        """The reference launch sequence with its layer-0 stage vectors (sgpu_qwen_forward_stages):
        (logits, [(stage, vector), ...] in launch order)."""
        cb, got = _stage_collector()
        call("sgpu_qwen_forward_stages", self.h, token, pos, self.logits.ctypes.data, ct.cast(cb, ct.c_void_p), None)
        return self.logits, got

    def phase_times(self, pos: int, reps: int = 20) -> dict:
        """In-graph us per launch of each decode phase at position pos (sgpu_qwen_phase_times)."""
        us = np.zeros(len(QWEN_PHASES), np.float32)
        call("sgpu_qwen_phase_times", self.h, pos, reps, us.ctypes.data)
        return {k: float(v) for k, v in zip(QWEN_PHASES, us)}

    def prefill(self, ids) -> np.ndarray:
        """Positions 0..len(ids)-1 in one batched pass; logits of the last row."""
        a = np.ascontiguousarray(ids, np.int32)
        call("sgpu_qwen_prefill", self.h, a.ctypes.data, a.size, self.logits.ctypes.data)
        return self.logits

    def close(self):
        if self.h:
            lib().sgpu_qwen_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gpt2_cfg(**kw) -> Gpt2Cfg:
    c = Gpt2Cfg()
    lib().sgpu_gpt2_default_cfg(ct.byref(c))
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def gpt2_random_weights(cfg: Gpt2Cfg, seed: int, amp: float = 0.03) -> np.ndarray:
    n = lib().sgpu_gpt2_file_floats(ct.byref(cfg))
    if n == 0:
        raise SgpuError(SGPU_ERR_INVALID_ARG, "sgpu_gpt2_file_floats")
    w = np.empty(n, np.float32)
    call("sgpu_gpt2_fill_random", w.ctypes.data, ct.byref(cfg), seed, amp)
    return w


GPT2_PATH_REFERENCE, GPT2_PATH_FUSED, GPT2_PATH_GRAPH = 0, 1, 2


class Gpt2Engine:
    """sgpu_gpt2_* engine: fp32 weights resident on the device."""

    def __init__(self, cfg: Gpt2Cfg, weights: np.ndarray, path: int = GPT2_PATH_REFERENCE):
        self.cfg = cfg
        h = ct.c_void_p()
        call("sgpu_gpt2_create", ct.byref(h), ct.byref(cfg), np.ascontiguousarray(weights, np.float32).ctypes.data)
        self.h = h.value
        self.logits = np.empty(cfg.V, np.float32)
        call("sgpu_gpt2_set_path", self.h, path)

    def set_path(self, path: int) -> None:
        call("sgpu_gpt2_set_path", self.h, path)

    def generate(self, prompt, n_gen: int) -> np.ndarray:
        """Greedy ids: the argmax after the prompt and after each of n_gen generated positions."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen + 1, np.int32)
        call("sgpu_gpt2_generate", self.h, p.ctypes.data, p.size, n_gen, out.ctypes.data)
        return out

    def forward(self, token: int, pos: int, want_logits: bool = True, fused: bool = False):
        call("sgpu_gpt2_forward", self.h, token, pos, int(want_logits),
             self.logits.ctypes.data if want_logits else None, int(fused))
        return self.logits if want_logits else None

    def forward_trace(self, token: int, pos: int, fused: bool = False):
        """The reference launch sequence for one position: (logits, residual after each layer)."""
        trace = np.empty((self.cfg.NL, self.cfg.C), np.float32)
        call("sgpu_gpt2_forward_trace", self.h, token, pos, self.logits.ctypes.data, trace.ctypes.data, int(fused))
        return self.logits, trace

    def forward_stages(self, token: int, pos: int, fused: bool = False):
        """The reference launch sequence with its layer-0 stage vectors (sgpu_gpt2_forward_stages):
        (logits, [(stage, vector), ...] in launch order)."""
        cb, got = _stage_collector()
        call("sgpu_gpt2_forward_stages", self.h, token, pos, self.logits.ctypes.data, int(fused),
             ct.cast(cb, ct.c_void_p), None)
        return self.logits, got

    def prefill(self, ids):
        a = np.ascontiguousarray(ids, np.int32)
        call("sgpu_gpt2_prefill", self.h, a.ctypes.data, a.size, self.logits.ctypes.data)
        return self.logits

    def close(self):
        if self.h:
            lib().sgpu_gpt2_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
