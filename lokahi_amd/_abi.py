"""ctypes binding of libstrata_hip.so (the C ABI declared in include/strata_hip.h).

Loading fails loudly: if the library is missing or the device is not gfx950
the caller gets an exception; there is no CPU fallback anywhere in this
package.  ``STRATA_HIP_LIB`` overrides the library path.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libstrata_hip.so"

STRATA_OK = 0
STRATA_EHIP = -5
STRATA_ENOMEM = -12
STRATA_EINVAL = -22
STRATA_ENOTSUP = -95

F32 = 0
BF16 = 1

c_void_pp = C.POINTER(C.c_void_p)


class StrataError(RuntimeError):
    """A HIP/runtime failure inside the library (not a caller error)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"strata error {code}: {message}")
        self.code = code


class Q4Weight(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("N", C.c_int64), ("y", C.c_void_p)]


class LlamaConfigC(C.Structure):
    _fields_ = [("vocab_size", C.c_int), ("hidden_size", C.c_int), ("intermediate_size", C.c_int),
                ("num_layers", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("group_size", C.c_int), ("rms_norm_eps", C.c_float),
                ("rope_theta", C.c_float)]


class LlamaLayerC(C.Structure):
    _fields_ = [("input_norm", C.c_void_p), ("post_norm", C.c_void_p), ("q", Q4Weight),
                ("k", Q4Weight), ("v", Q4Weight), ("o", Q4Weight), ("gate", Q4Weight),
                ("up", Q4Weight), ("down", Q4Weight)]


_SIGS = {
    "strata_abi_version": ([], C.c_int),
    "strata_last_error": ([], C.c_char_p),
    "strata_ctx_create": ([C.c_int, c_void_pp], C.c_int),
    "strata_ctx_destroy": ([C.c_void_p], C.c_int),
    "strata_selftest": ([C.c_void_p, C.c_char_p, C.c_size_t], C.c_int),
    "strata_linear_q4": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p,
                          C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p,
                          C.c_int, C.c_void_p], C.c_int),
    "strata_linear_q4_multi": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int64,
                                C.POINTER(Q4Weight), C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_void_p], C.c_int),
    "strata_q4_layout_create": ([C.c_void_p, C.POINTER(Q4Weight), C.c_int, C.c_int64, c_void_pp],
                                C.c_int),
    "strata_q4_layout_destroy": ([C.c_void_p], C.c_int),
    "strata_bench_read": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p,
                           C.c_void_p], C.c_int),
    "strata_linear_q4_layout": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_void_p,
                                 C.POINTER(C.c_void_p), C.c_int, C.c_void_p], C.c_int),
    "strata_linear_bf16": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p,
                            C.c_int64, C.c_void_p, C.c_int, C.c_void_p], C.c_int),
    "strata_rope": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                     C.c_int, C.c_int, C.c_float, C.c_int, C.c_void_p], C.c_int),
    "strata_attn_gqa": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                         C.c_int, C.c_int64, C.c_int64, C.c_void_p, C.c_int, C.c_int, C.c_int,
                         C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                         C.c_void_p, C.c_void_p], C.c_int),
    "strata_attn_gqa_noalloc": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                 C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p, C.c_int,
                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                 C.c_int, C.c_float, C.c_void_p, C.c_void_p], C.c_int),
    "strata_kv_create": ([C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                          C.c_void_p, C.c_void_p, c_void_pp], C.c_int),
    "strata_kv_destroy": ([C.c_void_p], C.c_int),
    "strata_kv_append": ([C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                          C.c_void_p], C.c_int),
    "strata_rope_kv_append": ([C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                               C.c_int, C.c_int, C.c_int, C.c_float, C.c_void_p, C.c_void_p],
                              C.c_int),
    "strata_kv_view": ([C.c_void_p, C.c_int, c_void_pp, c_void_pp, C.POINTER(C.c_int64),
                        C.POINTER(C.c_int64), C.POINTER(C.c_int)], C.c_int),
    "strata_kv_len": ([C.c_void_p, C.c_int, C.POINTER(C.c_int)], C.c_int),
    "strata_kv_clear": ([C.c_void_p], C.c_int),
    "strata_rmsnorm": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                        C.c_float, C.c_void_p, C.c_void_p], C.c_int),
    "strata_silu_mul": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p],
                        C.c_int),
    "strata_add": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p],
                   C.c_int),
    "strata_embed": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_int64,
                      C.c_void_p, C.c_void_p], C.c_int),
    "strata_argmax": ([C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p],
                      C.c_int),
    "strata_quantize_q4": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_int,
                            C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "strata_decoder_create": ([C.c_void_p, C.POINTER(LlamaConfigC), C.c_void_p, C.c_void_p,
                               C.c_void_p, C.POINTER(LlamaLayerC), C.c_void_p, C.c_int, C.c_int,
                               c_void_pp], C.c_int),
    "strata_decoder_destroy": ([C.c_void_p], C.c_int),
    "strata_decoder_forward": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p],
                               C.c_int),
    "strata_decoder_generate": ([C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_float,
                                 C.c_int, C.c_void_p, C.c_void_p], C.c_int),
    "strata_kv_restore": ([C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                           C.c_void_p], C.c_int),
    "strata_decoder_set_lm_head_q4": ([C.c_void_p, C.POINTER(Q4Weight)], C.c_int),
    "strata_dequantize_q4": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                              C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p], C.c_int),
}

EXPORTED = tuple(_SIGS.keys())

_lib = None
_lock = threading.Lock()


def lib_path() -> Path:
    return Path(os.environ.get("STRATA_HIP_LIB", str(LIB_PATH)))


def load(path=None):
    """Load the library and declare every entry point's signature."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else lib_path()
        if not p.exists():
            raise OSError(f"libstrata_hip.so not found at {p}; run lokahi_amd.build first")
        lib = C.CDLL(str(p))
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)  # AttributeError if an entry point is missing
            fn.argtypes = args
            fn.restype = res
        if lib.strata_abi_version() != 2:
            raise OSError("libstrata_hip.so ABI version mismatch")
        if path is None:
            _lib = lib
        return lib


def last_error() -> str:
    return load().strata_last_error().decode(errors="replace")


def check(rc: int) -> None:
    """Map a status code to the reference's exception types."""
    if rc == STRATA_OK:
        return
    msg = last_error()
    if rc == STRATA_EINVAL:
        raise ValueError(msg)
    if rc == STRATA_ENOTSUP:
        raise NotImplementedError(msg)
    raise StrataError(rc, msg)


class Context:
    """Owns one strata_ctx bound to a HIP device."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = C.c_void_p()
        check(self.lib.strata_ctx_create(device, C.byref(h)))
        self.handle = h
        self.device = device

    def selftest(self) -> str:
        buf = C.create_string_buffer(1024)
        rc = self.lib.strata_selftest(self.handle, buf, len(buf))
        text = buf.value.decode()
        check(rc)
        return text

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self.lib.strata_ctx_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


_contexts = {}


def context(device: int = 0) -> Context:
    with _lock:
        ctx = _contexts.get(device)
    if ctx is None:
        ctx = Context(device)
        with _lock:
            _contexts.setdefault(device, ctx)
            ctx = _contexts[device]
    return ctx
