"""ctypes binding of libmi_attn.so (the C ABI in include/mi_attn.h).

The library is the only compute path: if it is missing or fails to load,
every call raises — there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmi_attn.so"

MI_OK = 0
MI_ERR_INVALID_ARG = 1
MI_ERR_OUT_OF_RANGE = 2
MI_ERR_OOM = 3
MI_ERR_HIP = 4
MI_ERR_UNSUPPORTED = 5

_STATUS_NAMES = {
    MI_ERR_INVALID_ARG: "MI_ERR_INVALID_ARG",
    MI_ERR_OUT_OF_RANGE: "MI_ERR_OUT_OF_RANGE",
    MI_ERR_OOM: "MI_ERR_OOM",
    MI_ERR_HIP: "MI_ERR_HIP",
    MI_ERR_UNSUPPORTED: "MI_ERR_UNSUPPORTED",
}

# (name, restype, argtypes) of every symbol the header declares.
P = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64
SZ = C.c_size_t
ST = C.c_int
SIGNATURES = [
    ("mi_last_error", C.c_char_p, []),
    ("mi_version", C.c_char_p, []),
    ("mi_roofline_peaks", None, [C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    ("mi_kv_create", ST, [I32, I32, I32, I32, I64, C.POINTER(P)]),
    ("mi_kv_destroy", None, [P]),
    ("mi_kv_reserve", ST, [P, I64]),
    ("mi_kv_capacity", ST, [P, C.POINTER(I64)]),
    ("mi_kv_shape", ST, [P, C.POINTER(I32), C.POINTER(I32), C.POINTER(I32), C.POINTER(I32)]),
    ("mi_kv_set_pos", ST, [P, I64]),
    ("mi_kv_reset", ST, [P]),
    ("mi_kv_pos", ST, [P, C.POINTER(I64)]),
    ("mi_kv_len", ST, [P, I32, C.POINTER(I64)]),
    ("mi_kv_set_len", ST, [P, I32, I64]),
    ("mi_kv_layer_ptrs", ST, [P, I32, C.POINTER(P), C.POINTER(P)]),
    ("mi_kv_append", ST, [P, I32, P, P, I64, I32, P]),
    ("mi_kv_upload", ST, [P, I32, P, P, I64, I64]),
    ("mi_kv_download", ST, [P, I32, P, P, I64, I64]),
    ("mi_kv_copy_from", ST, [P, P]),
    ("mi_attn_decode", ST, [P, I32, P, P, P, I64, P]),
    ("mi_attn_step", ST, [P, I32, P, P, P, P, P, I64, P]),
    ("mi_attn_prefill", ST, [P, I32, P, P, P, P, P, I64, I32, P]),
    ("mi_attn_verify", ST, [P, I32, P, P, P, P, P, I64, I32, P]),
    ("mi_attn_ragged_workspace_size", SZ, [I32, I32, I32, I32, I32]),
    ("mi_attn_decode_ragged", ST, [P, P, P, P, I32, I32, I32, I32, I32, P, P, P, P, SZ, P]),
    ("mi_attn_decode_ragged_noalloc", ST, [P, P, P, P, I32, I32, I32, I32, I32, P, P, P, P]),
    ("mi_kv_pack", ST, [P, P, P, P, I64, I64, I32, I32, P]),
    ("mi_qk_norm_rope_append", ST, [P, I32, P, P, P, P, P, I32, C.c_float, C.c_float, I64, I32,
                                    P, P, P]),
    ("mi_attn_step_proj", ST, [P, I32, P, P, P, P, P, I32, C.c_float, C.c_float, P, I64, P]),
    ("mi_matvec_bf16", ST, [P, P, P, I32, I32, P]),
    ("mi_matvec_q4", ST, [P, P, P, P, I32, P, I32, I32, P]),
    ("mi_prof_enable", None, [C.c_int]),
    ("mi_prof_read", ST, [C.c_char_p, C.POINTER(C.c_double), C.POINTER(I64)]),
    ("mi_bench_mfma_ceiling", ST, [P, I32, I32, P, P, P]),
]


class MiError(RuntimeError):
    """A failed mi_* call; `.status` holds the mi_status code."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class MiValueError(MiError, ValueError):
    """Invalid argument / out-of-range position (the reference maps such
    errors to PyValueError, src/python_bindings.rs:117)."""


_lib = None


def lib() -> C.CDLL:
    """Loads the library once; raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m moe_infer_amd.build` "
                "(or __graft_entry__.build()); there is no fallback path")
        handle = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != MI_OK:
        msg = lib().mi_last_error().decode(errors="replace")
        if status in (MI_ERR_INVALID_ARG, MI_ERR_OUT_OF_RANGE):
            raise MiValueError(status, msg)
        raise MiError(status, msg)


def peaks() -> tuple[float, float]:
    """(HBM GB/s, dense f16 MFMA TFLOP/s) the roofline fractions divide by."""
    h, f = C.c_double(), C.c_double()
    lib().mi_roofline_peaks(C.byref(h), C.byref(f))
    return h.value, f.value


def prof_enable(on: bool) -> None:
    lib().mi_prof_enable(1 if on else 0)


def prof_read(kernel: str) -> tuple[float, int]:
    """(mean microseconds, launches) of `kernel` since prof_enable."""
    us, n = C.c_double(), C.c_int64()
    check(lib().mi_prof_read(kernel.encode(), C.byref(us), C.byref(n)))
    return us.value, n.value
