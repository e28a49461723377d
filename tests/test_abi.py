"""The C-ABI library loads, exports every entry point include/mi_attn.h
declares, and its host-side argument checks return status codes (no GPU
needed: every case below fails before any HIP call)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from moe_infer_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mi_attn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("mi_kv_create", "mi_kv_append", "mi_kv_set_pos", "mi_kv_reset",
                 "mi_attn_decode", "mi_attn_prefill", "mi_attn_verify", "mi_attn_decode_ragged",
                 "mi_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    bound = {n for n, _, _ in _lib.SIGNATURES}
    assert set(names) == bound, "ctypes signatures and header differ"


def test_peaks_and_version():
    assert _lib.peaks() == (8000.0, 2500.0)
    assert b"gfx950" in _lib.lib().mi_version()


def test_host_side_errors_without_gpu():
    lib = _lib.lib()
    h = C.c_void_p()
    assert lib.mi_kv_create(1, 16, 2, 128, 64, C.byref(h)) == _lib.MI_ERR_UNSUPPORTED
    assert b"head_dim" in lib.mi_last_error()
    assert lib.mi_kv_create(1, 16, 3, 256, 64, C.byref(h)) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_kv_create(0, 16, 2, 256, 64, C.byref(h)) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_kv_create(1, 16, 2, 256, 64, None) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_kv_set_pos(None, 0) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_attn_decode(None, 0, None, None, None, 1, None) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_attn_prefill(None, 0, None, None, None, None, None, 0, 4, None) == \
        _lib.MI_ERR_INVALID_ARG
    assert lib.mi_attn_decode_ragged(None, None, None, None, 1, 1, 16, 2, 256, None, None, None,
                                     None, 0, None) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_attn_decode_ragged(None, None, None, None, 1, 1, 16, 2, 64, None, None, None,
                                     None, 0, None) == _lib.MI_ERR_UNSUPPORTED
    fake = C.c_void_p(256)  # never dereferenced: the argument checks come first
    assert lib.mi_attn_decode_ragged(fake, fake, fake, fake, 70000, 1, 16, 2, 256, fake, None,
                                     fake, fake, 1 << 20, None) == _lib.MI_ERR_UNSUPPORTED
    assert b"65535" in lib.mi_last_error()
    with pytest.raises(_lib.MiValueError):
        _lib.check(lib.mi_kv_set_pos(None, 0))
    # the MFMA ceiling probe checks its arguments before launching
    assert lib.mi_bench_mfma_ceiling(None, 1, 1, None, None, None) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_bench_mfma_ceiling(fake, 0, 1, fake, fake, None) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_bench_mfma_ceiling(fake, 1, 0, fake, fake, None) == _lib.MI_ERR_INVALID_ARG
