"""mi_attn_decode_ragged_noalloc (the ragged decode on the library's static
device scratch, for callers that cannot allocate) against the existing
entry point mi_attn_decode_ragged with a caller workspace, through the C
ABI: two calls in a row, the second with a smaller batch, bit for bit; a
batch beyond the scratch is refused with MI_ERR_UNSUPPORTED."""
import ctypes as C

import numpy as np
import pytest
import torch

from moe_infer_amd import _lib, kv_pack, ragged_workspace
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _case(rng, lengths):
    lengths = np.array(lengths, np.int32)
    offsets = np.zeros(len(lengths), np.int32)
    offsets[1:] = np.cumsum((lengths + 31) // 32 * 32)[:-1]
    rows = max(int(offsets[-1] + (lengths[-1] + 31) // 32 * 32), 32)
    k, v = f16(rng, rows, G * D), f16(rng, rows, G * D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    b = len(lengths)
    q, g = f16(rng, b, H, D), f16(rng, b, H, D)
    return dict(lengths=lengths, offsets=offsets, k=k, v=v, kb=kb, vb=vb, q=q, g=g,
                off_t=torch.from_numpy(offsets).cuda(), len_t=torch.from_numpy(lengths).cuda(),
                q_t=dev(q), g_t=dev(g), max_len=int(lengths.max()))


def _with_workspace(c):
    b = len(c["lengths"])
    out = torch.empty_like(c["q_t"])
    ws = ragged_workspace(b, c["max_len"])
    _lib.check(_lib.lib().mi_attn_decode_ragged(
        _p(c["kb"]), _p(c["vb"]), _p(c["off_t"]), _p(c["len_t"]), b, c["max_len"], H, G, D,
        _p(c["q_t"]), _p(c["g_t"]), _p(out), _p(ws), ws.numel(),
        C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    return out


def _noalloc(c, out=None):
    b = len(c["lengths"])
    out = torch.empty_like(c["q_t"]) if out is None else out
    st = _lib.lib().mi_attn_decode_ragged_noalloc(
        _p(c["kb"]), _p(c["vb"]), _p(c["off_t"]), _p(c["len_t"]), b, c["max_len"], H, G, D,
        _p(c["q_t"]), _p(c["g_t"]), _p(out), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st, out


def test_noalloc_ragged_matches_the_workspace_entry_point():
    announce("no-alloc ragged: two calls, second smaller")
    rng = np.random.default_rng(77)
    big = _case(rng, list(rng.integers(1, 20000, size=96)) + [0, 1, 31, 32, 33])
    small = _case(rng, [700, 5, 0, 4097, 33])
    st, out_big = _noalloc(big)
    _lib.check(st)
    torch.cuda.synchronize()
    st, out_small = _noalloc(small)  # the scratch still holds the first call's partials
    _lib.check(st)
    torch.cuda.synchronize()
    for name, c, out in (("big", big, out_big), ("small", small, out_small)):
        ref = _with_workspace(c)
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), name
    s = 4  # the oracle on a few sequences of the second call
    a, n = small["offsets"][s], small["lengths"][s]
    assert_close(host(out_small)[s], O.decode(small["q"][s], small["k"][a:a + n],
                                              small["v"][a:a + n], n, gate=small["g"][s]),
                 "no-alloc ragged seq 4 vs oracle")
    assert np.all(host(out_small)[2] == 0)  # length 0


def test_noalloc_ragged_rejects_a_batch_beyond_the_scratch():
    need = _lib.lib().mi_attn_ragged_workspace_size(4000, 1024, H, G, D)
    assert need > (16 << 20)
    rng = np.random.default_rng(5)
    c = _case(rng, [1, 2])
    st = _lib.lib().mi_attn_decode_ragged_noalloc(
        _p(c["kb"]), _p(c["vb"]), _p(c["off_t"]), _p(c["len_t"]), 4000, 1024, H, G, D,
        _p(c["q_t"]), _p(c["g_t"]), _p(c["q_t"]), None)
    assert st == _lib.MI_ERR_UNSUPPORTED
    assert b"scratch" in _lib.lib().mi_last_error()
