"""The MFMA issue-ceiling probe (mi_bench_mfma_ceiling) that bench.py prices
the prefill against: its output is the sum of the four accumulation chains
each thread ran, so with operands whose products are exact in f32 it has a
closed form, and its clock readings give the issue rate (32 clocks per
v_mfma_f32_32x32x16_f16 when nothing else runs)."""
import ctypes as C

import numpy as np
import pytest
import torch

from moe_infer_amd import _lib

from .gpu_util import announce

pytestmark = pytest.mark.gpu


def test_mfma_ceiling_closed_form_and_issue_rate():
    announce("mfma ceiling probe")
    wgs, iters = 4, 64
    # A fragments all 1/8, B fragments all 1/4: every product is 1/32 and each
    # MFMA adds 16 of them (k = 16) to every accumulator element, so after
    # iters * 8 MFMAs over 4 chains each of the 64 accumulator values of a
    # thread holds iters * 2 * 16 / 32 and the thread's sum is 64 times that.
    ops = torch.empty(256, 12, 8, dtype=torch.float16)
    ops[:, :8, :] = 0.125
    ops[:, 8:, :] = 0.25
    ops = ops.cuda()
    out = torch.full((wgs * 256,), -1.0, dtype=torch.float32, device="cuda")
    clk = torch.zeros(2 * wgs, dtype=torch.int64, device="cuda")
    st = _lib.lib().mi_bench_mfma_ceiling(C.c_void_p(ops.data_ptr()), iters, wgs,
                                          C.c_void_p(out.data_ptr()), C.c_void_p(clk.data_ptr()),
                                          C.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st)
    torch.cuda.synchronize()
    expect = 64 * iters * 2 * 16 / 32
    assert torch.all(out == expect), (out.min().item(), out.max().item(), expect)
    c = clk.cpu().numpy().reshape(wgs, 2).astype(np.float64)
    assert np.all(c[:, 0] > 0) and np.all(c[:, 1] > 0)
    per_mfma = c[:, 0] / (iters * 8)
    # one wave per SIMD issuing back to back: 32 clocks each, plus loop and
    # timer overhead on so short a run
    assert np.all(per_mfma >= 31) and np.all(per_mfma < 64), per_mfma
