"""o_proj matvecs on the GPU (mi_matvec_bf16, mi_matvec_q4) against the
oracle's restatements of the reference's matvec_bf16
(src/engine/shaders.metal:2392-2425) and dequant_matvec_4bit
(src/math_util.rs:14-57), on the same f16 input widened to f32.

Both sides accumulate in f32 in different orders, so the bound is relative
to the output scale: max |gpu - ref| <= 1e-4 * max |ref| (the sum has 4096
terms; a dropped term or a wrong group/nibble is off by ~1e-2 of the scale or
more)."""
import numpy as np
import pytest
import torch

from moe_infer_amd import matvec_bf16, matvec_q4
from moe_infer_amd._lib import MiValueError
from oracle import oracle as O

from .gpu_util import announce, host

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _bf16(rng, *shape, scale=1.0):
    return torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(
        torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def _check(gpu, ref, what):
    g = host(gpu).astype(np.float64)
    r = ref.astype(np.float64)
    err = float(np.abs(g - r).max())
    scale = float(np.abs(r).max())
    print(f"[parity] {what}: max_abs={err:.3e} |ref|max={scale:.3e}", flush=True)
    assert np.all(np.isfinite(g)), what
    assert err <= TOL * scale + 1e-6, f"{what}: {err:.3e} > {TOL} * {scale:.3e}"


@pytest.mark.parametrize("out_dim,in_dim", [(2048, 4096), (37, 512), (1000, 1536), (8, 9216)])
def test_matvec_bf16(out_dim, in_dim):
    announce(f"matvec_bf16 {out_dim}x{in_dim}")
    rng = np.random.default_rng(out_dim + in_dim)
    w = _bf16(rng, out_dim, in_dim, scale=0.05)
    x = rng.standard_normal(in_dim).astype(np.float16)
    out = matvec_bf16(torch.from_numpy(x).cuda(), w.cuda())
    _check(out, O.matvec_bf16(_bits(w), x.astype(np.float32)), f"bf16 {out_dim}x{in_dim}")


@pytest.mark.parametrize("out_dim,in_dim,gs", [(2048, 4096, 64), (2048, 4096, 32),
                                                (45, 2048, 128), (300, 6144, 2048)])
def test_matvec_q4(out_dim, in_dim, gs):
    announce(f"matvec_q4 {out_dim}x{in_dim} gs={gs}")
    rng = np.random.default_rng(out_dim * 7 + gs)
    wp = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    sc = torch.from_numpy(rng.uniform(0.005, 0.02, (out_dim, in_dim // gs)).astype(
        np.float32)).to(torch.bfloat16)
    bi = torch.from_numpy(rng.uniform(-0.08, 0.0, (out_dim, in_dim // gs)).astype(
        np.float32)).to(torch.bfloat16)
    x = rng.standard_normal(in_dim).astype(np.float16)
    out = matvec_q4(torch.from_numpy(x).cuda(), torch.from_numpy(wp.view(np.int32)).cuda(),
                    sc.cuda(), bi.cuda(), group_size=gs)
    ref = O.dequant_matvec_4bit(wp, _bits(sc), _bits(bi), x.astype(np.float32), gs)
    _check(out, ref, f"q4 {out_dim}x{in_dim} gs={gs}")


def test_matvec_q4_single_nibble():
    """One nibble set per row at a known column: out[r] = (n * s + b) x[c] +
    b * (sum of x over the other columns of every group) — checked against the
    oracle, and row r only depends on row r's words (no transposition)."""
    announce("matvec_q4 single nibble")
    out_dim, in_dim, gs = 16, 2048, 64
    wp = np.zeros((out_dim, in_dim // 8), np.uint32)
    for r in range(out_dim):
        c = 97 * r + 5
        wp[r, c // 8] = np.uint32((r % 15 + 1) << (4 * (c % 8)))
    sc = torch.full((out_dim, in_dim // gs), 0.5, dtype=torch.bfloat16)
    bi = torch.zeros((out_dim, in_dim // gs), dtype=torch.bfloat16)
    x = np.arange(in_dim, dtype=np.float16) / np.float16(1024)
    out = host(matvec_q4(torch.from_numpy(x).cuda(), torch.from_numpy(wp.view(np.int32)).cuda(),
                         sc.cuda(), bi.cuda(), group_size=gs))
    expect = np.array([(r % 15 + 1) * 0.5 * float(x[97 * r + 5]) for r in range(out_dim)])
    np.testing.assert_allclose(out, expect, rtol=1e-6, atol=0)


def test_matvec_rejects():
    x = torch.zeros(1000, dtype=torch.float16, device="cuda")
    with pytest.raises(MiValueError):
        matvec_bf16(x, torch.zeros(4, 1000, dtype=torch.bfloat16, device="cuda"))
    x = torch.zeros(2048, dtype=torch.float16, device="cuda")
    wp = torch.zeros(4, 256, dtype=torch.int32, device="cuda")
    with pytest.raises(MiValueError):  # group size not a multiple of 32
        matvec_q4(x, wp, torch.zeros(4, 2048 // 48, dtype=torch.bfloat16, device="cuda"),
                  torch.zeros(4, 2048 // 48, dtype=torch.bfloat16, device="cuda"),
                  group_size=48)
