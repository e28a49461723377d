"""Pins the oracle's o_proj matvecs: matvec_bf16 (restating the Metal kernel
src/engine/shaders.metal:2392-2425) and dequant_matvec_4bit (restating
src/math_util.rs:14-57) against numpy float64 evaluations that decode the
weights independently (torch bf16 widening; a vectorised nibble unpack), and
against closed forms that fail on a wrong nibble order, a wrong group index
or a transposed weight."""
import numpy as np
import torch

from oracle import oracle as O


def bf16_bits(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


def bf16_vals(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(
        torch.bfloat16).float().numpy().astype(np.float64)


def test_matvec_bf16_matches_numpy():
    rng = np.random.default_rng(1)
    w = bf16_bits(rng.standard_normal((64, 512)) * 0.05)
    x = rng.standard_normal(512).astype(np.float32)
    ref = bf16_vals(w) @ x.astype(np.float64)
    out = O.matvec_bf16(w, x)
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-5 * np.abs(ref).max() + 1e-6)


def test_matvec_bf16_row_major_orientation():
    """Row r of W (not column r) multiplies x."""
    w = np.zeros((4, 16), np.uint16)
    w[2, 5] = bf16_bits(3.0)
    x = np.zeros(16, np.float32)
    x[5] = 2.0
    out = O.matvec_bf16(w, x)
    np.testing.assert_array_equal(out, [0, 0, 6, 0])


def unpack_nibbles(wp):
    """uint32 [out, in/8] -> int [out, in]: nibble n of word p is column 8p+n."""
    shifts = np.arange(8, dtype=np.uint32) * 4
    return ((wp[:, :, None] >> shifts) & 0xF).reshape(wp.shape[0], -1).astype(np.float64)


def test_dequant_matvec_matches_numpy():
    rng = np.random.default_rng(2)
    out_dim, in_dim, gs = 32, 1024, 64
    wp = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    sc = bf16_bits(rng.uniform(0.01, 0.1, (out_dim, in_dim // gs)))
    bi = bf16_bits(rng.uniform(-0.3, 0.3, (out_dim, in_dim // gs)))
    x = rng.standard_normal(in_dim).astype(np.float32)
    wf = unpack_nibbles(wp) * np.repeat(bf16_vals(sc), gs, axis=1) + \
        np.repeat(bf16_vals(bi), gs, axis=1)
    ref = wf @ x.astype(np.float64)
    out = O.dequant_matvec_4bit(wp, sc, bi, x, gs)
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5 * np.abs(ref).max() + 1e-5)


def test_dequant_nibble_order_and_groups():
    """A single nibble 5 at word 3, position 6 (column 30) of row 1 with scale
    2, bias 0.5 in group 0 (columns 0..31, group size 32) and zero x except
    column 30 and one column of group 1."""
    out_dim, in_dim, gs = 2, 64, 32
    wp = np.zeros((out_dim, in_dim // 8), np.uint32)
    wp[1, 3] = np.uint32(5 << (6 * 4))
    sc = bf16_bits(np.array([[1.0, 1.0], [2.0, 4.0]]))
    bi = bf16_bits(np.array([[0.0, 0.0], [0.5, -1.0]]))
    x = np.zeros(in_dim, np.float32)
    x[30] = 1.0
    x[40] = 1.0
    out = O.dequant_matvec_4bit(wp, sc, bi, x, gs)
    # row 1: column 30 -> 5*2 + 0.5; column 40 (group 1, nibble 0) -> 0*4 - 1
    np.testing.assert_array_equal(out, [0.0, 10.5 - 1.0])
