"""Pins the oracle's Q/K head RMS norm + NeoX partial RoPE
(oracle_q_head_norm_rope / oracle_k_head_norm_rope, restating
src/math_util.rs:501-593).  The reference ships no vectors for these
functions, so they are checked against what the mathematics fixes:

* bf16 widening, exhaustively against torch.bfloat16;
* the inverse frequencies against theta^(-2i/r) evaluated in float64;
* position 0 (no rotation) against a float64 RMS norm written with
  numpy.linalg.norm;
* any position against the rotation written as a complex multiplication
  (x_d + i x_{d+r/2}) * exp(i * theta_d), a different formula that a swapped
  sign, a wrong partner index or a wrong frequency index fails;
* the defining property of RoPE: q(p1) . k(p2) depends on p1 - p2 only;
* dims >= rotary_dim pass through the norm untouched, the gate half is a
  copy, and the Q and K functions agree on the same head data."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

H, G, D, R = 16, 2, 256, 64
THETA, EPS = 1e7, 1e-6


def bf16_bits(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


def bf16_vals(bits):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()


def test_bf16_widening_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    ours = np.array([O.lib().oracle_bf16_to_f32(int(b)) for b in bits], np.float32)
    ref = bf16_vals(bits)
    np.testing.assert_array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_inv_freq_closed_form():
    f = O.rope_inv_freq(THETA, R).astype(np.float64)
    i = np.arange(R // 2)
    ref = THETA ** (-2.0 * i / R)
    assert f[0] == 1.0
    np.testing.assert_allclose(f, ref, rtol=2e-7)


def _rms_norm64(x, w):
    x = x.astype(np.float64)
    rms = np.linalg.norm(x, axis=-1, keepdims=True) / np.sqrt(x.shape[-1])
    return x / np.sqrt(rms ** 2 + EPS) * w


def _rope_complex64(y, pos, rot=R):
    """NeoX rotation as a complex product, angles from the oracle's f32
    theta = f32(pos) * inv_freq (the rounding the reference performs)."""
    inv = O.rope_inv_freq(THETA, rot)
    theta = (np.float32(pos) * inv).astype(np.float64)
    h = rot // 2
    z = (y[..., :h] + 1j * y[..., h:rot]) * np.exp(1j * theta)
    out = y.copy()
    out[..., :h] = z.real
    out[..., h:rot] = z.imag
    return out


@pytest.fixture
def data():
    rng = np.random.default_rng(7)
    q_proj = rng.standard_normal((H, 2 * D)).astype(np.float32) * 3
    k = rng.standard_normal((G, D)).astype(np.float32) * 0.5
    qw = bf16_bits(1.0 + 0.3 * rng.standard_normal(D))
    kw = bf16_bits(1.0 + 0.3 * rng.standard_normal(D))
    return q_proj, k, qw, kw


def test_position_zero_is_plain_rms_norm(data):
    q_proj, k, qw, kw = data
    q, gate = O.q_head_norm_rope(q_proj, qw, 0)
    np.testing.assert_allclose(q, _rms_norm64(q_proj[:, :D], bf16_vals(qw)), rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(gate, q_proj[:, D:])
    kk = O.k_head_norm_rope(k, kw, 0)
    np.testing.assert_allclose(kk, _rms_norm64(k, bf16_vals(kw)), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("pos", [1, 7, 4095, 32767, 65535])
def test_rotation_matches_complex_form(data, pos):
    q_proj, k, qw, kw = data
    q, _ = O.q_head_norm_rope(q_proj, qw, pos)
    ref = _rope_complex64(_rms_norm64(q_proj[:, :D], bf16_vals(qw)), pos)
    np.testing.assert_allclose(q, ref, rtol=0, atol=2e-5 * np.abs(ref).max())
    kk = O.k_head_norm_rope(k, kw, pos)
    refk = _rope_complex64(_rms_norm64(k, bf16_vals(kw)), pos)
    np.testing.assert_allclose(kk, refk, rtol=0, atol=2e-5 * np.abs(refk).max())
    # columns past rotary_dim are the plain norm
    np.testing.assert_allclose(q[:, R:], _rms_norm64(q_proj[:, :D], bf16_vals(qw))[:, R:],
                               rtol=1e-5, atol=1e-5)


def test_other_rotary_dims(data):
    q_proj, k, qw, kw = data
    for rot in (0, 8, 128, 256):
        q = np.empty(H * D, np.float32)
        g = np.empty(H * D, np.float32)
        O.lib().oracle_q_head_norm_rope(O._p(np.ascontiguousarray(q_proj)), O._p(qw), O._p(q),
                                        O._p(g), H, D, rot, THETA, 123, EPS)
        y = _rms_norm64(q_proj[:, :D], bf16_vals(qw))
        ref = _rope_complex64(y, 123, rot) if rot else y
        np.testing.assert_allclose(q.reshape(H, D), ref, rtol=0, atol=2e-5 * np.abs(ref).max())


def test_relative_position_property():
    """q(p1) . k(p2) over the rotated columns depends only on p1 - p2."""
    rng = np.random.default_rng(3)
    ones = bf16_bits(np.ones(D))
    qp = np.zeros((H, 2 * D), np.float32)
    qp[0, :D] = rng.standard_normal(D)
    kv = rng.standard_normal((G, D)).astype(np.float32)
    dots = []
    for p1, p2 in [(10, 3), (107, 100), (1007, 1000)]:
        q, _ = O.q_head_norm_rope(qp, ones, p1)
        kk = O.k_head_norm_rope(kv, ones, p2)
        dots.append(float(np.dot(q[0, :R].astype(np.float64), kk[0, :R])))
    np.testing.assert_allclose(dots, dots[0], rtol=0, atol=1e-4 * abs(dots[0]) + 1e-4)
    # and it does depend on the offset
    q, _ = O.q_head_norm_rope(qp, ones, 11)
    kk = O.k_head_norm_rope(kv, ones, 3)
    assert abs(float(np.dot(q[0, :R], kk[0, :R])) - dots[0]) > 1e-3


def test_q_and_k_forms_agree(data):
    q_proj, _, qw, _ = data
    for pos in (0, 5, 40000):
        q, _ = O.q_head_norm_rope(q_proj, qw, pos)
        heads = np.ascontiguousarray(q_proj[:, :D])
        kk = O.k_head_norm_rope(heads, qw, pos, G=H)
        np.testing.assert_array_equal(q, kk)


def test_norm_preserved_per_pair(data):
    q_proj, _, qw, _ = data
    y = _rms_norm64(q_proj[:, :D], bf16_vals(qw))
    q, _ = O.q_head_norm_rope(q_proj, qw, 9999)
    h = R // 2
    np.testing.assert_allclose(q[:, :h] ** 2 + q[:, h:R] ** 2, y[:, :h] ** 2 + y[:, h:R] ** 2,
                               rtol=1e-4, atol=1e-6)
