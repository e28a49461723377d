"""Pins the CPU oracle (oracle/attn_oracle.c) before it is trusted as the
checker of the HIP kernels.  The reference ships no attention golden vectors
(its only attention checks are end-to-end logit comparisons that need model
weights), so each oracle function is checked against what the mathematics
fixes: an independent library evaluation (numpy einsum + scipy softmax in
float64), closed forms chosen so that a dropped term, a wrong index or a
transposed operand fails, and exhaustive f16 conversion against numpy."""
import numpy as np
import pytest
from scipy.special import softmax as sp_softmax

from oracle import oracle as O

from .conftest import f16

H, G, D = 16, 2, 256


def lib_attention(q, k_rows, v_rows, seq_len, gate=None):
    """float64 attention by library routines: heads grouped by repeat."""
    q = q.astype(np.float64).reshape(H, D)
    k = k_rows.astype(np.float64).reshape(-1, G, D)[:seq_len]
    v = v_rows.astype(np.float64).reshape(-1, G, D)[:seq_len]
    kh = np.repeat(k, H // G, axis=1)        # [L, H, D]: q-head h uses KV head h // 8
    vh = np.repeat(v, H // G, axis=1)
    s = np.einsum("hd,lhd->hl", q, kh) / np.sqrt(D)
    p = sp_softmax(s, axis=1)
    out = np.einsum("hl,lhd->hd", p, vh)
    if gate is not None:
        out = out / (1.0 + np.exp(-gate.astype(np.float64).reshape(H, D)))
    return out


# ------------------------------------------------------------ f16 bits --

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    ours = O.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -25, 2.0 ** -24,
                  3 * 2.0 ** -26, np.inf, -np.inf, 5.96e-8, 6.1e-5], np.float32),
    ]).astype(np.float32)
    # every midpoint between adjacent halves (ties go to even)
    h = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    ours = O.f32_to_f16(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ------------------------------------------- the reference f32 functions --

def test_scores_softmax_values_match_library_f64(rng):
    L, max_seq = 37, 50
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal((max_seq, G * D)).astype(np.float32)
    v = rng.standard_normal((max_seq, G * D)).astype(np.float32)
    s = O.attention_scores_batched(q, k, H, G, D, L, max_seq).reshape(H, max_seq)
    qh = q.reshape(H, D).astype(np.float64)
    kk = k.reshape(max_seq, G, D).astype(np.float64)
    for h in range(H):  # head h reads KV head h // 8 (math_util.rs:330-331)
        ref = kk[:L, h // 8] @ qh[h] / 16.0
        np.testing.assert_allclose(s[h, :L], ref, rtol=1e-5, atol=1e-4)
    assert np.all(s[:, L:] == 0)  # rows past seq_len untouched
    p = O.attention_softmax_batched(s.ravel(), H, L, max_seq).reshape(H, max_seq)
    np.testing.assert_allclose(p[:, :L], sp_softmax(s[:, :L].astype(np.float64), axis=1),
                               rtol=1e-5, atol=1e-7)
    o = O.attention_values_batched(p.ravel(), v, H, G, D, L, max_seq).reshape(H, D)
    vv = v.reshape(max_seq, G, D).astype(np.float64)
    for h in range(H):
        np.testing.assert_allclose(o[h], p[h, :L].astype(np.float64) @ vv[:L, h // 8],
                                   rtol=1e-4, atol=1e-5)


def test_softmax_guard_and_empty():
    # seq_len 0: nothing touched, values zero-filled (math_util.rs:357, 372)
    s = np.full(H * 4, 3.0, np.float32)
    p = O.attention_softmax_batched(s, H, 0, 4)
    assert np.array_equal(p, s)
    o = O.attention_values_batched(p, np.ones((4, G * D), np.float32), H, G, D, 0, 4)
    assert np.all(o == 0)


def test_sigmoid_gate_closed_forms():
    out = np.linspace(-3, 3, 64).astype(np.float32)
    assert np.array_equal(O.sigmoid_gate(out, np.zeros(64, np.float32)), out * 0.5)
    big = O.sigmoid_gate(out, np.full(64, 100.0, np.float32))
    np.testing.assert_array_equal(big, out)
    tiny = O.sigmoid_gate(out, np.full(64, -100.0, np.float32))
    assert np.max(np.abs(tiny)) < 1e-40
    g = np.linspace(-5, 5, 64).astype(np.float32)
    np.testing.assert_allclose(O.sigmoid_gate(out, g), out / (1 + np.exp(-g.astype(np.float64))),
                               rtol=1e-6)


def test_kv_cache_append_copies_one_row():
    kv_dim = G * D
    kc = np.zeros((5, kv_dim), np.float32)
    vc = np.zeros((5, kv_dim), np.float32)
    k = np.arange(kv_dim, dtype=np.float32)
    O.kv_cache_append(k, -k, kc, vc, 3, kv_dim)
    assert np.array_equal(kc[3], k) and np.array_equal(vc[3], -k)
    assert not kc[[0, 1, 2, 4]].any() and not vc[[0, 1, 2, 4]].any()


# --------------------------------------------------- composed decode step --

@pytest.mark.parametrize("L", [1, 2, 33, 300])
def test_decode_matches_library_f64(rng, L):
    q, k, v, g = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D), f16(rng, H * D)
    ref = lib_attention(q, k, v, L, g)
    np.testing.assert_allclose(O.decode(q, k, v, L, gate=g), ref, rtol=0, atol=2e-5)
    np.testing.assert_allclose(O.decode_f64(q, k, v, L, gate=g), ref, rtol=0, atol=1e-12)
    np.testing.assert_allclose(O.decode(q, k, v, L), lib_attention(q, k, v, L), atol=2e-5)


def test_decode_closed_forms(rng):
    L = 40
    q, k, v = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D)
    vv = v.astype(np.float64).reshape(L, G, D)
    # (i) one row: out = V0 exactly, for every head of each group
    o = O.decode(q, k, v, 1)
    for h in range(H):
        assert np.array_equal(o[h], v[0].reshape(G, D)[h // 8].astype(np.float32))
    # (ii) all keys equal -> uniform weights -> mean of V over the window
    keq = np.tile(k[:1], (L, 1))
    o = O.decode(q, keq, v, L).astype(np.float64)
    for h in range(H):
        np.testing.assert_allclose(o[h], vv[:, h // 8].mean(0), atol=1e-5)
    # (iii) q = 0 -> mean of V
    o = O.decode(np.zeros(H * D, np.float16), k, v, L).astype(np.float64)
    for h in range(H):
        np.testing.assert_allclose(o[h], vv[:, h // 8].mean(0), atol=1e-5)
    # (iv) a dominant key selects its value row
    qq = np.zeros(H * D, np.float16)
    qq[:] = 1.0
    kd = np.zeros((L, G * D), np.float16)
    kd[17] = 4.0  # score 4*256/16 = 64 against 0: weight 1 - 1e-26
    o = O.decode(qq, kd, v, L)
    for h in range(H):
        np.testing.assert_allclose(o[h], v[17].reshape(G, D)[h // 8].astype(np.float32),
                                   atol=1e-6)


def test_decode_group_structure_and_permutation(rng):
    L = 64
    k, v = f16(rng, L, G * D), f16(rng, L, G * D)
    # identical q across the eight heads of a group -> identical outputs,
    # and the two groups read different KV heads
    q1 = f16(rng, D)
    q = np.tile(q1, H)
    o = O.decode(q, k, v, L)
    assert all(np.array_equal(o[h], o[0]) for h in range(8))
    assert all(np.array_equal(o[h], o[8]) for h in range(8, 16))
    assert not np.allclose(o[0], o[8])
    # non-causal decode is invariant to permuting the KV rows
    perm = rng.permutation(L)
    o2 = O.decode(q, k[perm], v[perm], L)
    np.testing.assert_allclose(o, o2, atol=2e-6)


def test_mtp_form_agrees_with_math_util_form(rng):
    L = 90
    q, k, v = (rng.standard_normal(s).astype(np.float32) for s in (H * D, (L, G * D), (L, G * D)))
    a = O.mtp_cpu_attention(q, k, v, H, G, D, L, 1.0 / 16.0)
    b = O.decode_f32_from_f32(q, None, k, v, H, G, D, L)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------- causal / ragged --

def test_causal_rows_equal_decode_at_growing_lengths(rng):
    past, n = 11, 6
    q, k, v, g = f16(rng, n, H, D), f16(rng, past + n, G * D), f16(rng, past + n, G * D), \
        f16(rng, n, H, D)
    o = O.causal(q, k, v, past, gate=g)
    for i in range(n):
        ref = lib_attention(q[i], k, v, past + i + 1, g[i])
        np.testing.assert_allclose(o[i], ref, atol=2e-5)
        # the row must not see the key after it: changing it changes nothing
    k2 = k.copy()
    k2[past + n - 1] = 7.0
    o2 = O.causal(q, k2, v, past, gate=g)
    np.testing.assert_array_equal(o[:-1], o2[:-1])
    assert not np.array_equal(o[-1], o2[-1])
    np.testing.assert_allclose(O.causal_f64(q, k, v, past, gate=g), o, atol=2e-5)


def test_ragged_is_independent_decodes(rng):
    lengths = np.array([5, 0, 17, 1], np.int32)
    offsets = np.array([0, 8, 8, 32], np.int32)
    rows = 40
    q, k, v = f16(rng, 4, H, D), f16(rng, rows, G * D), f16(rng, rows, G * D)
    o = O.decode_ragged(q, k, v, offsets, lengths)
    for s in range(4):
        a, n = offsets[s], lengths[s]
        if n == 0:
            assert np.all(o[s] == 0)
        else:
            np.testing.assert_allclose(o[s], lib_attention(q[s], k[a:a + n], v[a:a + n], n),
                                       atol=2e-5)


def test_cache_model_semantics():
    m = O.CacheModel(2, 4, 4)
    m.append(0, np.ones((3, 4)), 2 * np.ones((3, 4)), 0)
    assert m.len[0] == 3 and m.len[1] == 0
    m.set_pos(1)
    assert m.len == [1, 1] and m.pos == 1
    assert np.all(m.k[0][2] == 1)  # rollback keeps rows
    m.append(0, 5 * np.ones((5, 4)), np.zeros((5, 4)), 1)  # grows by doubling
    assert m.k[0].shape[0] == 8 and m.len[0] == 6 and np.all(m.k[0][0] == 1)
    m.reset()
    assert m.pos == 0 and m.len == [0, 0] and np.all(m.k[0][1] == 5)


@pytest.mark.parametrize("threads", [1, 3, 16])
def test_decode_baseline_heads_over_threads_same_bits(rng, threads):
    """The CPU baseline's OpenMP variant (query heads over threads) runs the
    same per-head loops: bit-equal to the single-threaded step, and close to
    the f64 decode."""
    H, G, D, L = 16, 2, 256, 300
    q, g = f16(rng, H * D), f16(rng, H * D)
    k, v = f16(rng, 512, G * D), f16(rng, 512, G * D)
    base = O.DecodeBaseline(q, k, v, g)
    one = base.run(L).copy()
    many = base.run_omp(L, threads).copy()
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
    ref = O.decode_f64(q, k[:L], v[:L], L, gate=g)
    assert np.max(np.abs(one - ref.reshape(H, D))) < 1e-5
