"""Fused Q/K head RMS norm + NeoX partial RoPE + KV append on the GPU
(mi_qk_norm_rope_append) against the oracle's restatement of
q_head_norm_rope / k_head_norm_rope (src/math_util.rs:501-593).

Tolerance: the kernel computes in f32 and rounds once to f16, so its Q and
K outputs must lie within one f16 unit in the last place of the oracle's
f32 value (a tighter bound than the path's max-abs 2e-3 / rel 1e-2, which
normed values up to ~9 would not meet through f16 rounding alone).  The
gate half and V are conversions of the input and must be bit-exact
(round-to-nearest-even f16).  Rows of the cache outside [pos, pos+n) must
be untouched."""
import numpy as np
import pytest
import torch

from moe_infer_amd import Cache, _lib, attn_decode, qk_norm_rope_append
from oracle import oracle as O

from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256
THETA, EPS = 1e7, 1e-6


def bf16_bits(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def inputs(rng, n):
    q_proj = (rng.standard_normal((n, H, 2 * D)) * 3).astype(np.float32)
    k = (rng.standard_normal((n, G, D)) * 0.5).astype(np.float32)
    v = rng.standard_normal((n, G, D)).astype(np.float32)
    qw = bf16_bits(1.0 + 0.3 * rng.standard_normal(D))
    kw = bf16_bits(1.0 + 0.3 * rng.standard_normal(D))
    return q_proj, k, v, qw, kw


def oracle_rows(q_proj, k, qw, kw, pos, rot=64):
    qwb = qw.view(torch.int16).numpy().view(np.uint16)
    kwb = kw.view(torch.int16).numpy().view(np.uint16)
    n = q_proj.shape[0]
    qs, ks = np.empty((n, H, D), np.float32), np.empty((n, G, D), np.float32)
    for t in range(n):
        qo = np.empty(H * D, np.float32)
        go = np.empty(H * D, np.float32)
        O.lib().oracle_q_head_norm_rope(O._p(np.ascontiguousarray(q_proj[t])), O._p(qwb),
                                        O._p(qo), O._p(go), H, D, rot, THETA, pos + t, EPS)
        qs[t] = qo.reshape(H, D)
        kb = np.ascontiguousarray(k[t]).reshape(-1).copy()
        O.lib().oracle_k_head_norm_rope(O._p(kb), O._p(kwb), G, D, rot, THETA, pos + t, EPS)
        ks[t] = kb.reshape(G, D)
    return qs, ks


def assert_within_one_ulp(gpu_f16, ref_f32, what):
    g = np.asarray(gpu_f16, np.float16).astype(np.float64)
    r = np.asarray(ref_f32, np.float64).reshape(g.shape)
    ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float64)
    err = np.abs(g - r)
    worst = float((err / ulp).max())
    print(f"[parity] {what}: max err {err.max():.3e}, {worst:.3f} f16 ulp", flush=True)
    assert worst <= 1.0, f"{what}: {worst:.3f} f16 ulp from the oracle"


def f16_bits(x):
    return O.f32_to_f16(np.asarray(x, np.float32))


def run_case(pos, n, rot=64, seed=0, prefill_rows=0):
    announce(f"qk_norm_rope pos={pos} n={n} rot={rot}")
    rng = np.random.default_rng(seed + pos + n + rot)
    q_proj, k, v, qw, kw = inputs(rng, n)
    c = Cache(num_layers=1, capacity=max(256, pos + n))
    if prefill_rows:
        kp = rng.standard_normal((prefill_rows, G * D)).astype(np.float16)
        vp = rng.standard_normal((prefill_rows, G * D)).astype(np.float16)
        c.upload(0, kp, vp)
    q_out, g_out = qk_norm_rope_append(
        c, 0, torch.from_numpy(q_proj).cuda(), torch.from_numpy(k).cuda(),
        torch.from_numpy(v).cuda(), qw.cuda(), kw.cuda(), pos, rotary_dim=rot,
        rope_theta=THETA, eps=EPS)
    qr, kr = oracle_rows(q_proj, k, qw, kw, pos, rot)
    assert_within_one_ulp(host(q_out), qr, f"q pos={pos} n={n}")
    np.testing.assert_array_equal(host(g_out).view(np.uint16),
                                  f16_bits(q_proj[:, :, D:]).reshape(n, H, D))
    assert c.len(0) == pos + n
    kc, vc = c.download(0, rows=n, row0=pos)
    assert_within_one_ulp(kc, kr.reshape(n, G * D), f"k pos={pos} n={n}")
    np.testing.assert_array_equal(vc.view(np.uint16), f16_bits(v).reshape(n, G * D))
    if prefill_rows:
        lo = min(pos, prefill_rows)
        k0, v0 = c.download(0, rows=lo, row0=0) if lo else (kp[:0], vp[:0])
        np.testing.assert_array_equal(k0, kp[:lo])
        np.testing.assert_array_equal(v0, vp[:lo])
        hi = pos + n
        if hi < prefill_rows:
            k1, v1 = c.download(0, rows=prefill_rows - hi, row0=hi)
            np.testing.assert_array_equal(k1, kp[hi:])
            np.testing.assert_array_equal(v1, vp[hi:])
    c.close()
    return qr, kr, q_out, g_out


@pytest.mark.parametrize("pos", [0, 1, 31, 4095, 32767, 65535])
def test_single_token(pos):
    run_case(pos, 1)


@pytest.mark.parametrize("pos,n", [(0, 37), (100, 64), (5, 3), (4000, 300)])
def test_multi_token_inside_filled_cache(pos, n):
    run_case(pos, n, prefill_rows=pos + n + 40)


@pytest.mark.parametrize("rot", [0, 8, 128, 256])
def test_rotary_dims(rot):
    run_case(777, 5, rot=rot)


def test_grows_the_cache():
    announce("qk_norm_rope growth")
    rng = np.random.default_rng(11)
    c = Cache(num_layers=1, capacity=256)
    q_proj, k, v, qw, kw = inputs(rng, 2)
    qk_norm_rope_append(c, 0, torch.from_numpy(q_proj).cuda(), torch.from_numpy(k).cuda(),
                        torch.from_numpy(v).cuda(), qw.cuda(), kw.cuda(), 1000)
    assert c.capacity >= 1002 and c.len(0) == 1002
    _, kr = oracle_rows(q_proj, k, qw, kw, 1000)
    kc, vc = c.download(0, rows=2, row0=1000)
    assert_within_one_ulp(kc, kr.reshape(2, G * D), "k after growth")
    np.testing.assert_array_equal(vc.view(np.uint16), f16_bits(v).reshape(2, G * D))


def test_rejects_bad_rotary_dim():
    c = Cache(num_layers=1, capacity=256)
    rng = np.random.default_rng(1)
    q_proj, k, v, qw, kw = inputs(rng, 1)
    args = (c, 0, torch.from_numpy(q_proj).cuda(), torch.from_numpy(k).cuda(),
            torch.from_numpy(v).cuda(), qw.cuda(), kw.cuda(), 0)
    for rot in (12, -8, 264):
        with pytest.raises(_lib.MiValueError):
            qk_norm_rope_append(*args, rotary_dim=rot)
    assert c.len(0) == 0


def test_decode_chain_matches_oracle_chain():
    """T tokens through norm+rope+append, then decode of the last token:
    equal to the oracle's norm+rope (f16-rounded) followed by its decode."""
    announce("qk_norm_rope -> decode chain")
    rng = np.random.default_rng(5)
    T = 300
    q_proj, k, v, qw, kw = inputs(rng, T)
    c = Cache(num_layers=1, capacity=512)
    q_out, g_out = qk_norm_rope_append(
        c, 0, torch.from_numpy(q_proj).cuda(), torch.from_numpy(k).cuda(),
        torch.from_numpy(v).cuda(), qw.cuda(), kw.cuda(), 0)
    out = attn_decode(c, 0, q_out[T - 1].contiguous(), T, gate=g_out[T - 1].contiguous())
    qr, kr = oracle_rows(q_proj, k, qw, kw, 0)
    q16 = qr[T - 1].astype(np.float16)
    ref = O.decode(q16, kr.reshape(T, G * D).astype(np.float16),
                   v.reshape(T, G * D).astype(np.float16), T,
                   gate=q_proj[T - 1, :, D:].astype(np.float16))
    assert_close(out, ref, "norm-rope-append then decode")


# ---------------------------------------------- whole step from projections --

def step_proj_reference(q_proj, k, v, qw, kw, prev_k, prev_v, pos, rot=64):
    """Oracle chain of one step: norm + rope (f32), f16 rounding of q and of
    the cached rows, decode in f32, sigmoid gate with the f32 gate."""
    qr, kr = oracle_rows(q_proj[None], k[None], qw, kw, pos, rot)
    k_rows = np.concatenate([prev_k, kr.reshape(1, G * D).astype(np.float16)])
    v_rows = np.concatenate([prev_v, v.reshape(1, G * D).astype(np.float16)])
    att = O.decode(qr[0].astype(np.float16), k_rows, v_rows, pos + 1)
    return O.sigmoid_gate(att.reshape(-1), q_proj[:, D:].reshape(-1)).reshape(H, D), kr[0]


@pytest.mark.parametrize("pos", [0, 1, 31, 32, 1000, 32767])
def test_step_proj_matches_oracle_chain(pos):
    from moe_infer_amd import attn_step_proj
    announce(f"attn_step_proj pos={pos}")
    rng = np.random.default_rng(100 + pos)
    q_proj, k, v, qw, kw = inputs(rng, 1)
    prev_k = rng.standard_normal((pos, G * D)).astype(np.float16)
    prev_v = rng.standard_normal((pos, G * D)).astype(np.float16)
    c = Cache(num_layers=1, capacity=pos + 1)
    if pos:
        c.upload(0, prev_k, prev_v)
    out = attn_step_proj(c, 0, torch.from_numpy(q_proj[0]).cuda(), torch.from_numpy(k[0]).cuda(),
                         torch.from_numpy(v[0]).cuda(), qw.cuda(), kw.cuda(), pos)
    ref, kref = step_proj_reference(q_proj[0], k[0], v[0], qw, kw, prev_k, prev_v, pos)
    assert_close(out, ref, f"step_proj pos={pos}")
    assert c.len(0) == pos + 1
    kc, vc = c.download(0, rows=1, row0=pos)
    assert_within_one_ulp(kc, kref.reshape(1, G * D), f"step_proj k row pos={pos}")
    np.testing.assert_array_equal(vc.view(np.uint16), f16_bits(v[0]).reshape(1, G * D))
    if pos:
        k0, v0 = c.download(0, rows=pos, row0=0)
        np.testing.assert_array_equal(k0, prev_k)
        np.testing.assert_array_equal(v0, prev_v)


@pytest.mark.parametrize("rot", [0, 128, 256])
def test_step_proj_rotary_dims(rot):
    from moe_infer_amd import attn_step_proj
    announce(f"attn_step_proj rot={rot}")
    rng = np.random.default_rng(rot)
    pos = 300
    q_proj, k, v, qw, kw = inputs(rng, 1)
    prev_k = rng.standard_normal((pos, G * D)).astype(np.float16)
    prev_v = rng.standard_normal((pos, G * D)).astype(np.float16)
    c = Cache(num_layers=1, capacity=512)
    c.upload(0, prev_k, prev_v)
    out = attn_step_proj(c, 0, torch.from_numpy(q_proj[0]).cuda(), torch.from_numpy(k[0]).cuda(),
                         torch.from_numpy(v[0]).cuda(), qw.cuda(), kw.cuda(), pos,
                         rotary_dim=rot)
    ref, _ = step_proj_reference(q_proj[0], k[0], v[0], qw, kw, prev_k, prev_v, pos, rot)
    assert_close(out, ref, f"step_proj rot={rot}")


def test_step_proj_sequence_equals_two_kernel_route():
    """40 steps from an empty cache through attn_step_proj against the same
    40 tokens through mi_qk_norm_rope_append + attn_decode: equal caches
    (within one f16 ulp: host vs device sin/cos) and outputs within the
    contract tolerance of the oracle chain at the last step."""
    from moe_infer_amd import attn_step_proj
    announce("attn_step_proj sequence")
    rng = np.random.default_rng(77)
    T = 40
    q_proj, k, v, qw, kw = inputs(rng, T)
    c1 = Cache(num_layers=1, capacity=256)
    c2 = Cache(num_layers=1, capacity=256)
    for t in range(T):
        qp = torch.from_numpy(q_proj[t]).cuda()
        kt, vt = torch.from_numpy(k[t]).cuda(), torch.from_numpy(v[t]).cuda()
        out1 = attn_step_proj(c1, 0, qp, kt, vt, qw.cuda(), kw.cuda(), t)
        q2, g2 = qk_norm_rope_append(c2, 0, qp.reshape(1, H, 2 * D), kt.reshape(1, G, D),
                                     vt.reshape(1, G, D), qw.cuda(), kw.cuda(), t)
        out2 = attn_decode(c2, 0, q2[0].contiguous(), t + 1, gate=g2[0].contiguous())
    k1, v1 = c1.download(0)
    k2, v2 = c2.download(0)
    np.testing.assert_array_equal(v1, v2)
    d = np.abs(k1.astype(np.float64) - k2.astype(np.float64))
    assert float((d / np.spacing(np.abs(k2))).max()) <= 1.0
    qr, kr = oracle_rows(q_proj, k, qw, kw, 0)
    att = O.decode(qr[T - 1].astype(np.float16), kr.reshape(T, G * D).astype(np.float16),
                   v.reshape(T, G * D).astype(np.float16), T)
    ref = O.sigmoid_gate(att.reshape(-1), q_proj[T - 1, :, D:].reshape(-1))
    assert_close(out1, ref, "step_proj sequence last token")
    assert_close(out2, ref, "two-kernel route last token")


def test_step_proj_rejects_partial_slices():
    from moe_infer_amd import attn_step_proj
    rng = np.random.default_rng(2)
    q_proj, k, v, qw, kw = inputs(rng, 1)
    c = Cache(num_layers=1, capacity=256)
    with pytest.raises(_lib.MiError):
        attn_step_proj(c, 0, torch.from_numpy(q_proj[0]).cuda(), torch.from_numpy(k[0]).cuda(),
                       torch.from_numpy(v[0]).cuda(), qw.cuda(), kw.cuda(), 0, rotary_dim=32)
    assert c.len(0) == 0


@pytest.mark.parametrize("past,n", [(0, 200), (37, 130)])
def test_prefill_over_rope_appended_rows(past, n):
    """Batched prefill path: norm + RoPE + append of n tokens in one call,
    then mi_attn_prefill with k = v = NULL over the rows in place; equal to
    the oracle's norm + RoPE (f16-rounded) followed by its causal attention."""
    from moe_infer_amd import attn_prefill
    announce(f"rope -> prefill past={past} n={n}")
    rng = np.random.default_rng(past + n)
    q_proj, k, v, qw, kw = inputs(rng, n)
    prev_k = rng.standard_normal((past, G * D)).astype(np.float16)
    prev_v = rng.standard_normal((past, G * D)).astype(np.float16)
    c = Cache(num_layers=1, capacity=past + n)
    if past:
        c.upload(0, prev_k, prev_v)
        c.set_len(0, past)
    q_out, g_out = qk_norm_rope_append(
        c, 0, torch.from_numpy(q_proj).cuda(), torch.from_numpy(k).cuda(),
        torch.from_numpy(v).cuda(), qw.cuda(), kw.cuda(), past)
    out = attn_prefill(c, 0, q_out, None, None, past, gate=g_out)
    assert c.len(0) == past + n
    qr, kr = oracle_rows(q_proj, k, qw, kw, past)
    k_rows = np.concatenate([prev_k, kr.reshape(n, G * D).astype(np.float16)])
    v_rows = np.concatenate([prev_v, v.reshape(n, G * D).astype(np.float16)])
    ref = O.causal(qr.astype(np.float16), k_rows, v_rows, past,
                   gate=q_proj[:, :, D:].astype(np.float16))
    assert_close(out, ref, f"rope -> prefill past={past} n={n}")


def test_prefill_null_rows_must_be_present():
    from moe_infer_amd import attn_prefill
    c = Cache(num_layers=1, capacity=256)
    q = torch.zeros(4, H, D, dtype=torch.float16, device="cuda")
    with pytest.raises(_lib.MiValueError):
        attn_prefill(c, 0, q, None, None, 0)
