"""Causal batched prefill (MFMA flash-attention kernel) against the CPU
oracle of attn_sdpa_causal_n (src/engine/shaders.metal:2656-2769: query i
attends rows [0, past_pos + i]), through the C ABI."""
import numpy as np
import pytest

from moe_infer_amd import Cache, attn_decode, attn_prefill
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev, host

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256


@pytest.mark.parametrize("n,past", [(1, 0), (2, 0), (5, 3), (64, 0), (127, 0), (128, 0),
                                    (129, 0), (300, 0), (200, 77), (256, 64), (130, 1000)])
@pytest.mark.parametrize("gated", [True, False])
def test_prefill_matches_oracle(n, past, gated):
    announce(f"prefill n={n} past={past} gated={gated}")
    rng = np.random.default_rng(7 * n + past)
    kp, vp = f16(rng, past, G * D), f16(rng, past, G * D)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    c = Cache(num_layers=1, capacity=past + n)
    if past:
        c.upload(0, kp, vp)
        c.set_pos(past)
    out = attn_prefill(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g) if gated else None)
    kall, vall = np.concatenate([kp, k]), np.concatenate([vp, v])
    ref = O.causal(q, kall, vall, past, gate=g if gated else None)
    assert_close(out, ref, f"prefill n={n} past={past}")
    # the n new rows are in the cache, bit for bit
    assert c.len(0) == past + n
    kd, vd = c.download(0, rows=past + n)
    assert np.array_equal(kd.view(np.uint16), kall.view(np.uint16))
    assert np.array_equal(vd.view(np.uint16), vall.view(np.uint16))


def test_prefill_4k_sampled_rows_and_decode_consistency():
    """BASELINE config C4 (4096 tokens, past 0, seed 4): sampled rows
    against the oracle, and every sampled row equals a GPU decode of the
    same query at seq_len = i + 1 (size-independent property)."""
    announce("prefill C4 n=4096")
    n = 4096
    rng = np.random.default_rng(4)
    q, k, v = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D)
    c = Cache(num_layers=1, capacity=n)
    out = host(attn_prefill(c, 0, dev(q), dev(k), dev(v), 0))
    rows = [0, 1, 63, 64, 127, 128, 129, 1000, 2047, 2048, 3071, 4000, 4094, 4095]
    for i in rows:
        ref = O.decode(q[i].ravel(), k, v, i + 1)
        assert_close(out[i], ref, f"prefill C4 row {i}")
        dec = attn_decode(c, 0, dev(q[i].ravel()), i + 1)
        assert_close(out[i], host(dec).reshape(H, D), f"prefill C4 row {i} vs GPU decode",
                     atol=1e-3)
    assert np.all(np.isfinite(out))


def test_prefill_rising_scores():
    """Scores that rise by ~20 (base 2) per 64-key tile: the steady-state
    tiles exceed the running reference max far enough that the kernel must
    redo them with the new row max (its weights would leave f16 range), and
    the output stays on the oracle (the latest keys dominate)."""
    announce("prefill rising scores n=512")
    n = 512
    rng = np.random.default_rng(11)
    r = rng.standard_normal(D)
    r /= np.linalg.norm(r)
    q = np.tile((16.0 * r).astype(np.float16), (n, H, 1))   # every head: |q| = 16
    beta = 3.5                                               # q.k rises 3.5 per key
    t = np.arange(n, dtype=np.float64)[:, None]
    kh = (beta * t / 16.0) * r[None, :] + 0.05 * rng.standard_normal((n, D))
    k = np.concatenate([kh, kh], axis=1).astype(np.float16)
    v = f16(rng, n, G * D)
    c = Cache(num_layers=1, capacity=n)
    out = host(attn_prefill(c, 0, dev(q), dev(k), dev(v), 0))
    assert np.all(np.isfinite(out))
    for i in [0, 63, 64, 200, 255, 256, 383, 384, 447, 500, 511]:
        ref = O.decode(q[i].ravel(), k, v, i + 1)
        assert_close(out[i], ref, f"rising scores row {i}")


@pytest.mark.parametrize("past,n", [(308, 141), (200, 56), (31, 162)])
def test_prefill_cache_full_to_capacity(past, n):
    """The cache holds exactly past + n rows, rounded up to 256, and the
    last 64-key tile ends at the allocation's end.  Waves whose queries
    are all past n must not copy a K tile beyond it (they once did, in
    the steady-state schedule)."""
    announce(f"prefill full cache past={past} n={n}")
    rng = np.random.default_rng(past + 3 * n)
    kp, vp = f16(rng, past, G * D), f16(rng, past, G * D)
    q, k, v = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D)
    c = Cache(num_layers=1, capacity=past + n)
    assert c.capacity == (past + n + 255) // 256 * 256
    if past:
        c.upload(0, kp, vp)
        c.set_pos(past)
    out = attn_prefill(c, 0, dev(q), dev(k), dev(v), past)
    ref = O.causal(q, np.concatenate([kp, k]), np.concatenate([vp, v]), past)
    assert_close(out, ref, f"prefill full cache past={past} n={n}")


@pytest.mark.parametrize("past,n", [(32768, 257), (32768, 1000), (65000, 257), (65000, 1000),
                                    (0, 4095), (0, 4097)])
def test_prefill_long_past_and_c4_adjacent(past, n):
    """Chunked prefill after a long prompt (the engine's forward_batched with
    n > 16 at a large engine_pos, src/engine/qwen35_moe/batched.rs:233-260)
    and the sizes either side of C4: sampled rows against the oracle, and
    every row equal to a GPU decode of the same query at seq_len
    past + i + 1."""
    import torch
    from moe_infer_amd import kv_cache_append
    announce(f"prefill long past={past} n={n}")
    rng = np.random.default_rng(past + n)
    gen = torch.Generator(device="cuda").manual_seed(past + 7 * n)
    c = Cache(num_layers=1, capacity=past + n)
    if past:
        kp = torch.randn(past, G * D, generator=gen, device="cuda").half()
        vp = torch.randn(past, G * D, generator=gen, device="cuda").half()
        kv_cache_append(c, 0, kp, vp, 0)
        c.set_pos(past)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    qd, gd = dev(q), dev(g)
    out = host(attn_prefill(c, 0, qd, dev(k), dev(v), past, gate=gd))
    assert np.all(np.isfinite(out))
    kall, vall = c.download(0, rows=past + n)
    assert np.array_equal(kall[past:].view(np.uint16), k.view(np.uint16))
    assert np.array_equal(vall[past:].view(np.uint16), v.view(np.uint16))
    for i in sorted({0, 1, 63, 64, 127, 128, n // 2, n - 2, n - 1}):
        ref = O.decode(q[i].ravel(), kall, vall, past + i + 1, gate=g[i].ravel())
        assert_close(out[i], ref, f"prefill past={past} n={n} row {i}")
    dec = torch.empty(n, H, D, dtype=torch.float16, device="cuda")
    for i in range(n):
        attn_decode(c, 0, qd[i], past + i + 1, gate=gd[i], out=dec[i])
    assert_close(out, host(dec), f"prefill past={past} n={n}: all rows vs GPU decode",
                 atol=1e-3)


@pytest.mark.parametrize("n,past", [(1, 0), (129, 0), (200, 77), (300, 1000), (1000, 31)])
def test_prefill_32_query_kernel_matches(n, past, monkeypatch):
    """The earlier 32-queries-per-wave kernel (MI_ATTN_PREFILL_QPW=32, read
    at each call) against the oracle, and against the default 64-query
    kernel on the same inputs."""
    announce(f"prefill qpw=32 n={n} past={past}")
    rng = np.random.default_rng(3 * n + past)
    kp, vp = f16(rng, past, G * D), f16(rng, past, G * D)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    outs = []
    for qpw in ("32", "64"):
        monkeypatch.setenv("MI_ATTN_PREFILL_QPW", qpw)
        c = Cache(num_layers=1, capacity=past + n)
        if past:
            c.upload(0, kp, vp)
            c.set_pos(past)
        outs.append(host(attn_prefill(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g))))
    ref = O.causal(q, np.concatenate([kp, k]), np.concatenate([vp, v]), past, gate=g)
    assert_close(outs[0], ref, f"prefill qpw=32 n={n} past={past}")
    assert_close(outs[0], outs[1], f"prefill qpw=32 vs 64 n={n} past={past}", atol=1e-3)


def test_prefill_restart_after_late_large_scores():
    """Key 300 scores ~20 (base 2) above the first tile's keys for every
    query of KV group 0 (each query has a component along r, the key is 28 r):
    with the 64-query kernel's reference max fixed at the first tile, that
    weight would leave f16 range, so the workgroups start over against the
    exact row max.  Output on the oracle (rows past 300 are dominated by
    v[300]), every row finite."""
    announce("prefill late large scores n=700")
    n = 700
    rng = np.random.default_rng(12)
    r = rng.standard_normal(D)
    r /= np.linalg.norm(r)
    q = rng.standard_normal((n, H, D)).astype(np.float32)
    q[:, :8, :] += 8.0 * r
    q = q.astype(np.float16)
    k = f16(rng, n, G * D)
    k[300, :D] = (28.0 * r).astype(np.float16)
    v = f16(rng, n, G * D)
    c = Cache(num_layers=1, capacity=n)
    out = host(attn_prefill(c, 0, dev(q), dev(k), dev(v), 0))
    assert np.all(np.isfinite(out))
    for i in [0, 299, 300, 301, 383, 384, 450, 511, 512, 640, 699]:
        assert_close(out[i], O.decode(q[i].ravel(), k, v, i + 1), f"late large scores row {i}")


@pytest.mark.parametrize("past,n", [(4096, 17), (5000, 100), (8192, 1024), (20000, 5),
                                    (9000, 33)])
def test_prefill_split_k_form(past, n, monkeypatch):
    """Up to 1024 new tokens after a past of 4096 rows or more run the
    split-K form (the prefill tiles over key chunks, row blocks of 16 tokens,
    then the merge): sampled rows against the oracle, every row against the
    unsplit kernel (MI_ATTN_PREFILL_SPLIT=0)."""
    import torch
    from moe_infer_amd import kv_cache_append
    announce(f"prefill split-K past={past} n={n}")
    rng = np.random.default_rng(past + 3 * n)
    gen = torch.Generator(device="cuda").manual_seed(past + 11 * n)
    c = Cache(num_layers=1, capacity=past + n)
    kp = torch.randn(past, G * D, generator=gen, device="cuda").half()
    vp = torch.randn(past, G * D, generator=gen, device="cuda").half()
    kv_cache_append(c, 0, kp, vp, 0)
    c.set_pos(past)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    out = host(attn_prefill(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g)))
    kall, vall = c.download(0, rows=past + n)
    for i in sorted({0, 1, 15, 16, n // 2, n - 1}):
        if i < n:
            ref = O.decode(q[i].ravel(), kall, vall, past + i + 1, gate=g[i].ravel())
            assert_close(out[i], ref, f"split-K prefill past={past} n={n} row {i}")
    monkeypatch.setenv("MI_ATTN_PREFILL_SPLIT", "0")
    c.set_pos(past)
    whole = host(attn_prefill(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g)))
    assert_close(out, whole, f"split-K vs unsplit past={past} n={n}", atol=1e-3)


def test_prefill_split_k_restart():
    """Scores of odd 64-key tiles far above even ones for some rows: chunks
    whose first tile is even take the restart path in the split-K form."""
    announce("prefill split-K restart")
    rng = np.random.default_rng(77)
    past, n = 12000, 40
    L = past + n
    q = f16(rng, n, H, D)
    qdir = q[0].astype(np.float32).reshape(G, 8, D)[:, 0]
    qdir /= np.linalg.norm(qdir, axis=-1, keepdims=True)
    ramp = ((np.arange(L) // 64) % 2).astype(np.float32)[:, None, None] * 21.0
    kall = (0.3 * rng.standard_normal((L, G, D)).astype(np.float32) + ramp * qdir[None])
    kall = kall.astype(np.float16).reshape(L, G * D)
    vall = f16(rng, L, G * D)
    c = Cache(num_layers=1, capacity=L)
    c.upload(0, kall[:past], vall[:past])
    c.set_pos(past)
    out = attn_prefill(c, 0, dev(q), dev(kall[past:]), dev(vall[past:]), past)
    assert_close(out, O.causal(q, kall, vall, past), "split-K prefill restart")
