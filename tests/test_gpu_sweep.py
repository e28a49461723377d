"""Seeded random sweep over shapes the hand-picked cases do not hit: prefill
and verify at random (past, n), decode at random lengths with the cache
grown by appends, ragged batches of random lengths, each against the CPU
oracle (reference math of src/math_util.rs:323-392 and the causal bound of
src/engine/shaders.metal:2656-2769).  Sizes are bounded so that the oracle
finishes in seconds; the seed list is fixed, so a failure names its case."""
import numpy as np
import pytest

from moe_infer_amd import (Cache, attn_decode, attn_decode_ragged, attn_prefill, attn_verify,
                           kv_pack)
from oracle import oracle as O

from .conftest import f16
from .gpu_util import announce, assert_close, dev

pytestmark = pytest.mark.gpu
H, G, D = 16, 2, 256


def _filled(rng, past, capacity):
    kp, vp = f16(rng, past, G * D), f16(rng, past, G * D)
    c = Cache(num_layers=1, capacity=capacity)
    if past:
        c.upload(0, kp, vp)
        c.set_pos(past)
    return c, kp, vp


@pytest.mark.parametrize("seed", range(16))
def test_prefill_random_shapes(seed):
    rng = np.random.default_rng(1000 + seed)
    past = int(rng.integers(0, 1200))
    n = int(rng.integers(17, 260))
    gated = bool(seed % 2)
    announce(f"sweep prefill seed={seed} past={past} n={n} gated={gated}")
    c, kp, vp = _filled(rng, past, past + n)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    out = attn_prefill(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g) if gated else None)
    ref = O.causal(q, np.concatenate([kp, k]), np.concatenate([vp, v]), past,
                   gate=g if gated else None)
    assert_close(out, ref, f"sweep prefill seed={seed}")


@pytest.mark.parametrize("seed", range(8))
def test_verify_random_shapes(seed):
    rng = np.random.default_rng(2000 + seed)
    past = int(rng.integers(0, 9000))
    n = int(rng.integers(1, 17))
    announce(f"sweep verify seed={seed} past={past} n={n}")
    c, kp, vp = _filled(rng, past, past + n)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    out = attn_verify(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g))
    ref = O.causal(q, np.concatenate([kp, k]), np.concatenate([vp, v]), past, gate=g)
    assert_close(out, ref, f"sweep verify seed={seed}")


@pytest.mark.parametrize("seed", range(8))
def test_split_prefill_and_wide_verify_random_shapes(seed):
    """Prefill after a past of 2048 rows or more (at most half of it new)
    takes the split-K form, and verify of more than 4 tokens the wide form:
    both run the prefill tiles over key chunks and merge the partials.
    Random (past, n) with unaligned chunk ends, against the oracle."""
    rng = np.random.default_rng(3000 + seed)
    past = int(rng.integers(2048, 6000))
    n = int(rng.integers(5, 100))
    gated = bool(seed % 2)
    use_verify = seed % 4 >= 2
    announce(f"sweep split-K seed={seed} past={past} n={n} gated={gated} verify={use_verify}")
    c, kp, vp = _filled(rng, past, past + n)
    q, k, v, g = f16(rng, n, H, D), f16(rng, n, G * D), f16(rng, n, G * D), f16(rng, n, H, D)
    call = attn_verify if use_verify else attn_prefill
    out = call(c, 0, dev(q), dev(k), dev(v), past, gate=dev(g) if gated else None)
    ref = O.causal(q, np.concatenate([kp, k]), np.concatenate([vp, v]), past,
                   gate=g if gated else None)
    assert_close(out, ref, f"sweep split-K seed={seed}")


@pytest.mark.parametrize("seed", range(6))
def test_decode_random_lengths_after_appends(seed):
    """The cache is filled by several appends of random sizes (growth on the
    way), then decoded at a random length."""
    rng = np.random.default_rng(3000 + seed)
    from moe_infer_amd import kv_cache_append
    c = Cache(num_layers=1, capacity=64)
    ks, vs, pos = [], [], 0
    for _ in range(int(rng.integers(2, 6))):
        m = int(rng.integers(1, 3000))
        k, v = f16(rng, m, G * D), f16(rng, m, G * D)
        kv_cache_append(c, 0, dev(k), dev(v), pos)
        ks.append(k)
        vs.append(v)
        pos += m
    c.set_pos(pos)
    kall, vall = np.concatenate(ks), np.concatenate(vs)
    L = int(rng.integers(1, pos + 1))
    announce(f"sweep decode seed={seed} rows={pos} L={L}")
    q, g = f16(rng, H * D), f16(rng, H * D)
    out = attn_decode(c, 0, dev(q), L, gate=dev(g))
    assert_close(out, O.decode(q, kall[:L], vall[:L], L, gate=g), f"sweep decode seed={seed}")


@pytest.mark.parametrize("seed", range(4))
def test_ragged_random_batches(seed):
    rng = np.random.default_rng(4000 + seed)
    b = int(rng.integers(1, 300))
    lengths = rng.integers(0, 700, size=b).astype(np.int32)
    announce(f"sweep ragged seed={seed} batch={b}")
    offsets, rows = [], 0
    for n in lengths:
        offsets.append(rows)
        rows += (int(n) + 31) // 32 * 32
    offsets = np.array(offsets, np.int32)
    k, v = f16(rng, max(rows, 32), G * D), f16(rng, max(rows, 32), G * D)
    q, g = f16(rng, b, H, D), f16(rng, b, H, D)
    kb, vb = kv_pack(dev(k), dev(v), G)
    import torch
    out = attn_decode_ragged(kb, vb, torch.from_numpy(offsets).cuda(),
                             torch.from_numpy(lengths).cuda(), dev(q), max(int(lengths.max()), 1),
                             gate=dev(g))
    assert_close(out, O.decode_ragged(q, k, v, offsets, lengths, gate=g),
                 f"sweep ragged seed={seed}")
