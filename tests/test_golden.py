"""Committed seeded fixtures (tests/golden/attn_cases.npz, written by
tests/golden/make_golden.py): the oracle must keep reproducing them, and the
GPU kernels must match them within the north-star tolerance."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

FIX = np.load(Path(__file__).resolve().parent / "golden" / "attn_cases.npz")
H, G, D = 16, 2, 256
DECODE = sorted({k.split("_")[1][1:] for k in FIX.files if k.startswith("decode_")}, key=int)
CAUSAL = sorted({k[:k.index("_n") + 3].split("_", 1)[1] for k in FIX.files
                 if k.startswith("causal_")})


def case(prefix):
    return {k[len(prefix):]: FIX[k] for k in FIX.files if k.startswith(prefix)}


@pytest.mark.parametrize("L", DECODE)
def test_oracle_reproduces_decode_fixture(L):
    c = case(f"decode_L{L}_")
    n = int(L)
    np.testing.assert_allclose(O.decode(c["q"], c["k"], c["v"], n, gate=c["gate"]), c["out_f32"],
                               rtol=0, atol=1e-6)
    np.testing.assert_allclose(O.decode_f64(c["q"], c["k"], c["v"], n, gate=c["gate"]),
                               c["out_f64"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", CAUSAL)
def test_oracle_reproduces_causal_fixture(name):
    c = case(f"causal_{name}_")
    past = int(name.split("_")[0][1:])
    np.testing.assert_allclose(O.causal(c["q"], c["k"], c["v"], past, gate=c["gate"]),
                               c["out_f64"], rtol=0, atol=2e-5)


def test_oracle_reproduces_ragged_fixture():
    c = case("ragged_")
    np.testing.assert_allclose(
        O.decode_ragged(c["q"], c["k"], c["v"], c["offsets"], c["lengths"]), c["out_f32"],
        rtol=0, atol=1e-6)


@pytest.mark.gpu
def test_gpu_kernels_match_fixtures():
    import torch

    from moe_infer_amd import Cache, attn_decode, attn_decode_ragged, attn_prefill, kv_pack

    from .gpu_util import assert_close, dev
    for L in DECODE:
        c = case(f"decode_L{L}_")
        n = int(L)
        cache = Cache(num_layers=1, capacity=n)
        cache.upload(0, c["k"], c["v"])
        out = attn_decode(cache, 0, dev(c["q"]), n, gate=dev(c["gate"]))
        assert_close(out, c["out_f64"], f"fixture decode L={L}")
    for name in CAUSAL:
        c = case(f"causal_{name}_")
        past = int(name.split("_")[0][1:])
        n = c["q"].shape[0]
        cache = Cache(num_layers=1, capacity=past + n)
        if past:
            cache.upload(0, c["k"][:past], c["v"][:past])
        out = attn_prefill(cache, 0, dev(c["q"]), dev(c["k"][past:]), dev(c["v"][past:]), past,
                           gate=dev(c["gate"]))
        assert_close(out, c["out_f64"], f"fixture causal {name}")
    c = case("ragged_")
    kb, vb = kv_pack(dev(c["k"]), dev(c["v"]), G)
    out = attn_decode_ragged(kb, vb,
                             torch.from_numpy(c["offsets"]).cuda(),
                             torch.from_numpy(c["lengths"]).cuda(), dev(c["q"]),
                             int(c["lengths"].max()))
    assert_close(out, c["out_f32"], "fixture ragged")
