"""Writes the small seeded fixtures of tests/golden/attn_cases.npz.

The reference ships no attention vectors (its only numeric checks compare
end-to-end logits of a model whose weights are not available), so these are
regression vectors of this build: seeded f16 inputs and the CPU oracle's f64
and f32 outputs for them.  They pin later changes of the oracle and of the
kernels to today's checked behaviour (the oracle itself is pinned by
tests/test_oracle.py).  Run: python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

H, G, D = 16, 2, 256
OUT = Path(__file__).resolve().parent / "attn_cases.npz"


def f16(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def main():
    arrays = {}
    rng = np.random.default_rng(20240601)
    for L in (1, 7, 33):
        q, k, v, g = f16(rng, H * D), f16(rng, L, G * D), f16(rng, L, G * D), f16(rng, H * D)
        p = f"decode_L{L}_"
        arrays.update({p + "q": q, p + "k": k, p + "v": v, p + "gate": g,
                       p + "out_f64": O.decode_f64(q, k, v, L, gate=g).astype(np.float32),
                       p + "out_f32": O.decode(q, k, v, L, gate=g)})
    for past, n in ((0, 2), (5, 2), (21, 3)):
        q, k, v, g = (f16(rng, n, H, D), f16(rng, past + n, G * D), f16(rng, past + n, G * D),
                      f16(rng, n, H, D))
        p = f"causal_p{past}_n{n}_"
        arrays.update({p + "q": q, p + "k": k, p + "v": v, p + "gate": g,
                       p + "out_f64": O.causal_f64(q, k, v, past, gate=g).astype(np.float32)})
    lengths = np.array([5, 0, 17], np.int32)
    offsets = np.array([0, 32, 32], np.int32)
    q, k, v = f16(rng, 3, H, D), f16(rng, 64, G * D), f16(rng, 64, G * D)
    arrays.update({"ragged_q": q, "ragged_k": k, "ragged_v": v, "ragged_offsets": offsets,
                   "ragged_lengths": lengths,
                   "ragged_out_f32": O.decode_ragged(q, k, v, offsets, lengths)})
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
