"""Helpers of the GPU parity tests: device tensors from numpy f16 arrays and
the tolerance of the north-star contract (f32 accumulation; on f16 outputs
max-abs error <= 2e-3 and relative error <= 1e-2, where relative error is
max|gpu - ref| / max|ref|)."""
import sys

import numpy as np
import torch

ATOL = 2e-3
RTOL = 1e-2


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16)).to("cuda")


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def assert_close(gpu, ref, what="", atol=ATOL, rtol=RTOL):
    g = host(gpu).astype(np.float64) if isinstance(gpu, torch.Tensor) else np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64).reshape(g.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite GPU output"
    err = np.abs(g - r)
    max_abs = float(err.max()) if err.size else 0.0
    scale = float(np.abs(r).max()) if r.size else 0.0
    rel = max_abs / scale if scale > 0 else max_abs
    print(f"[parity] {what}: max_abs={max_abs:.3e} rel={rel:.3e} (|ref|max={scale:.3e})",
          file=sys.stderr, flush=True)
    assert max_abs <= atol, f"{what}: max abs error {max_abs:.3e} > {atol}"
    assert rel <= rtol, f"{what}: relative error {rel:.3e} > {rtol}"


def announce(msg: str) -> None:
    print(f"[case] {msg}", file=sys.stderr, flush=True)
