"""Tensor-level entry points of the gfx950 attention library.

Each function validates shapes, dtypes and devices on the host, then calls
the C ABI (include/mi_attn.h) on the current HIP stream.  Tensors are torch
f16 CUDA tensors, contiguous.  H query heads, G KV heads, D = 256.

Reference operators these stand for (fbundle/moe_infer):
  attn_decode   attention_scores/softmax/values_batched + sigmoid_gate_inplace
                (src/math_util.rs:264-269, 323-383); Metal attn_sdpa_block +
                attn_sdpa_reduce (src/engine/shaders.metal:1559-1776)
  attn_step     the engine's append-then-attend step
                (src/engine/qwen35_moe/cpu.rs:136-167, fused_exp2.rs:669-733)
  attn_prefill  kv_cache_append_n + attn_sdpa_causal_n + sigmoid_gate
                (src/engine/qwen35_moe/batched.rs:233-260)
  attn_verify   attn_sdpa_causal_n with past_pos = ctx and n = K drafts
  attn_decode_ragged  (no reference counterpart) independent sequences
  attn_step_proj  the whole step from projections: norm + RoPE + append +
                attend + gate (src/engine/qwen35_moe/fused_exp2.rs:630-733)
  matvec_bf16 / matvec_q4  o_proj of the gated output: matvec_bf16
                (shaders.metal:2392-2425), dequant_matvec_4bit (math_util.rs:14-57)
  qk_norm_rope_append  q_head_norm_rope + k_head_norm_rope + kv_cache_append
                (src/math_util.rs:387-392, 501-593; shaders.metal:2244-2363)
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib

HEAD_DIM = 256
KV_KBLOCK = 32
KV_VBLOCK = 8


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> C.c_void_p | None:
    return None if t is None else C.c_void_p(t.data_ptr())


def _check_tensor(name: str, t: torch.Tensor, numel: int, dtype=torch.float16) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() != numel:
        raise ValueError(f"{name} has {t.numel()} elements, expected {numel}")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


def _check_qgo(cache, q, gate, out, n):
    H, D = cache.num_q_heads, cache.head_dim
    _check_tensor("q", q, n * H * D)
    if gate is not None:
        _check_tensor("gate", gate, n * H * D)
    if out is None:
        out = torch.empty_like(q)
    _check_tensor("out", out, n * H * D)
    return out


def _check_kv_rows(cache, k, v, n):
    G, D = cache.num_kv_heads, cache.head_dim
    _check_tensor("k", k, n * G * D)
    _check_tensor("v", v, n * G * D)


def kv_cache_append(cache, layer: int, k: torch.Tensor, v: torch.Tensor, pos: int) -> None:
    """Writes n rows k, v ([n, G*D]) at rows [pos, pos+n) of `layer`;
    len(layer) = pos + n."""
    n = k.numel() // (cache.num_kv_heads * cache.head_dim)
    _check_kv_rows(cache, k, v, n)
    _lib.check(_lib.lib().mi_kv_append(cache._h, cache.slot(layer), _ptr(k), _ptr(v),
                                       int(pos), n, _stream()))


def qk_norm_rope_append(cache, layer: int, q_proj: torch.Tensor, k: torch.Tensor,
                        v: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                        pos: int, rotary_dim: int = 64, rope_theta: float = 1e7,
                        eps: float = 1e-6, q_out=None, gate_out=None):
    """Per-head RMS norm + NeoX partial RoPE of n tokens at positions
    pos .. pos+n-1, fused with the cache append of the rotated K and raw V.

    q_proj: [n, H, 2D] f32 (query then gate per head); k, v: [n, G, D] f32;
    q_norm_w, k_norm_w: [D] bf16.  Returns (q, gate), each [n, H, D] f16.
    len(layer) becomes pos + n."""
    H, G, D = cache.num_q_heads, cache.num_kv_heads, cache.head_dim
    n = q_proj.numel() // (H * 2 * D)
    if n <= 0:
        raise ValueError("q_proj holds no token")
    _check_tensor("q_proj", q_proj, n * H * 2 * D, torch.float32)
    _check_tensor("k", k, n * G * D, torch.float32)
    _check_tensor("v", v, n * G * D, torch.float32)
    _check_tensor("q_norm_w", q_norm_w, D, torch.bfloat16)
    _check_tensor("k_norm_w", k_norm_w, D, torch.bfloat16)
    if q_out is None:
        q_out = torch.empty((n, H, D), dtype=torch.float16, device=q_proj.device)
    if gate_out is None:
        gate_out = torch.empty((n, H, D), dtype=torch.float16, device=q_proj.device)
    _check_tensor("q_out", q_out, n * H * D)
    _check_tensor("gate_out", gate_out, n * H * D)
    _lib.check(_lib.lib().mi_qk_norm_rope_append(
        cache._h, cache.slot(layer), _ptr(q_proj), _ptr(k), _ptr(v), _ptr(q_norm_w),
        _ptr(k_norm_w), int(rotary_dim), float(rope_theta), float(eps), int(pos), n,
        _ptr(q_out), _ptr(gate_out), _stream()))
    return q_out, gate_out


def attn_step_proj(cache, layer: int, q_proj: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, pos: int,
                   rotary_dim: int = 64, rope_theta: float = 1e7, eps: float = 1e-6,
                   out=None) -> torch.Tensor:
    """One token's full-attention step from its f32 projections (q_proj
    [H, 2D], k, v [G, D]) and bf16 norm weights: norm + RoPE at `pos`,
    append at `pos`, decode over pos + 1 rows, sigmoid gate.  Returns
    [H, D] f16; len(layer) becomes pos + 1."""
    H, G, D = cache.num_q_heads, cache.num_kv_heads, cache.head_dim
    _check_tensor("q_proj", q_proj, H * 2 * D, torch.float32)
    _check_tensor("k", k, G * D, torch.float32)
    _check_tensor("v", v, G * D, torch.float32)
    _check_tensor("q_norm_w", q_norm_w, D, torch.bfloat16)
    _check_tensor("k_norm_w", k_norm_w, D, torch.bfloat16)
    if out is None:
        out = torch.empty((H, D), dtype=torch.float16, device=q_proj.device)
    _check_tensor("out", out, H * D)
    _lib.check(_lib.lib().mi_attn_step_proj(
        cache._h, cache.slot(layer), _ptr(q_proj), _ptr(k), _ptr(v), _ptr(q_norm_w),
        _ptr(k_norm_w), int(rotary_dim), float(rope_theta), float(eps), _ptr(out), int(pos),
        _stream()))
    return out


def attn_decode(cache, layer: int, q: torch.Tensor, seq_len: int,
                gate: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """One query token ([H, D] or [H*D]) over rows [0, seq_len) of `layer`."""
    out = _check_qgo(cache, q, gate, out, 1)
    _lib.check(_lib.lib().mi_attn_decode(cache._h, cache.slot(layer), _ptr(q), _ptr(gate),
                                         _ptr(out), int(seq_len), _stream()))
    return out


def attn_step(cache, layer: int, q, k, v, pos: int, gate=None, out=None) -> torch.Tensor:
    """Append k, v at `pos`, then decode with seq_len = pos + 1."""
    out = _check_qgo(cache, q, gate, out, 1)
    _check_kv_rows(cache, k, v, 1)
    _lib.check(_lib.lib().mi_attn_step(cache._h, cache.slot(layer), _ptr(q), _ptr(k), _ptr(v),
                                       _ptr(gate), _ptr(out), int(pos), _stream()))
    return out


def attn_prefill(cache, layer: int, q, k, v, past_pos: int, gate=None, out=None) -> torch.Tensor:
    """Causal batched prefill of n = q.shape[0] tokens ([n, H, D]).  With
    k = v = None the rows [past_pos, past_pos + n) are already in the cache
    (e.g. from qk_norm_rope_append) and are not appended again."""
    n = q.numel() // (cache.num_q_heads * cache.head_dim)
    out = _check_qgo(cache, q, gate, out, n)
    if k is not None or v is not None:  # None, None: rows already in the cache
        _check_kv_rows(cache, k, v, n)
    _lib.check(_lib.lib().mi_attn_prefill(cache._h, cache.slot(layer), _ptr(q), _ptr(k),
                                          _ptr(v), _ptr(gate), _ptr(out), int(past_pos), n,
                                          _stream()))
    return out


def attn_verify(cache, layer: int, q, k, v, past_pos: int, gate=None, out=None) -> torch.Tensor:
    """K-token speculative verify: same contract as attn_prefill, split-K
    kernel (HBM-bound) for small K."""
    n = q.numel() // (cache.num_q_heads * cache.head_dim)
    out = _check_qgo(cache, q, gate, out, n)
    if k is not None or v is not None:  # None, None: rows already in the cache
        _check_kv_rows(cache, k, v, n)
    _lib.check(_lib.lib().mi_attn_verify(cache._h, cache.slot(layer), _ptr(q), _ptr(k),
                                         _ptr(v), _ptr(gate), _ptr(out), int(past_pos), n,
                                         _stream()))
    return out


def kv_pack(k_rows: torch.Tensor, v_rows: torch.Tensor, num_kv_heads: int,
            out: tuple[torch.Tensor, torch.Tensor] | None = None, row0: int = 0):
    """Token-major K, V rows [n, G*D] -> (k_blocks, v_blocks) in the device
    cache layout (32-row K blocks, 8-row transposed V blocks), written at rows
    [row0, row0+n) of `out` (allocated zeroed, whole blocks, when None)."""
    G, D = num_kv_heads, HEAD_DIM
    n = k_rows.numel() // (G * D)
    _check_tensor("k_rows", k_rows, n * G * D)
    _check_tensor("v_rows", v_rows, n * G * D)
    need = (row0 + n + KV_KBLOCK - 1) // KV_KBLOCK * KV_KBLOCK * G * D
    if out is None:
        out = (torch.zeros(need, dtype=torch.float16, device=k_rows.device),
               torch.zeros(need, dtype=torch.float16, device=k_rows.device))
    for t in out:
        if t.numel() < need:
            raise ValueError("output buffers hold fewer whole blocks than the rows need")
    _lib.check(_lib.lib().mi_kv_pack(_ptr(k_rows), _ptr(v_rows), _ptr(out[0]), _ptr(out[1]),
                                     int(row0), n, G, D, _stream()))
    return out


def ragged_workspace(batch: int, max_len: int, num_q_heads: int = 16, num_kv_heads: int = 2,
                     device="cuda") -> torch.Tensor:
    nbytes = _lib.lib().mi_attn_ragged_workspace_size(batch, max_len, num_q_heads,
                                                      num_kv_heads, HEAD_DIM)
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def attn_decode_ragged(k_blocks: torch.Tensor, v_blocks: torch.Tensor, offsets: torch.Tensor,
                       lengths: torch.Tensor, q: torch.Tensor, max_len: int,
                       num_kv_heads: int = 2, gate=None, out=None,
                       workspace: torch.Tensor | None = None,
                       validate: bool = True) -> torch.Tensor:
    """Ragged batch: sequence s uses rows [offsets[s], offsets[s]+lengths[s])
    of k_blocks / v_blocks (the device cache layout, see kv_pack).
    q: [batch, H, D].  offsets must be multiples of 32."""
    batch = offsets.numel()
    G, D = num_kv_heads, HEAD_DIM
    H = q.numel() // (batch * D)
    for name, t in (("offsets", offsets), ("lengths", lengths)):
        _check_tensor(name, t, batch, dtype=torch.int32)
    _check_tensor("q", q, batch * H * D)
    if gate is not None:
        _check_tensor("gate", gate, batch * H * D)
    if out is None:
        out = torch.empty_like(q)
    _check_tensor("out", out, batch * H * D)
    rows = k_blocks.numel() // (G * D)
    _check_tensor("k_blocks", k_blocks, rows * G * D)
    if rows % KV_KBLOCK or v_blocks.numel() != k_blocks.numel():
        raise ValueError("k_blocks / v_blocks must hold the same whole 32-row blocks")
    _check_tensor("v_blocks", v_blocks, rows * G * D)
    if validate:  # host copy of the table (synchronises): bounds the kernel's reads
        off = offsets.cpu().tolist()
        ln = lengths.cpu().tolist()
        for s_, (o, n_) in enumerate(zip(off, ln)):
            if o < 0 or o % KV_KBLOCK or n_ < 0 or n_ > max_len or o + n_ > rows:
                raise ValueError(f"sequence {s_}: offset {o}, length {n_} invalid for "
                                 f"{rows} rows, max_len {max_len}")
    if workspace is None:
        workspace = ragged_workspace(batch, max_len, H, G, q.device)
    _lib.check(_lib.lib().mi_attn_decode_ragged(
        _ptr(k_blocks), _ptr(v_blocks), _ptr(offsets), _ptr(lengths), batch, int(max_len), H, G,
        D, _ptr(q), _ptr(gate), _ptr(out), _ptr(workspace), workspace.numel(), _stream()))
    return out


def matvec_bf16(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """o_proj: out[r] = sum_c w[r, c] * x[c]; x f16 [in], w bf16 [out, in];
    returns f32 [out]."""
    if w.dim() != 2:
        raise ValueError("w must be [out_dim, in_dim]")
    out_dim, in_dim = w.shape
    _check_tensor("x", x, in_dim)
    _check_tensor("w", w, out_dim * in_dim, torch.bfloat16)
    if out is None:
        out = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    _check_tensor("out", out, out_dim, torch.float32)
    _lib.check(_lib.lib().mi_matvec_bf16(_ptr(x), _ptr(w), _ptr(out), out_dim, in_dim,
                                         _stream()))
    return out


def matvec_q4(x: torch.Tensor, w_packed: torch.Tensor, scales: torch.Tensor,
              biases: torch.Tensor, group_size: int = 64,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """o_proj with 4-bit affine weights: w_packed int32/uint32 [out, in/8]
    (8 nibbles per word, low nibble first), scales / biases bf16
    [out, in/group_size]; x f16 [in]; returns f32 [out]."""
    if w_packed.dim() != 2:
        raise ValueError("w_packed must be [out_dim, in_dim / 8]")
    out_dim, in_dim = w_packed.shape[0], w_packed.shape[1] * 8
    _check_tensor("x", x, in_dim)
    _check_tensor("w_packed", w_packed, out_dim * in_dim // 8, w_packed.dtype)
    if w_packed.dtype not in (torch.int32, torch.uint32):
        raise TypeError("w_packed must be int32 or uint32")
    ng = in_dim // group_size
    _check_tensor("scales", scales, out_dim * ng, torch.bfloat16)
    _check_tensor("biases", biases, out_dim * ng, torch.bfloat16)
    if out is None:
        out = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    _check_tensor("out", out, out_dim, torch.float32)
    _lib.check(_lib.lib().mi_matvec_q4(_ptr(x), _ptr(w_packed), _ptr(scales), _ptr(biases),
                                       int(group_size), _ptr(out), out_dim, in_dim, _stream()))
    return out
