"""ctypes front end of the CPU oracle (attn_oracle.c) plus a host model of
the reference's KV-cache semantics.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product (moe_infer_amd)
never imports it.

Arrays in and out are numpy; f16 inputs are np.float16 arrays (passed to C
as their bit patterns).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_attn.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        P, I64 = C.c_void_p, C.c_int64
        sigs = {
            "oracle_build_info": (C.c_char_p, []),
            "oracle_f16_to_f32": (C.c_float, [C.c_uint16]),
            "oracle_f32_to_f16": (C.c_uint16, [C.c_float]),
            "oracle_widen_f16": (None, [P, P, I64]),
            "oracle_narrow_f32": (None, [P, P, I64]),
            "oracle_attention_scores_batched": (None, [P, P, P, I64, I64, I64, I64, I64, I64]),
            "oracle_attention_softmax_batched": (None, [P, I64, I64, I64]),
            "oracle_attention_values_batched": (None, [P, P, P, I64, I64, I64, I64, I64, I64]),
            "oracle_kv_cache_append": (None, [P, P, P, P, I64, I64]),
            "oracle_sigmoid_gate_inplace": (None, [P, P, I64]),
            "oracle_decode_heads_omp": (None, [P, P, P, P, P, P, I64, I64, I64, I64, I64, I64,
                                               C.c_int]),
            "oracle_mtp_cpu_attention": (None, [P, P, P, P, I64, I64, I64, I64, C.c_float]),
            "oracle_attn_decode_f32": (None, [P, P, P, P, I64, I64, I64, I64, P]),
            "oracle_attn_decode_f16": (None, [P, P, P, P, I64, I64, I64, I64, P]),
            "oracle_attn_causal_n_f16": (None, [P, P, P, P, I64, I64, I64, I64, I64, P]),
            "oracle_attn_decode_ragged_f16": (None, [P, P, P, P, P, P, I64, I64, I64, I64, P]),
            "oracle_attn_decode_f64": (None, [P, P, P, P, I64, I64, I64, I64, P]),
            "oracle_attn_causal_n_f64": (None, [P, P, P, P, I64, I64, I64, I64, I64, P]),
            "oracle_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "oracle_rope_inv_freq": (None, [C.c_float, I64, P]),
            "oracle_q_head_norm_rope": (None, [P, P, P, P, I64, I64, I64, C.c_float, I64,
                                               C.c_float]),
            "oracle_k_head_norm_rope": (None, [P, P, I64, I64, I64, C.c_float, I64, C.c_float]),
            "oracle_matvec_bf16": (None, [P, P, P, I64, I64]),
            "oracle_dequant_matvec_4bit": (None, [P, P, P, P, P, I64, I64, I64]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def build_flags() -> str:
    """Compiler and flags of the built oracle library."""
    return lib().oracle_build_info().decode()


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _h(a):
    """Contiguous float16 array (or None)."""
    return None if a is None else np.ascontiguousarray(a, dtype=np.float16)


def _f(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# ----------------------------------------------------------- conversions --

def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oracle_widen_f16(_p(bits), _p(out), bits.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even narrowing; returns uint16 bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_narrow_f32(_p(x), _p(out), x.size)
    return out


# ------------------------------------------------ reference f32 functions --

def attention_scores_batched(q, k_cache, H, G, D, seq_len, max_seq):
    q, k_cache = _f(q), _f(k_cache)
    scores = np.zeros(H * max_seq, dtype=np.float32)
    lib().oracle_attention_scores_batched(_p(q), _p(k_cache), _p(scores), H, G, D, G * D,
                                          seq_len, max_seq)
    return scores


def attention_softmax_batched(scores, H, seq_len, max_seq):
    s = np.array(scores, dtype=np.float32, copy=True)
    lib().oracle_attention_softmax_batched(_p(s), H, seq_len, max_seq)
    return s


def attention_values_batched(scores, v_cache, H, G, D, seq_len, max_seq):
    scores, v_cache = _f(scores), _f(v_cache)
    out = np.empty(H * D, dtype=np.float32)
    lib().oracle_attention_values_batched(_p(scores), _p(v_cache), _p(out), H, G, D, G * D,
                                          seq_len, max_seq)
    return out


def kv_cache_append(k, v, k_cache, v_cache, pos, kv_dim):
    k, v = _f(k), _f(v)
    assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
    lib().oracle_kv_cache_append(_p(k), _p(v), _p(k_cache), _p(v_cache), pos, kv_dim)


def sigmoid_gate(out, gate):
    o = np.array(out, dtype=np.float32, copy=True)
    g = _f(gate)
    lib().oracle_sigmoid_gate_inplace(_p(o), _p(g), o.size)
    return o


def mtp_cpu_attention(q, k_cache, v_cache, H, G, D, seq_len, kq_scale):
    q, k_cache, v_cache = _f(q), _f(k_cache), _f(v_cache)
    out = np.empty(H * D, dtype=np.float32)
    lib().oracle_mtp_cpu_attention(_p(q), _p(k_cache), _p(v_cache), _p(out), H, G, D, seq_len,
                                   kq_scale)
    return out


def decode_f32_from_f32(q, gate, k_rows, v_rows, H, G, D, seq_len):
    q, gate, k_rows, v_rows = _f(q), _f(gate), _f(k_rows), _f(v_rows)
    out = np.empty(H * D, dtype=np.float32)
    lib().oracle_attn_decode_f32(_p(q), _p(gate), _p(k_rows), _p(v_rows), H, G, D, seq_len,
                                 _p(out))
    return out


# ------------------------------------------------ composed, f16 inputs --

def decode(q, k_rows, v_rows, seq_len, gate=None, H=16, G=2, D=256):
    """Reference f32 decode of one token over the first seq_len rows."""
    q, gate, k_rows, v_rows = _h(q), _h(gate), _h(k_rows), _h(v_rows)
    assert k_rows.size >= seq_len * G * D and v_rows.size >= seq_len * G * D
    out = np.empty(H * D, dtype=np.float32)
    lib().oracle_attn_decode_f16(_p(q), _p(gate), _p(k_rows), _p(v_rows), H, G, D, seq_len,
                                 _p(out))
    return out.reshape(H, D)


def decode_f64(q, k_rows, v_rows, seq_len, gate=None, H=16, G=2, D=256):
    q, gate, k_rows, v_rows = _h(q), _h(gate), _h(k_rows), _h(v_rows)
    out = np.empty(H * D, dtype=np.float64)
    lib().oracle_attn_decode_f64(_p(q), _p(gate), _p(k_rows), _p(v_rows), H, G, D, seq_len,
                                 _p(out))
    return out.reshape(H, D)


def causal(q, k_rows, v_rows, past, gate=None, H=16, G=2, D=256):
    """attn_sdpa_causal_n semantics: q [n,H,D]; rows [past+n, G*D]."""
    q, gate, k_rows, v_rows = _h(q), _h(gate), _h(k_rows), _h(v_rows)
    n = q.size // (H * D)
    assert k_rows.size >= (past + n) * G * D
    out = np.empty(n * H * D, dtype=np.float32)
    lib().oracle_attn_causal_n_f16(_p(q), _p(gate), _p(k_rows), _p(v_rows), H, G, D, past, n,
                                   _p(out))
    return out.reshape(n, H, D)


def causal_f64(q, k_rows, v_rows, past, gate=None, H=16, G=2, D=256):
    q, gate, k_rows, v_rows = _h(q), _h(gate), _h(k_rows), _h(v_rows)
    n = q.size // (H * D)
    out = np.empty(n * H * D, dtype=np.float64)
    lib().oracle_attn_causal_n_f64(_p(q), _p(gate), _p(k_rows), _p(v_rows), H, G, D, past, n,
                                   _p(out))
    return out.reshape(n, H, D)


def decode_ragged(q, k_rows, v_rows, offsets, lengths, gate=None, H=16, G=2, D=256):
    q, gate, k_rows, v_rows = _h(q), _h(gate), _h(k_rows), _h(v_rows)
    offsets = np.ascontiguousarray(offsets, dtype=np.int32)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    b = offsets.size
    out = np.empty(b * H * D, dtype=np.float32)
    lib().oracle_attn_decode_ragged_f16(_p(q), _p(gate), _p(k_rows), _p(v_rows), _p(offsets),
                                        _p(lengths), b, H, G, D, _p(out))
    return out.reshape(b, H, D)


# ------------------------------------------------ Q/K head norm + RoPE --

def rope_inv_freq(rope_theta=1e7, rotary_dim=64):
    out = np.empty(rotary_dim // 2, dtype=np.float32)
    lib().oracle_rope_inv_freq(rope_theta, rotary_dim, _p(out))
    return out


def q_head_norm_rope(q_proj, q_norm_w, pos, H=16, D=256, rotary_dim=64, rope_theta=1e7,
                     eps=1e-6):
    """q_proj [H, 2D] (f32 values; f16 inputs are widened exactly), q_norm_w
    bf16 bit patterns uint16[D] -> (q_out [H, D], gate [H, D]) f32."""
    qp = _f(q_proj)
    w = np.ascontiguousarray(q_norm_w, dtype=np.uint16)
    q = np.empty(H * D, np.float32)
    g = np.empty(H * D, np.float32)
    lib().oracle_q_head_norm_rope(_p(qp), _p(w), _p(q), _p(g), H, D, rotary_dim, rope_theta,
                                  pos, eps)
    return q.reshape(H, D), g.reshape(H, D)


def k_head_norm_rope(k, k_norm_w, pos, G=2, D=256, rotary_dim=64, rope_theta=1e7, eps=1e-6):
    kb = np.array(k, dtype=np.float32, copy=True).reshape(-1)
    w = np.ascontiguousarray(k_norm_w, dtype=np.uint16)
    lib().oracle_k_head_norm_rope(_p(kb), _p(w), G, D, rotary_dim, rope_theta, pos, eps)
    return kb.reshape(G, D)


# ------------------------------------------------------ o_proj matvec --

def matvec_bf16(w_bits, x):
    """w_bits: uint16 bf16 patterns [out, in]; x float [in] -> f32 [out]."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    xx = _f(x)
    out = np.empty(w.shape[0], np.float32)
    lib().oracle_matvec_bf16(_p(w), _p(xx), _p(out), w.shape[0], w.shape[1])
    return out


def dequant_matvec_4bit(w_packed, scales, biases, x, group_size=64):
    """w_packed uint32 [out, in/8]; scales, biases bf16 bits [out, in/gs]."""
    wp = np.ascontiguousarray(w_packed, dtype=np.uint32)
    sc = np.ascontiguousarray(scales, dtype=np.uint16)
    bi = np.ascontiguousarray(biases, dtype=np.uint16)
    xx = _f(x)
    out_dim, in_dim = wp.shape[0], wp.shape[1] * 8
    out = np.empty(out_dim, np.float32)
    lib().oracle_dequant_matvec_4bit(_p(wp), _p(sc), _p(bi), _p(xx), _p(out), out_dim, in_dim,
                                     group_size)
    return out


# ------------------------------------------------------ cache semantics --

class CacheModel:
    """Host model of the reference cache state (src/cache.rs:84-128,
    src/engine/qwen35_moe/cpu.rs:141-144, mtp.rs:39-47): token-major rows
    per layer, `len` per layer and `pos`.  append overwrites rows and sets
    len = pos + n; set_pos changes pos and every len and no row; reset is
    set_pos(0); copy_from copies rows, len and pos."""

    def __init__(self, layers: int, kv_dim: int, capacity: int):
        self.k = [np.zeros((capacity, kv_dim), np.float16) for _ in range(layers)]
        self.v = [np.zeros((capacity, kv_dim), np.float16) for _ in range(layers)]
        self.len = [0] * layers
        self.pos = 0

    def _grow(self, rows):
        cap = self.k[0].shape[0]
        if rows <= cap:
            return
        while cap < rows:
            cap *= 2
        for arrs in (self.k, self.v):
            for i, a in enumerate(arrs):
                b = np.zeros((cap, a.shape[1]), np.float16)
                b[:a.shape[0]] = a
                arrs[i] = b

    def append(self, layer, k, v, pos):
        k = np.asarray(k, np.float16).reshape(-1, self.k[0].shape[1])
        v = np.asarray(v, np.float16).reshape(-1, self.k[0].shape[1])
        self._grow(pos + k.shape[0])
        self.k[layer][pos:pos + k.shape[0]] = k
        self.v[layer][pos:pos + k.shape[0]] = v
        self.len[layer] = pos + k.shape[0]

    def set_pos(self, pos):
        self.pos = pos
        self.len = [pos] * len(self.len)

    def reset(self):
        self.set_pos(0)

    def copy_from(self, other: "CacheModel"):
        self.k = [a.copy() for a in other.k]
        self.v = [a.copy() for a in other.v]
        self.len = list(other.len)
        self.pos = other.pos


# ------------------------------------------------ CPU baseline (bench.py) --

class DecodeBaseline:
    """The reference CPU engine's attention core for one decode step, as
    cpu.rs:146-167 runs it: scores -> softmax -> values -> sigmoid gate over
    an f32 cache, with the scores buffer allocated once at the cache's
    max_seq (the engine's scratch, cpu.rs:149-163).  The f16 inputs are
    widened to f32 once, here, so that run() times only the reference's f32
    loops (src/math_util.rs:264-269, 323-383)."""

    def __init__(self, q, k_rows, v_rows, gate, H=16, G=2, D=256):
        self.H, self.G, self.D = H, G, D
        self.q = f16_to_f32(_h(q).view(np.uint16))
        self.gate = f16_to_f32(_h(gate).view(np.uint16))
        self.k = f16_to_f32(_h(k_rows).view(np.uint16))
        self.v = f16_to_f32(_h(v_rows).view(np.uint16))
        self.max_seq = self.k.size // (G * D)
        self.scores = np.zeros(H * self.max_seq, dtype=np.float32)
        self.out = np.empty(H * D, dtype=np.float32)
        self._args = [_p(a) for a in (self.q, self.gate, self.k, self.v, self.scores, self.out)]

    def run(self, seq_len: int) -> np.ndarray:
        L = lib()
        q, gate, k, v, scores, out = self._args
        H, G, D = self.H, self.G, self.D
        L.oracle_attention_scores_batched(q, k, scores, H, G, D, G * D, seq_len, self.max_seq)
        L.oracle_attention_softmax_batched(scores, H, seq_len, self.max_seq)
        L.oracle_attention_values_batched(scores, v, out, H, G, D, G * D, seq_len, self.max_seq)
        L.oracle_sigmoid_gate_inplace(out, gate, H * D)
        return self.out.reshape(H, D)

    def run_omp(self, seq_len: int, threads: int) -> np.ndarray:
        """The same step with the query heads spread over `threads` OpenMP
        threads (same per-head loops, same bits)."""
        q, gate, k, v, scores, out = self._args
        H, G, D = self.H, self.G, self.D
        lib().oracle_decode_heads_omp(q, k, v, gate, scores, out, H, G, D, G * D, seq_len,
                                      self.max_seq, threads)
        return self.out.reshape(H, D)
