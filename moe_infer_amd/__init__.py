"""MI355X (gfx950) attention path of the Qwen3.6 full-attention layers.

GQA decode over an f16 KV cache, causal batched prefill, K-token speculative
verify and ragged batched decode, as hand-written CDNA4 HIP kernels behind
the C ABI of include/mi_attn.h (libmi_attn.so).  The Python layer mirrors the
reference engine's Cache / Engine API for this path.
"""
from . import _lib
from .attention import (attn_decode, attn_decode_ragged, attn_prefill, attn_step, attn_step_proj,
                        attn_verify, kv_cache_append, kv_pack, matvec_bf16, matvec_q4,
                        qk_norm_rope_append, ragged_workspace)
from .engine import Engine, EngineInterrupted, EngineSnapshot, record_engine_telemetry
from .kv_cache import Cache

__all__ = ["Cache", "Engine", "EngineInterrupted", "EngineSnapshot", "record_engine_telemetry", "attn_decode",
           "attn_decode_ragged", "attn_prefill", "attn_step", "attn_step_proj", "attn_verify",
           "kv_cache_append", "kv_pack", "matvec_bf16", "matvec_q4", "qk_norm_rope_append",
           "ragged_workspace", "_lib"]
