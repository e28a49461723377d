"""The engine's full-attention step over a device KV cache, with the
reference Engine's method names for the attention / cache subset
(src/python_bindings.rs:104-318, trait Engine in src/engine.rs:32-93).

What the reference's Engine does around attention (embedding, projections,
norms, RoPE, MoE, lm_head) is outside this library; callers hand in the
per-layer q / k / v / gate projections and get the gated attention output.

  forward(layers)            one token through every full-attention layer:
                             append at engine_pos, attend [0, pos], gate;
                             then pos += 1 (fused_exp2.rs:989-1039)
  forward_batched(layers)    n tokens per layer, causal (batched.rs:129-312);
                             pos += n (fused_exp3.rs:291).  n <= VERIFY_MAX_TOKENS
                             runs the split-K verify kernel (HBM-bound, the
                             whole cache in one pass per 4 tokens), larger n
                             the MFMA prefill kernel
  forward_proj(layers) /     the same two steps from the f32 projections:
  forward_batched_proj(...)  per-head Q/K RMS norm + NeoX partial RoPE fused in
                             (cpu.rs:122-145, fused_exp2.rs:630-733)
  mtp_forward(...)           MTP layer: append at mtp_pos, attend, mtp_pos += 1
                             (mtp.rs:143-156, 223)
  mtp_verify(...)            K draft tokens at once (split-K verify kernel)
  mtp_reset / mtp_rollback   MtpState::reset / rollback (mtp.rs:39-47)
  snapshot_state / restore_snapshot   positions only: KV rows past the restored
                             position stay but are never read (fused_exp3.rs:321-365)
  telemetry()                per-call wall times when recording is on
                             (record_engine_telemetry, engine.rs:13-24)
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from . import attention
from .kv_cache import Cache

_RECORD_TELEMETRY = False


def record_engine_telemetry(on: bool) -> None:
    global _RECORD_TELEMETRY
    _RECORD_TELEMETRY = bool(on)


class EngineInterrupted(RuntimeError):
    """Raised when a forward call's check_signal returns True before a layer
    (the reference's MoEError::Metal("interrupted"), surfaced to Python as a
    RuntimeError: fused_exp2.rs:1017-1019, python_bindings.rs:152)."""

    def __init__(self):
        super().__init__("Metal error: interrupted")


def _poll(check_signal) -> None:
    if check_signal is not None and check_signal():
        raise EngineInterrupted()


class _LayerRun:
    """Polls check_signal before each layer and remembers the layers run.
    On an interrupt it puts those layers' len back to the call's start
    position before re-raising, so the rows they appended lie past len and
    no later call (e.g. a verify with k = v = NULL, which reads len) takes
    them for cached rows."""

    def __init__(self, cache, pos, check_signal):
        self.cache, self.pos, self.check = cache, pos, check_signal
        self.done: list[int] = []

    def __enter__(self):
        return self

    def before(self, layer) -> None:
        _poll(self.check)
        self.done.append(layer)

    def __exit__(self, exc_type, exc, tb):
        if exc_type is not None and issubclass(exc_type, EngineInterrupted):
            for layer in self.done:
                self.cache.set_len(layer, self.pos)
        return False


@dataclass(frozen=True)
class EngineSnapshot:
    pos: int
    mtp_pos: int


# Largest token count forward_batched sends to mi_attn_verify (split-K over
# the cache: the decode kernel's form up to 4 tokens, the prefill tiles'
# split-K form above), the speculative-verify case; more tokens go to
# mi_attn_prefill, which itself splits over the past when the past is long
# next to them.
VERIFY_MAX_TOKENS = 16


def _cfg(config, key, default):
    if config is None:
        return default
    if isinstance(config, dict):
        if key in config:
            return config[key]
        tc = config.get("text_config")
        if isinstance(tc, dict) and key in tc:
            return tc[key]
        return default
    return getattr(config, key, default)


class Engine:
    def __init__(self, cache: Cache, mtp_capacity: int = 4096, config=None):
        """config: the model's config.json dict (or None for Qwen3.6's values);
        rope_theta, partial_rotary_factor and rms_norm_eps feed the
        projection-input methods (constants.rs:166-167, constants.rs:15)."""
        self.cache = cache
        hd = cache.head_dim
        self.rope_theta = float(_cfg(config, "rope_theta", 1e7))
        self.rotary_dim = int(round(float(_cfg(config, "partial_rotary_factor", 0.25)) * hd))
        self.rms_norm_eps = float(_cfg(config, "rms_norm_eps", 1e-6))
        self.mtp_cache = Cache(num_layers=1, num_q_heads=cache.num_q_heads,
                               num_kv_heads=cache.num_kv_heads, head_dim=cache.head_dim,
                               capacity=mtp_capacity)
        self._telemetry: dict[str, list[float] | float] = {}

    # -- positions -----------------------------------------------------------
    def engine_pos(self) -> int:
        return self.cache.pos

    @property
    def mtp_pos(self) -> int:
        return self.mtp_cache.pos

    def _record(self, key: str, t0: float) -> None:
        if _RECORD_TELEMETRY:
            torch.cuda.synchronize()
            self._telemetry.setdefault(key, []).append((time.perf_counter() - t0) * 1e3)

    # -- main model ------------------------------------------------------------
    def forward(self, layers, check_signal=None):
        """layers: sequence of (layer, q[H*D], k[G*D], v[G*D], gate|None).
        Returns the gated attention outputs, one per entry.

        check_signal: optional callable polled before every layer; when it
        returns True the call raises EngineInterrupted and engine_pos is not
        advanced, as the reference's per-layer poll does
        (fused_exp2.rs:1017-1019); the layers already run get their len put
        back to engine_pos, so the rows they appended lie past len and are
        overwritten by the next call at the same position."""
        t0 = time.perf_counter()
        pos = self.cache.pos
        outs = []
        with _LayerRun(self.cache, pos, check_signal) as run:
            for layer, q, k, v, gate in layers:
                run.before(layer)
                outs.append(attention.attn_step(self.cache, layer, q, k, v, pos, gate=gate))
        self.cache.set_pos(pos + 1)
        self.cache.gpu_dirty = True
        self._record("engine.full_attention_ms", t0)
        return outs

    def forward_batched(self, layers, check_signal=None):
        """layers: sequence of (layer, q[n,H,D], k[n,G*D], v[n,G*D], gate|None);
        n == 1 falls back to the token-serial step (fused_exp3.rs:169-171).
        check_signal: as for forward()."""
        t0 = time.perf_counter()
        pos = self.cache.pos
        outs, n = [], None
        with _LayerRun(self.cache, pos, check_signal) as run:
            for layer, q, k, v, gate in layers:
                run.before(layer)
                n_l = q.numel() // (self.cache.num_q_heads * self.cache.head_dim)
                if n is not None and n_l != n:
                    raise ValueError("every layer must carry the same token count")
                n = n_l
                if n == 1:
                    outs.append(attention.attn_step(self.cache, layer, q, k, v, pos, gate=gate))
                elif n <= VERIFY_MAX_TOKENS:
                    outs.append(attention.attn_verify(self.cache, layer, q, k, v, pos, gate=gate))
                else:
                    outs.append(attention.attn_prefill(self.cache, layer, q, k, v, pos, gate=gate))
        if n is not None:
            self.cache.set_pos(pos + n)
            self.cache.gpu_dirty = True
        self._record("engine.full_attention_batched_ms", t0)
        return outs

    # -- the same steps from the projections -------------------------------------
    def forward_proj(self, layers, check_signal=None):
        """layers: sequence of (layer, q_proj[H,2D] f32, k[G,D] f32, v[G,D] f32,
        q_norm_w[D] bf16, k_norm_w[D] bf16).  Norm + RoPE at engine_pos, append,
        attend [0, pos], gate from q_proj; then pos += 1.  check_signal: as for
        forward()."""
        t0 = time.perf_counter()
        pos = self.cache.pos
        outs = []
        with _LayerRun(self.cache, pos, check_signal) as run:
            for layer, qp, k, v, qw, kw in layers:
                run.before(layer)
                outs.append(attention.attn_step_proj(self.cache, layer, qp, k, v, qw, kw, pos,
                                                     rotary_dim=self.rotary_dim,
                                                     rope_theta=self.rope_theta,
                                                     eps=self.rms_norm_eps))
        self.cache.set_pos(pos + 1)
        self.cache.gpu_dirty = True
        self._record("engine.full_attention_ms", t0)
        return outs

    def forward_batched_proj(self, layers, check_signal=None):
        """layers: sequence of (layer, q_proj[n,H,2D], k[n,G,D], v[n,G,D],
        q_norm_w, k_norm_w), all f32 but the bf16 weights; token i at
        position engine_pos + i.  Returns [n,H,D] f16 per layer; pos += n.
        check_signal: as for forward()."""
        t0 = time.perf_counter()
        pos = self.cache.pos
        outs, n = [], None
        H, D = self.cache.num_q_heads, self.cache.head_dim
        with _LayerRun(self.cache, pos, check_signal) as run:
            for layer, qp, k, v, qw, kw in layers:
                run.before(layer)
                n_l = qp.numel() // (H * 2 * D)
                if n is not None and n_l != n:
                    raise ValueError("every layer must carry the same token count")
                n = n_l
                if n == 1:
                    o = attention.attn_step_proj(self.cache, layer, qp, k, v, qw, kw, pos,
                                                 rotary_dim=self.rotary_dim,
                                                 rope_theta=self.rope_theta, eps=self.rms_norm_eps)
                    outs.append(o.reshape(1, H, D))
                    continue
                q, g = attention.qk_norm_rope_append(self.cache, layer, qp, k, v, qw, kw, pos,
                                                     rotary_dim=self.rotary_dim,
                                                     rope_theta=self.rope_theta,
                                                     eps=self.rms_norm_eps)
                attend = attention.attn_verify if n <= VERIFY_MAX_TOKENS else attention.attn_prefill
                outs.append(attend(self.cache, layer, q, None, None, pos, gate=g))
        if n is not None:
            self.cache.set_pos(pos + n)
            self.cache.gpu_dirty = True
        self._record("engine.full_attention_batched_ms", t0)
        return outs

    # -- MTP draft head ----------------------------------------------------------
    def mtp_forward(self, q, k, v, gate=None):
        pos = self.mtp_cache.pos
        out = attention.attn_step(self.mtp_cache, 0, q, k, v, pos, gate=gate)
        self.mtp_cache.set_pos(pos + 1)
        return out

    def mtp_verify(self, q, k, v, gate=None):
        """K tokens appended at mtp_pos; query i attends [0, mtp_pos + i]."""
        pos = self.mtp_cache.pos
        n = q.numel() // (self.mtp_cache.num_q_heads * self.mtp_cache.head_dim)
        out = attention.attn_verify(self.mtp_cache, 0, q, k, v, pos, gate=gate)
        self.mtp_cache.set_pos(pos + n)
        return out

    def mtp_reset(self) -> None:
        self.mtp_cache.set_pos(0)

    def mtp_rollback(self, pos: int) -> None:
        self.mtp_cache.set_pos(pos)

    # -- speculative-decoding rollback ------------------------------------------------
    def snapshot_state(self) -> EngineSnapshot:
        return EngineSnapshot(self.cache.pos, self.mtp_cache.pos)

    def restore_snapshot(self, snap: EngineSnapshot) -> None:
        self.cache.set_pos(snap.pos)
        self.mtp_cache.set_pos(snap.mtp_pos)

    # -- cache transfer (the cache already lives on the device) -----------------------
    def upload_cache(self, cache: Cache) -> None:
        if cache is not self.cache:
            self.cache.copy_from(cache)
        cache.cpu_dirty = False

    def download_cache(self, cache: Cache) -> None:
        if cache is not self.cache:
            cache.copy_from(self.cache)
        cache.gpu_dirty = False

    def telemetry(self) -> dict:
        return dict(self._telemetry)
