"""Device KV cache of the full-attention layers, with the reference's
`Cache` API (src/python_bindings.rs:59-100 over src/cache.rs).

`Cache(config)` allocates one f16 K/V store per full-attention layer on the
current GPU through mi_kv_create.  Model layer indices are those of the
reference: with linear-attention layers present, layer i is full attention
when (i + 1) % 4 == 0 (src/cache.rs:64, src/constants.rs:18); without them
every layer is.  Semantics kept from the reference:

  pos / set_pos(p)  position-only rollback: len = p on every layer, no row
                    is modified (cache.rs:102-109)
  reset()           set_pos(0) (cache.rs:84-94; linear state is not held here)
  copy_from(other)  rows, len and pos (cache.rs:112-128)
  save / load       flat binary + JSON manifest {"tensors": {name: {offset,
                    size, shape, dtype}}}, names cache.layer_{i}.k_cache /
                    v_cache / len and cache.pos written last (cache.rs:133-231).
                    K/V are written as float16 [capacity, kv_dim]; load also
                    accepts the reference's float32 files (exact narrowing is
                    not possible in general: values are rounded to nearest f16)

Differences by design: capacity grows by doubling instead of the fixed
MAX_SEQ = 4096 (src/constants.rs:12); the store is f16, not f32.
"""
from __future__ import annotations

import ctypes as C
import json

import numpy as np

from . import _lib

FULL_ATTN_INTERVAL = 4


def _cfg_get(config, key, default=None):
    if config is None:
        return default
    if isinstance(config, dict):
        if key in config:
            return config[key]
        tc = config.get("text_config")  # model/config.rs text_config fallback
        if isinstance(tc, dict) and key in tc:
            return tc[key]
        return default
    return getattr(config, key, default)


class Cache:
    """KV cache handle (one mi_kv).  Not thread-safe (the reference's
    pyclass is `unsendable`)."""

    def __init__(self, config=None, *, num_layers: int | None = None, num_q_heads: int = 16,
                 num_kv_heads: int = 2, head_dim: int = 256, capacity: int = 4096):
        n_hidden = _cfg_get(config, "num_hidden_layers", num_layers or 1)
        num_q_heads = _cfg_get(config, "num_attention_heads", num_q_heads)
        num_kv_heads = _cfg_get(config, "num_key_value_heads", num_kv_heads)
        head_dim = _cfg_get(config, "head_dim", head_dim)
        has_linear = (_cfg_get(config, "linear_num_value_heads", 0) or 0) > 0 and \
                     (_cfg_get(config, "linear_num_key_heads", 0) or 0) > 0
        if has_linear:
            self.full_layers = [i for i in range(n_hidden) if (i + 1) % FULL_ATTN_INTERVAL == 0]
        else:
            self.full_layers = list(range(n_hidden))
        self._slot = {layer: s for s, layer in enumerate(self.full_layers)}
        self.num_layers = n_hidden
        self.num_q_heads = int(num_q_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.kv_dim = self.num_kv_heads * self.head_dim
        h = C.c_void_p()
        _lib.check(_lib.lib().mi_kv_create(len(self.full_layers), self.num_q_heads,
                                           self.num_kv_heads, self.head_dim, int(capacity),
                                           C.byref(h)))
        self._h = h
        # dirty-flag protocol of src/python_bindings.rs:573-597 / cache.rs:36-41
        self.cpu_dirty = False
        self.gpu_dirty = False

    # -- lifetime ---------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            _lib.lib().mi_kv_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- indexing ---------------------------------------------------------
    def slot(self, layer: int) -> int:
        """Full-attention slot of model layer `layer`; raises like the
        reference's as_full() panic (cache.rs:17-19) on a linear layer."""
        try:
            return self._slot[layer]
        except KeyError:
            raise ValueError(f"layer {layer} is not a full-attention layer") from None

    # -- position ---------------------------------------------------------
    @property
    def pos(self) -> int:
        v = C.c_int64()
        _lib.check(_lib.lib().mi_kv_pos(self._h, C.byref(v)))
        return v.value

    def set_pos(self, pos: int) -> None:
        _lib.check(_lib.lib().mi_kv_set_pos(self._h, int(pos)))

    def reset(self) -> None:
        _lib.check(_lib.lib().mi_kv_reset(self._h))
        self.cpu_dirty = True
        self.gpu_dirty = False

    def len(self, layer: int) -> int:
        v = C.c_int64()
        _lib.check(_lib.lib().mi_kv_len(self._h, self.slot(layer), C.byref(v)))
        return v.value

    def set_len(self, layer: int, length: int) -> None:
        _lib.check(_lib.lib().mi_kv_set_len(self._h, self.slot(layer), int(length)))

    @property
    def capacity(self) -> int:
        v = C.c_int64()
        _lib.check(_lib.lib().mi_kv_capacity(self._h, C.byref(v)))
        return v.value

    def reserve(self, capacity: int) -> None:
        _lib.check(_lib.lib().mi_kv_reserve(self._h, int(capacity)))

    def layer_ptrs(self, layer: int) -> tuple[int, int]:
        k, v = C.c_void_p(), C.c_void_p()
        _lib.check(_lib.lib().mi_kv_layer_ptrs(self._h, self.slot(layer), C.byref(k), C.byref(v)))
        return k.value, v.value

    # -- host transfer ------------------------------------------------------
    def download(self, layer: int, rows: int | None = None, row0: int = 0):
        """Token-major host copies (k, v) of rows [row0, row0+rows) as
        float16 arrays [rows, kv_dim]; rows defaults to len(layer) - row0."""
        if rows is None:
            rows = self.len(layer) - row0
        k = np.empty((rows, self.kv_dim), dtype=np.float16)
        v = np.empty((rows, self.kv_dim), dtype=np.float16)
        _lib.check(_lib.lib().mi_kv_download(self._h, self.slot(layer),
                                             k.ctypes.data_as(C.c_void_p),
                                             v.ctypes.data_as(C.c_void_p), int(row0), int(rows)))
        return k, v

    def upload(self, layer: int, k: np.ndarray, v: np.ndarray, row0: int = 0) -> None:
        k = np.ascontiguousarray(k, dtype=np.float16).reshape(-1, self.kv_dim)
        v = np.ascontiguousarray(v, dtype=np.float16).reshape(-1, self.kv_dim)
        if k.shape != v.shape:
            raise ValueError("k and v shapes differ")
        if row0 + k.shape[0] > self.capacity:
            self.reserve(row0 + k.shape[0])
        _lib.check(_lib.lib().mi_kv_upload(self._h, self.slot(layer),
                                           k.ctypes.data_as(C.c_void_p),
                                           v.ctypes.data_as(C.c_void_p), int(row0), k.shape[0]))

    def copy_from(self, other: "Cache") -> None:
        _lib.check(_lib.lib().mi_kv_copy_from(self._h, other._h))

    # -- persistence --------------------------------------------------------
    def save(self, bin_path: str, json_path: str) -> None:
        """Writes the reference's manifest layout (cache.rs:133-175) with f16
        K/V and only the full-attention layers.  Files saved here load here
        (and the reference's float32 files load here too); the reference's
        Cache::load reads every tensor as float32 over its full layer list,
        so it cannot read these."""
        if self.gpu_dirty:
            import sys
            print("[cache] WARNING: saving cache with gpu_dirty=true", file=sys.stderr)
        tensors = {}
        offset = 0
        cap = self.capacity
        with open(bin_path, "wb") as f:
            for layer in self.full_layers:
                k, v = self.download(layer, rows=cap)
                for name, arr in (("k_cache", k), ("v_cache", v)):
                    b = arr.tobytes()
                    f.write(b)
                    tensors[f"cache.layer_{layer}.{name}"] = {
                        "offset": offset, "size": len(b), "shape": [cap, self.kv_dim],
                        "dtype": "float16"}
                    offset += len(b)
                b = np.array([self.len(layer)], dtype=np.uint32).tobytes()
                f.write(b)
                tensors[f"cache.layer_{layer}.len"] = {"offset": offset, "size": 4, "shape": [],
                                                       "dtype": "uint32"}
                offset += 4
            b = np.array([self.pos], dtype=np.uint32).tobytes()
            f.write(b)
            tensors["cache.pos"] = {"offset": offset, "size": 4, "shape": [], "dtype": "uint32"}
        with open(json_path, "w") as f:
            json.dump({"tensors": tensors}, f, indent=2)

    @staticmethod
    def load(bin_path: str, json_path: str, config=None, **kw) -> "Cache":
        with open(json_path) as f:
            manifest = json.load(f)
        tensors = manifest.get("tensors")
        if not isinstance(tensors, dict):
            raise OSError("No 'tensors' key in manifest")
        data = np.memmap(bin_path, dtype=np.uint8, mode="r")

        def read(name, dtype):
            t = tensors.get(name)
            if t is None:
                raise OSError(f"missing tensor: {name}")
            off, size = int(t["offset"]), int(t["size"])
            return np.frombuffer(data[off:off + size], dtype=dtype), t

        full = sorted(int(k.split(".")[1][6:]) for k in tensors
                      if k.startswith("cache.layer_") and k.endswith(".k_cache"))
        if not full:
            raise OSError("manifest holds no full-attention layer")
        first, t0 = read(f"cache.layer_{full[0]}.k_cache", np.uint8)
        kv_dim = int(t0["shape"][1])
        if config is None:
            n_hidden = max(full) + 1
            gaps = any((i + 1) % FULL_ATTN_INTERVAL for i in full)
            config = {"num_hidden_layers": n_hidden, "num_key_value_heads": kw.pop("num_kv_heads", 2),
                      "num_attention_heads": kw.pop("num_q_heads", 16)}
            config["head_dim"] = kv_dim // config["num_key_value_heads"]
            if not gaps and len(full) < n_hidden:
                config["linear_num_value_heads"] = 1
                config["linear_num_key_heads"] = 1
        cap = int(t0["shape"][0])
        cache = Cache(config, capacity=cap, **kw)
        if cache.full_layers != full:
            raise OSError(f"manifest layers {full} do not match the config's {cache.full_layers}")
        for layer in full:
            arrs = []
            for name in ("k_cache", "v_cache"):
                t = tensors[f"cache.layer_{layer}.{name}"]
                dt = {"float16": np.float16, "float32": np.float32}.get(t["dtype"])
                if dt is None:
                    raise OSError(f"unsupported dtype {t['dtype']}")
                a, _ = read(f"cache.layer_{layer}.{name}", dt)
                arrs.append(a.reshape(-1, kv_dim).astype(np.float16))
            cache.upload(layer, arrs[0], arrs[1])
            ln, _ = read(f"cache.layer_{layer}.len", np.uint32)
            cache.set_len(layer, int(ln[0]))
        pos, _ = read("cache.pos", np.uint32)
        # restore pos without touching per-layer len
        lens = {layer: cache.len(layer) for layer in full}
        cache.set_pos(int(pos[0]))
        for layer, ln in lens.items():
            cache.set_len(layer, ln)
        cache.cpu_dirty = True
        del data
        return cache

    def __repr__(self) -> str:
        return f"Cache(pos={self.pos})"

