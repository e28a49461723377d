// KV-cache state of the full-attention layers: allocation and doubling
// growth, position-only rollback, append kernels, host transfer, and the
// error channel of the whole library.
//
// Reference semantics: src/cache.rs (Cache::new :45-76, reset :84-94,
// set_pos :102-109, copy_from :112-128, FullState :273-287), the GPU KV
// buffers of src/engine/qwen35_moe/metal_context.rs (:316-319, growth
// :368-431, upload/download :804-882) and the append kernels
// kv_cache_append / kv_cache_append_n (src/engine/shaders.metal:2370-2383,
// 2774-2792).
//
// Device layout (per layer, mi::k_offset / mi::v_offset): K in 32-row blocks
// whose 16-byte column chunks are ordered as the decode kernel's MFMA A
// operand rows; V in 8-row transposed blocks [cap/8][G][D][8], so one
// 16-byte load returns the eight keys of one value column — the operand
// order the decode and prefill MFMA kernels consume without an LDS
// transpose.
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace mi {

mi_status fail(mi_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

mi_status hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MI_OK;
  mi_status st = (e == hipErrorOutOfMemory) ? MI_ERR_OOM : MI_ERR_HIP;
  return fail(st, "%s failed: %s", what, hipGetErrorString(e));
}

void clear_error() { g_err[0] = 0; }

mi_status check_shape(int32_t H, int32_t G, int32_t D) {
  if (H <= 0 || G <= 0 || D <= 0 || H % G != 0)
    return fail(MI_ERR_INVALID_ARG, "bad head shape H=%d G=%d D=%d", H, G, D);
  if (D != kHeadDim || H / G != kGroup)
    return fail(MI_ERR_UNSUPPORTED,
                "kernels are built for head_dim=%d and %d query heads per KV "
                "head; got head_dim=%d, H/G=%d",
                kHeadDim, kGroup, D, H / G);
  return MI_OK;
}

}  // namespace mi

extern "C" const char* mi_last_error(void) { return g_err; }

extern "C" const char* mi_version(void) { return "mi_attn 0.1 gfx950"; }

extern "C" void mi_roofline_peaks(double* hbm_gbps, double* f16_tflops) {
  if (hbm_gbps) *hbm_gbps = MI_PEAK_HBM_GBPS;
  if (f16_tflops) *f16_tflops = MI_PEAK_F16_TFLOPS;
}

// ------------------------------------------------------------- kernels ----

// Writes n token-major rows k[n][G*D], v[n][G*D] at rows [pos, pos+n) of
// the device layout, in one launch.  Work items [0, nk) are K chunks: one
// 16-byte chunk (8 consecutive columns of one head) of one row, moved as is
// (chunks stay contiguous in the 32-row block layout).  Items [nk, nk+nv)
// are V columns: (8-row block b, head h, 8 consecutive columns d0..d0+7);
// the thread gathers those columns of the block's rows that lie in
// [pos, pos+n) and writes them as eight 16-byte column vectors (whole block
// covered) or element by element (first/last partial block: rows outside
// the range keep their contents).
__global__ void __launch_bounds__(256)
kv_pack_kernel(const _Float16* __restrict__ k, const _Float16* __restrict__ v,
               _Float16* __restrict__ kblk, _Float16* __restrict__ vblk, int64_t pos,
               int64_t n, int G, int D) {
  const int cvec = D / 8;
  const int64_t nk = n * G * cvec;
  const int64_t b_first = pos / MI_KV_VBLOCK;
  const int64_t b_last = (pos + n - 1) / MI_KV_VBLOCK;
  const int64_t nv = (b_last - b_first + 1) * G * cvec;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < nk + nv;
       idx += (int64_t)gridDim.x * blockDim.x) {
    if (idx < nk) {
      const int64_t rr = idx / (G * cvec);
      const int h = (int)((idx / cvec) % G);
      const int c = (int)(idx % cvec);
      *(f16x8*)(kblk + mi::k_offset(pos + rr, h, 8 * c, G, D)) =
          *(const f16x8*)(k + rr * G * D + h * D + 8 * c);
      continue;
    }
    const int64_t vi = idx - nk;
    const int64_t b = b_first + vi / (G * cvec);
    const int h = (int)((vi / cvec) % G);
    const int d0 = (int)(vi % cvec) * 8;
    const int64_t r0 = b * MI_KV_VBLOCK;
    _Float16* blk = vblk + ((b * G + h) * (int64_t)D + d0) * MI_KV_VBLOCK;
    if (r0 >= pos && r0 + MI_KV_VBLOCK <= pos + n) {
      f16x8 rowv[8];
#pragma unroll
      for (int rr = 0; rr < 8; rr++)
        rowv[rr] = *(const f16x8*)(v + (r0 + rr - pos) * G * D + h * D + d0);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        f16x8 col;
#pragma unroll
        for (int rr = 0; rr < 8; rr++) col[rr] = rowv[rr][i];
        *(f16x8*)(blk + i * MI_KV_VBLOCK) = col;
      }
    } else {
      for (int rr = 0; rr < 8; rr++) {
        const int64_t r = r0 + rr;
        if (r < pos || r >= pos + n) continue;
        const f16x8 row = *(const f16x8*)(v + (r - pos) * G * D + h * D + d0);
#pragma unroll
        for (int i = 0; i < 8; i++) blk[i * MI_KV_VBLOCK + rr] = row[i];
      }
    }
  }
}

// The same for head_dim 256 with 32-bit item indices (the host checks the
// item count fits): the row / head / chunk of an item come from shifts and
// one 32-bit division by G instead of the generic kernel's 64-bit divisions
// by run-time values, which cost more than the copy's own instructions.
// BLOCKED orders the K items by destination: item (32-row block, head, row
// half u, chunk c, row slot j) with j fastest, so each store instruction of
// a wave writes 1 KiB of contiguous block layout (four chunks of 16 row
// slots) and each load reads 64-byte pieces of 16 rows; items whose row lies
// outside [pos, pos+n) do nothing.
// Row-major order (each wave storing 16 bytes every 256) suits a few rows.
template <bool BLOCKED>
__global__ void __launch_bounds__(256)
kv_pack256_kernel(const _Float16* __restrict__ k, const _Float16* __restrict__ v,
                  _Float16* __restrict__ kblk, _Float16* __restrict__ vblk, int64_t pos,
                  uint32_t n, uint32_t G, uint32_t nblk, uint32_t nkblk) {
  constexpr int D = mi::kHeadDim;
  constexpr uint32_t cvec = D / 8;  // 16-byte chunks per head row
  // BLOCKED: one item moves four chunks c0 + 4 i of one row slot (loads
  // first, 64 bytes of the source row; then four stores)
  const uint32_t nk = BLOCKED ? nkblk * G * 2 * cvec * 4 : n * G * cvec;
  const uint32_t total = nk + nblk * G * cvec;
  const int64_t b_first = pos / MI_KV_VBLOCK;
  for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += gridDim.x * blockDim.x) {
    if (idx < nk) {
      if (BLOCKED) {
        // idx = (((bh * 2 + u) * 2 + cq) * 4 + cg) * 16 + j, c0 = 16 cq + cg
        const uint32_t j = idx & 15, c0 = 16 * ((idx >> 6) & 1) + ((idx >> 4) & 3);
        const uint32_t u = (idx >> 7) & 1;
        const uint32_t bh = idx >> 8, bb = bh / G, h = bh - bb * G;
        const int64_t b = pos / MI_KV_KBLOCK + bb;
        const int64_t r = b * MI_KV_KBLOCK + (((j >> 2) << 3) | (u << 2) | (j & 3));
        if (r < pos || r >= pos + n) continue;
        const _Float16* src = k + ((r - pos) * G + h) * D + 8 * c0;
        _Float16* dst = kblk + ((((b * G + h) * 2 + u) * cvec + c0) * 16 + j) * 8;
        f16x8 x[4];
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = *(const f16x8*)(src + 32 * i);
#pragma unroll
        for (int i = 0; i < 4; i++) *(f16x8*)(dst + 4 * 16 * 8 * i) = x[i];
      } else {
        const uint32_t rh = idx / cvec, c = idx % cvec;
        const uint32_t rr = rh / G, h = rh - rr * G;
        *(f16x8*)(kblk + mi::k_offset(pos + rr, (int)h, 8 * c, (int)G, D)) =
            *(const f16x8*)(k + ((int64_t)rr * G + h) * D + 8 * c);
      }
      continue;
    }
    const uint32_t vi = idx - nk;
    const uint32_t bh = vi / cvec, d0 = (vi % cvec) * 8;
    const uint32_t bb = bh / G, h = bh - bb * G;
    const int64_t b = b_first + bb;
    const int64_t r0 = b * MI_KV_VBLOCK;
    _Float16* blk = vblk + ((b * G + h) * (int64_t)D + d0) * MI_KV_VBLOCK;
    if (r0 >= pos && r0 + MI_KV_VBLOCK <= pos + n) {
      f16x8 rowv[8];
#pragma unroll
      for (int rr = 0; rr < 8; rr++)
        rowv[rr] = *(const f16x8*)(v + ((r0 + rr - pos) * G + h) * D + d0);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        f16x8 col;
#pragma unroll
        for (int rr = 0; rr < 8; rr++) col[rr] = rowv[rr][i];
        *(f16x8*)(blk + i * MI_KV_VBLOCK) = col;
      }
    } else {
      for (int rr = 0; rr < 8; rr++) {
        const int64_t r = r0 + rr;
        if (r < pos || r >= pos + n) continue;
        const f16x8 row = *(const f16x8*)(v + ((r - pos) * G + h) * D + d0);
#pragma unroll
        for (int i = 0; i < 8; i++) blk[i * MI_KV_VBLOCK + rr] = row[i];
      }
    }
  }
}

// ---------------------------------------------------------- host helpers --

namespace {

int64_t round_cap(int64_t rows) {
  if (rows < MI_KV_CAP_ALIGN) rows = MI_KV_CAP_ALIGN;
  return (rows + MI_KV_CAP_ALIGN - 1) / MI_KV_CAP_ALIGN * MI_KV_CAP_ALIGN;
}

// Host-state queries: a non-null handle and a layer in range (no device).
mi_status layer_in_range(const mi_kv* kv, int32_t layer) {
  if (!kv) return mi::fail(MI_ERR_INVALID_ARG, "null mi_kv handle");
  if (layer < 0 || layer >= kv->layers)
    return mi::fail(MI_ERR_INVALID_ARG, "layer %d out of [0, %d)", layer, kv->layers);
  return MI_OK;
}

size_t layer_bytes(const mi_kv* kv, int64_t cap) {
  return (size_t)cap * kv->G * kv->D * sizeof(_Float16);
}

void free_layers(mi_kv* kv) {
  for (auto p : kv->k) if (p) (void)hipFree(p);
  for (auto p : kv->v) if (p) (void)hipFree(p);
  kv->k.clear();
  kv->v.clear();
}

// Allocates `cap`-row buffers for every layer, copies the first
// `keep_rows` rows of the old buffers (all of them: rows past len are stale
// but must survive, as the reference's whole-buffer regrow keeps them) and
// zero-fills the rest.
mi_status realloc_layers(mi_kv* kv, int64_t cap, int64_t keep_rows) {
  std::vector<_Float16*> nk(kv->layers, nullptr), nv(kv->layers, nullptr);
  size_t bytes = layer_bytes(kv, cap);
  size_t keep = layer_bytes(kv, keep_rows);
  auto drop_new = [&](hipError_t e, const char* what) {
    for (auto p : nk) if (p) (void)hipFree(p);
    for (auto p : nv) if (p) (void)hipFree(p);
    return mi::hip_status(e, what);
  };
  // Work already enqueued on any stream (appends into the old buffers
  // included) completes before the rows are copied.
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return mi::hip_status(e, "hipDeviceSynchronize");
  for (int l = 0; l < kv->layers; l++) {
    if ((e = hipMalloc((void**)&nk[l], bytes)) != hipSuccess ||
        (e = hipMalloc((void**)&nv[l], bytes)) != hipSuccess)
      return drop_new(e, "hipMalloc(kv cache)");
    if (keep && ((e = hipMemcpy(nk[l], kv->k[l], keep, hipMemcpyDeviceToDevice)) != hipSuccess ||
                 (e = hipMemcpy(nv[l], kv->v[l], keep, hipMemcpyDeviceToDevice)) != hipSuccess))
      return drop_new(e, "hipMemcpy(kv cache rows)");
    if ((e = hipMemset((char*)nk[l] + keep, 0, bytes - keep)) != hipSuccess ||
        (e = hipMemset((char*)nv[l] + keep, 0, bytes - keep)) != hipSuccess)
      return drop_new(e, "hipMemset(kv cache)");
  }
  if ((e = hipDeviceSynchronize()) != hipSuccess) return drop_new(e, "hipDeviceSynchronize");
  free_layers(kv);
  kv->k = nk;
  kv->v = nv;
  kv->cap = cap;
  return MI_OK;
}

}  // namespace

namespace mi {

mi_status check_kv(const mi_kv* kv) {
  if (!kv) return mi::fail(MI_ERR_INVALID_ARG, "null mi_kv handle");
  int dev = 0;
  MI_HIP(hipGetDevice(&dev));
  if (dev != kv->device)
    return mi::fail(MI_ERR_INVALID_ARG, "the handle belongs to device %d; device %d is current",
                    kv->device, dev);
  return MI_OK;
}

mi_status check_layer(const mi_kv* kv, int32_t layer) {
  MI_TRY(check_kv(kv));
  if (layer < 0 || layer >= kv->layers)
    return mi::fail(MI_ERR_INVALID_ARG, "layer %d out of [0, %d)", layer, kv->layers);
  return MI_OK;
}

// Refuses an allocation on behalf of work enqueued on `stream` while that
// stream is being captured into a graph: the captured kernels would hold
// the address of memory the allocation replaces.
mi_status no_capture(hipStream_t stream, const char* what) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  MI_HIP(hipStreamIsCapturing(stream, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return fail(MI_ERR_INVALID_ARG,
                "%s needs to grow device memory while the stream is being captured; make one "
                "eager call of the same or larger size first (mi_kv_reserve for the cache)",
                what);
  return MI_OK;
}

// A grown workspace replaces the old one.  If a graph capture has used the
// old one, it is kept (not freed) until mi_kv_destroy: the captured graph
// holds its address and stays valid.  Otherwise it is freed at once
// (hipFree waits for the device work that may still use it).
mi_status kv_workspace(mi_kv* kv, size_t bytes, hipStream_t stream, void** ws) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  MI_HIP(hipStreamIsCapturing(stream, &cs));
  const bool capturing = cs != hipStreamCaptureStatusNone;
  if (bytes > kv->ws_bytes) {
    MI_TRY(no_capture(stream, "the split-K workspace"));
    void* p = nullptr;
    const size_t b = bytes + bytes / 4;
    MI_HIP(hipMalloc(&p, b));
    if (kv->ws) {
      if (kv->ws_captured) kv->ws_retired.push_back(kv->ws);
      else MI_HIP(hipFree(kv->ws));
    }
    kv->ws = p;
    kv->ws_bytes = b;
    kv->ws_captured = false;
  }
  if (capturing) kv->ws_captured = true;
  *ws = kv->ws;
  return MI_OK;
}

mi_status kv_grow(mi_kv* kv, int64_t rows, hipStream_t stream) {
  if (rows <= kv->cap) return MI_OK;
  MI_TRY(no_capture(stream, "the KV cache"));
  return mi_kv_reserve(kv, rows);
}

mi_status kv_pack_rows(const _Float16* k, const _Float16* v, _Float16* dst_k, _Float16* dst_v,
                       int64_t pos, int64_t n, int G, int D, hipStream_t stream) {
  const int64_t nblk = (pos + n - 1) / MI_KV_VBLOCK - pos / MI_KV_VBLOCK + 1;
  const int64_t items = (n + nblk) * G * (D / 8);
  const int grid = (int)std::min<int64_t>((items + 255) / 256, 4096);
  // destination-ordered K items from a few blocks' worth of rows on
  const int64_t nkblk = (pos + n - 1) / MI_KV_KBLOCK - pos / MI_KV_KBLOCK + 1;
  const int64_t bitems = (nkblk * MI_KV_KBLOCK / 4 + nblk) * G * (D / 8);
  const bool blocked = n >= 4 * MI_KV_KBLOCK;
  const int bgrid = (int)std::min<int64_t>((bitems + 255) / 256, 4096);
  if (D == kHeadDim && blocked && bitems + (int64_t)bgrid * 256 < ((int64_t)1 << 32)) {
    MI_HIP(mi::launch("kv_pack", kv_pack256_kernel<true>, dim3(bgrid), dim3(256), 0, stream, k, v,
                      dst_k, dst_v, pos, (uint32_t)n, (uint32_t)G, (uint32_t)nblk,
                      (uint32_t)nkblk));
    return MI_OK;
  }
  if (D == kHeadDim && items + (int64_t)grid * 256 < ((int64_t)1 << 32)) {
    MI_HIP(mi::launch("kv_pack", kv_pack256_kernel<false>, dim3(grid), dim3(256), 0, stream, k, v,
                      dst_k, dst_v, pos, (uint32_t)n, (uint32_t)G, (uint32_t)nblk, 0u));
    return MI_OK;
  }
  MI_HIP(mi::launch("kv_pack", kv_pack_kernel, dim3(grid), dim3(256), 0, stream, k, v, dst_k,
                    dst_v, pos, n, G, D));
  return MI_OK;
}

mi_status kv_append_rows(mi_kv* kv, int32_t layer, const _Float16* k,
                         const _Float16* v, int64_t pos, int32_t n,
                         hipStream_t stream) {
  return kv_pack_rows(k, v, kv->k[layer], kv->v[layer], pos, n, kv->G, kv->D, stream);
}

}  // namespace mi

// ------------------------------------------------------------- C ABI ------

extern "C" mi_status mi_kv_create(int32_t num_layers, int32_t num_q_heads,
                                  int32_t num_kv_heads, int32_t head_dim,
                                  int64_t capacity, mi_kv** out) {
  mi::clear_error();
  if (!out) return mi::fail(MI_ERR_INVALID_ARG, "null output pointer");
  *out = nullptr;
  if (num_layers <= 0) return mi::fail(MI_ERR_INVALID_ARG, "num_layers=%d", num_layers);
  if (capacity < 0) return mi::fail(MI_ERR_INVALID_ARG, "capacity=%lld", (long long)capacity);
  MI_TRY(mi::check_shape(num_q_heads, num_kv_heads, head_dim));
  mi_kv* kv = new mi_kv();
  kv->layers = num_layers;
  kv->H = num_q_heads;
  kv->G = num_kv_heads;
  kv->D = head_dim;
  kv->len.assign(num_layers, 0);
  (void)hipGetDevice(&kv->device);
  mi_status st = realloc_layers(kv, round_cap(capacity), 0);
  if (st != MI_OK) {
    delete kv;
    return st;
  }
  // the in-launch merge state (its counters must start at zero)
  hipError_t e = hipMalloc(&kv->mstate, mi::merge_state_bytes(kv->G));
  if (e == hipSuccess) e = hipMemset(kv->mstate, 0, mi::merge_state_bytes(kv->G));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    mi_kv_destroy(kv);
    return mi::hip_status(e, "in-launch merge state");
  }
  kv->merge_ok = mi::xcd_round_robin();
  *out = kv;
  return MI_OK;
}

extern "C" void mi_kv_destroy(mi_kv* kv) {
  if (!kv) return;
  (void)hipDeviceSynchronize();
  free_layers(kv);
  if (kv->ws) (void)hipFree(kv->ws);
  if (kv->mstate) (void)hipFree(kv->mstate);
  for (void* p : kv->ws_retired) (void)hipFree(p);
  delete kv;
}

extern "C" mi_status mi_kv_reserve(mi_kv* kv, int64_t capacity) {
  mi::clear_error();
  MI_TRY(mi::check_kv(kv));
  if (capacity <= kv->cap) return MI_OK;
  // Doubling growth (metal_context.rs:368-431), at least to `capacity`.
  int64_t cap = kv->cap;
  while (cap < capacity) cap *= 2;
  return realloc_layers(kv, round_cap(cap), kv->cap);
}

extern "C" mi_status mi_kv_capacity(const mi_kv* kv, int64_t* capacity) {
  if (!kv || !capacity) return mi::fail(MI_ERR_INVALID_ARG, "null argument");
  *capacity = kv->cap;
  return MI_OK;
}

extern "C" mi_status mi_kv_shape(const mi_kv* kv, int32_t* num_layers,
                                 int32_t* num_q_heads, int32_t* num_kv_heads,
                                 int32_t* head_dim) {
  if (!kv) return mi::fail(MI_ERR_INVALID_ARG, "null mi_kv handle");
  if (num_layers) *num_layers = kv->layers;
  if (num_q_heads) *num_q_heads = kv->H;
  if (num_kv_heads) *num_kv_heads = kv->G;
  if (head_dim) *head_dim = kv->D;
  return MI_OK;
}

extern "C" mi_status mi_kv_set_pos(mi_kv* kv, int64_t pos) {
  mi::clear_error();
  if (!kv) return mi::fail(MI_ERR_INVALID_ARG, "null mi_kv handle");
  if (pos < 0 || pos > kv->cap)
    return mi::fail(MI_ERR_OUT_OF_RANGE, "pos %lld outside [0, capacity %lld]",
                    (long long)pos, (long long)kv->cap);
  kv->pos = pos;
  for (auto& l : kv->len) l = pos;
  return MI_OK;
}

extern "C" mi_status mi_kv_reset(mi_kv* kv) { return mi_kv_set_pos(kv, 0); }

extern "C" mi_status mi_kv_pos(const mi_kv* kv, int64_t* pos) {
  if (!kv || !pos) return mi::fail(MI_ERR_INVALID_ARG, "null argument");
  *pos = kv->pos;
  return MI_OK;
}

extern "C" mi_status mi_kv_len(const mi_kv* kv, int32_t layer, int64_t* len) {
  MI_TRY(layer_in_range(kv, layer));
  if (!len) return mi::fail(MI_ERR_INVALID_ARG, "null argument");
  *len = kv->len[layer];
  return MI_OK;
}

extern "C" mi_status mi_kv_set_len(mi_kv* kv, int32_t layer, int64_t len) {
  MI_TRY(layer_in_range(kv, layer));
  if (len < 0 || len > kv->cap)
    return mi::fail(MI_ERR_OUT_OF_RANGE, "len %lld outside [0, capacity %lld]",
                    (long long)len, (long long)kv->cap);
  kv->len[layer] = len;
  return MI_OK;
}

extern "C" mi_status mi_kv_layer_ptrs(mi_kv* kv, int32_t layer, mi_f16** k,
                                      mi_f16** v) {
  MI_TRY(mi::check_layer(kv, layer));
  if (k) *k = (mi_f16*)kv->k[layer];
  if (v) *v = (mi_f16*)kv->v[layer];
  return MI_OK;
}

extern "C" mi_status mi_kv_append(mi_kv* kv, int32_t layer, const mi_f16* k,
                                  const mi_f16* v, int64_t pos, int32_t n,
                                  mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!k || !v) return mi::fail(MI_ERR_INVALID_ARG, "null k/v");
  if (n <= 0) return mi::fail(MI_ERR_INVALID_ARG, "n=%d", n);
  if (pos < 0) return mi::fail(MI_ERR_OUT_OF_RANGE, "pos=%lld", (long long)pos);
  MI_TRY(mi::kv_grow(kv, pos + n, (hipStream_t)stream));
  MI_TRY(mi::kv_append_rows(kv, layer, (const _Float16*)k, (const _Float16*)v, pos, n,
                            (hipStream_t)stream));
  kv->len[layer] = pos + n;
  return MI_OK;
}

extern "C" mi_status mi_kv_pack(const mi_f16* k_rows, const mi_f16* v_rows, mi_f16* dst_k,
                                mi_f16* dst_v, int64_t row0, int64_t rows,
                                int32_t num_kv_heads, int32_t head_dim, mi_stream stream) {
  mi::clear_error();
  if (!k_rows || !v_rows || !dst_k || !dst_v) return mi::fail(MI_ERR_INVALID_ARG, "null pointer");
  if (rows <= 0 || row0 < 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8)
    return mi::fail(MI_ERR_INVALID_ARG, "bad pack arguments");
  return mi::kv_pack_rows((const _Float16*)k_rows, (const _Float16*)v_rows, (_Float16*)dst_k,
                          (_Float16*)dst_v, row0, rows, num_kv_heads, head_dim,
                          (hipStream_t)stream);
}

namespace {

// Host image of the K and V blocks covering rows [row0, row0+rows) of one
// layer, with accessors by (row, head, column).
struct HostBlocks {
  const mi_kv* kv;
  int64_t kb0, vb0;  // first K / V block
  std::vector<_Float16> k, v;
  _Float16& K(int64_t r, int h, int i) {
    return k[mi::k_offset(r, h, i, kv->G, kv->D) - kb0 * MI_KV_KBLOCK * kv->G * kv->D];
  }
  _Float16& V(int64_t r, int h, int i) {
    return v[mi::v_offset(r, h, i, kv->G, kv->D) - vb0 * MI_KV_VBLOCK * kv->G * kv->D];
  }
};

mi_status fetch_blocks(const mi_kv* kv, int32_t layer, int64_t row0, int64_t rows,
                       HostBlocks& hb) {
  const int64_t rl = (int64_t)kv->G * kv->D;
  hb.kv = kv;
  hb.kb0 = row0 / MI_KV_KBLOCK;
  const int64_t kb1 = (row0 + rows - 1) / MI_KV_KBLOCK;
  hb.vb0 = row0 / MI_KV_VBLOCK;
  const int64_t vb1 = (row0 + rows - 1) / MI_KV_VBLOCK;
  hb.k.resize((size_t)((kb1 - hb.kb0 + 1) * MI_KV_KBLOCK * rl));
  hb.v.resize((size_t)((vb1 - hb.vb0 + 1) * MI_KV_VBLOCK * rl));
  MI_HIP(hipMemcpy(hb.k.data(), kv->k[layer] + hb.kb0 * MI_KV_KBLOCK * rl,
                   hb.k.size() * sizeof(_Float16), hipMemcpyDeviceToHost));
  MI_HIP(hipMemcpy(hb.v.data(), kv->v[layer] + hb.vb0 * MI_KV_VBLOCK * rl,
                   hb.v.size() * sizeof(_Float16), hipMemcpyDeviceToHost));
  return MI_OK;
}

mi_status check_rows(const mi_kv* kv, int64_t row0, int64_t rows) {
  if (row0 < 0 || rows < 0 || row0 + rows > kv->cap)
    return mi::fail(MI_ERR_OUT_OF_RANGE, "rows [%lld, %lld) outside capacity %lld",
                    (long long)row0, (long long)(row0 + rows), (long long)kv->cap);
  return MI_OK;
}

}  // namespace

extern "C" mi_status mi_kv_upload(mi_kv* kv, int32_t layer, const mi_f16* host_k,
                                  const mi_f16* host_v, int64_t row0, int64_t rows) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!host_k || !host_v) return mi::fail(MI_ERR_INVALID_ARG, "null host buffer");
  MI_TRY(check_rows(kv, row0, rows));
  if (rows == 0) return MI_OK;
  MI_HIP(hipDeviceSynchronize());
  HostBlocks hb;
  MI_TRY(fetch_blocks(kv, layer, row0, rows, hb));  // keeps rows outside the range
  const _Float16* sk = (const _Float16*)host_k;
  const _Float16* sv = (const _Float16*)host_v;
  const int64_t rl = (int64_t)kv->G * kv->D;
  for (int64_t r = row0; r < row0 + rows; r++)
    for (int h = 0; h < kv->G; h++)
      for (int i = 0; i < kv->D; i++) {
        hb.K(r, h, i) = sk[(r - row0) * rl + h * kv->D + i];
        hb.V(r, h, i) = sv[(r - row0) * rl + h * kv->D + i];
      }
  MI_HIP(hipMemcpy(kv->k[layer] + hb.kb0 * MI_KV_KBLOCK * rl, hb.k.data(),
                   hb.k.size() * sizeof(_Float16), hipMemcpyHostToDevice));
  MI_HIP(hipMemcpy(kv->v[layer] + hb.vb0 * MI_KV_VBLOCK * rl, hb.v.data(),
                   hb.v.size() * sizeof(_Float16), hipMemcpyHostToDevice));
  return MI_OK;
}

extern "C" mi_status mi_kv_download(const mi_kv* kv, int32_t layer, mi_f16* host_k,
                                    mi_f16* host_v, int64_t row0, int64_t rows) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!host_k || !host_v) return mi::fail(MI_ERR_INVALID_ARG, "null host buffer");
  MI_TRY(check_rows(kv, row0, rows));
  if (rows == 0) return MI_OK;
  MI_HIP(hipDeviceSynchronize());
  HostBlocks hb;
  MI_TRY(fetch_blocks(kv, layer, row0, rows, hb));
  _Float16* dk = (_Float16*)host_k;
  _Float16* dv = (_Float16*)host_v;
  const int64_t rl = (int64_t)kv->G * kv->D;
  for (int64_t r = row0; r < row0 + rows; r++)
    for (int h = 0; h < kv->G; h++)
      for (int i = 0; i < kv->D; i++) {
        dk[(r - row0) * rl + h * kv->D + i] = hb.K(r, h, i);
        dv[(r - row0) * rl + h * kv->D + i] = hb.V(r, h, i);
      }
  return MI_OK;
}

extern "C" mi_status mi_kv_copy_from(mi_kv* dst, const mi_kv* src) {
  mi::clear_error();
  MI_TRY(mi::check_kv(dst));
  MI_TRY(mi::check_kv(src));
  if (dst->layers != src->layers || dst->H != src->H || dst->G != src->G || dst->D != src->D)
    return mi::fail(MI_ERR_INVALID_ARG, "cache shape mismatch");
  if (dst == src) return MI_OK;
  if (dst->cap < src->cap) MI_TRY(realloc_layers(dst, src->cap, 0));
  MI_HIP(hipDeviceSynchronize());
  size_t bytes = layer_bytes(src, src->cap);
  for (int l = 0; l < src->layers; l++) {
    MI_HIP(hipMemcpy(dst->k[l], src->k[l], bytes, hipMemcpyDeviceToDevice));
    MI_HIP(hipMemcpy(dst->v[l], src->v[l], bytes, hipMemcpyDeviceToDevice));
  }
  MI_HIP(hipDeviceSynchronize());
  dst->pos = src->pos;
  dst->len = src->len;
  return MI_OK;
}
