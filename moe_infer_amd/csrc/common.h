// Shared definitions of the gfx950 attention library: vector types, MFMA
// wrappers, the error channel behind mi_last_error(), and the internal
// layout of an mi_kv handle.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <vector>

#include "mi_attn.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// MI_HIP for use inside namespace mi before the macros below.
#define MI_HIP_RAW(call)                                        \
  do {                                                          \
    hipError_t e_ = (call);                                     \
    if (e_ != hipSuccess) return mi::hip_status(e_, #call);     \
  } while (0)

namespace mi {

constexpr int kHeadDim = 256;  // Qwen3.6 full-attention head_dim
constexpr int kGroup = 8;      // query heads per KV head (16 / 2)
constexpr float kLog2e = 1.4426950408889634f;

// Records `msg` as this thread's last error and returns `st`.
mi_status fail(mi_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a HIP error to MI_ERR_HIP (or MI_ERR_OOM) with context; MI_OK on success.
mi_status hip_status(hipError_t e, const char* what);
void clear_error();

// Checks the head shape the kernels are built for.
mi_status check_shape(int32_t H, int32_t G, int32_t D);

// Q/K head norm + RoPE host side (rope.hip).  Validates the shared
// arguments of the fused entry points.
mi_status check_rope(const mi_kv* kv, int32_t rotary_dim, float rope_theta, float eps);
// rope_theta^(-2i/rotary_dim), i < rotary_dim/2, in f32 as the reference
// writes it (src/math_util.rs:524).
void rope_inv_freq(float rope_theta, int32_t rotary_dim, float* inv_freq);

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations, not for its outstanding global loads (which __syncthreads
// would drain), then synchronises the workgroup.
__device__ __forceinline__ void sync_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The sigmoid output gate, x * sigmoid(g) = x / (1 + e^-g) (reference
// sigmoid_gate_inplace, src/math_util.rs:264-269), with the hardware base-2
// exponential and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each)
// instead of the correctly rounded library expf and an IEEE division.
// g -> -inf gives 0, g -> +inf gives x.
__device__ __forceinline__ float gate_mul(float x, float g) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// Device layout of the cache (documented in mi_attn.h), in halves.
// K: 32-row blocks; within a block, row w sits at A-operand row
// j = 4*(w/8) + w%4 of half u = (w/4)%2, so that a 16-lane group reading
// one 16-byte column chunk of 16 rows reads 256 contiguous bytes.
__host__ __device__ inline int64_t k_offset(int64_t r, int h, int i, int G, int D) {
  const int64_t b = r >> 5;
  const int w = (int)(r & 31);
  const int u = (w >> 2) & 1;
  const int j = ((w >> 3) << 2) | (w & 3);
  return (((b * G + h) * 2 + u) * (D / 8) + (i >> 3)) * 128 + j * 8 + (i & 7);
}
// V: 8-row transposed blocks, eight keys of one column contiguous.
__host__ __device__ inline int64_t v_offset(int64_t r, int h, int i, int G, int D) {
  return (((r >> 3) * G + h) * D + i) * 8 + (r & 7);
}

// Reductions across lanes that are 16 and 32 apart (the four 16-lane rows
// of a wave), with the gfx950 row-swap instructions instead of LDS
// permutes.  v_permlane16_swap exchanges rows 1 <-> 0 and 3 <-> 2 between
// its two operands, v_permlane32_swap the upper and lower halves; with both
// operands equal to x, the pair (r[0], r[1]) holds x of the two partners in
// some order, so a symmetric op of the pair is the partner reduction.
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_rows(float x) {  // max over lanes l, l^16, l^32, l^48
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_xor32(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float sum_rows(float x) {  // sum over lanes l, l^16, l^32, l^48
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return sum_xor32(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

// Raises `kernel`'s dynamic LDS limit to `bytes` on the current device, once
// per device (the attribute is held per device); `done` is the kernel's
// bitmask of devices already set.
inline mi_status set_lds_limit(const void* kernel, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  MI_HIP_RAW(hipGetDevice(&dev));
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return MI_OK;
  MI_HIP_RAW(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
  done.fetch_or(bit, std::memory_order_release);
  return MI_OK;
}

// Timing event pair for one launch when profiling is on (mi_prof_enable),
// else two nulls.
void prof_events(const char* name, hipEvent_t* start, hipEvent_t* stop);

// Launches a kernel of this library on `s`; with profiling on, the
// dispatch's begin and end times are recorded under `name`.
template <typename F, typename... Args>
hipError_t launch(const char* name, F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                  Args... args) {
  hipEvent_t a, b;
  prof_events(name, &a, &b);
  hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, a, b, 0u, args...);
  return hipGetLastError();
}

}  // namespace mi

#define MI_HIP(call)                                        \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return mi::hip_status(e_, #call); \
  } while (0)

#define MI_TRY(call)                 \
  do {                               \
    mi_status s_ = (call);           \
    if (s_ != MI_OK) return s_;      \
  } while (0)

// Internal state of an mi_kv handle (opaque to callers).
struct mi_kv {
  int32_t layers = 0, H = 0, G = 0, D = 0;
  int64_t cap = 0;  // rows, multiple of MI_KV_CAP_ALIGN
  int64_t pos = 0;  // Cache::pos
  std::vector<int64_t> len;        // FullState::len per layer
  std::vector<_Float16*> k, v;     // device buffers, cap*G*D halves each
  int device = 0;
  // Split-K decode / verify partials, grown on demand and kept for reuse.
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // A graph capture has enqueued work that uses ws.
  bool ws_captured = false;
  // State of the split kernel's in-launch merge (counters, per-XCD
  // partials; zeroed at creation, reset by the kernels themselves), and
  // whether this device dispatches workgroup b to XCD b % 8 (probed at
  // creation; the merge is used only then).
  void* mstate = nullptr;
  bool merge_ok = false;
  // Workspaces replaced by a larger one after a capture used them; freed at
  // mi_kv_destroy (graphs captured before the growth still address them).
  std::vector<void*> ws_retired;
};

namespace mi {
// A non-null handle whose device is the current one (a handle's buffers and
// launches belong to the device that was current at mi_kv_create).
mi_status check_kv(const mi_kv* kv);
// check_kv and 0 <= layer < layers.
mi_status check_layer(const mi_kv* kv, int32_t layer);
// Ensures the handle's workspace holds at least `bytes` (synchronous grow;
// refused while `stream` is capturing a graph).
mi_status kv_workspace(mi_kv* kv, size_t bytes, hipStream_t stream, void** ws);
// Grows the cache to at least `rows` rows (mi_kv_reserve), refused while
// `stream` is capturing a graph.
mi_status kv_grow(mi_kv* kv, int64_t rows, hipStream_t stream);
// Bytes of mi_kv::mstate for G KV heads (decode.hip).
size_t merge_state_bytes(int G);
// Whether workgroup b of a launch runs on XCD b % 8 on the current device,
// checked once per device with a probe kernel (decode.hip).
bool xcd_round_robin();
// The wide verify's split pass (prefill.hip): the 64-query prefill body in
// its split-K form over `nchunks` chunks of `chunk` keys (a multiple of 64)
// of rows [0, past + n) of `layer`, for the n query tokens q [n][H][D] in
// row blocks of 16 tokens; writes the unnormalised partials part_o
// [G][nchunks][8 n][D] and part_ml [G][nchunks][8 n][2] that
// attn_combine_kernel merges.
mi_status verify_wide_split(const mi_kv* kv, int32_t layer, const _Float16* q, int64_t past,
                            int32_t n, int64_t chunk, int32_t nchunks, float* part_o,
                            float* part_ml, hipStream_t stream);
// Causal attention of n query tokens over rows [0, past + n) of `layer`
// (already in the cache) through the wide verify: the split pass above and
// the merge (decode.hip).  out [n][H][D], optional gate [n][H][D].
mi_status attend_wide(mi_kv* kv, int32_t layer, const _Float16* q, const _Float16* gate,
                      _Float16* out, int64_t past, int32_t n, hipStream_t stream);
// Workspace bytes attend_wide needs for these sizes.
size_t wide_workspace_bytes(int G, int64_t past, int32_t n);
// Enqueues the row copy of kv_cache_append_n on `stream` (no len update).
mi_status kv_append_rows(mi_kv* kv, int32_t layer, const _Float16* k,
                         const _Float16* v, int64_t pos, int32_t n,
                         hipStream_t stream);
}  // namespace mi
