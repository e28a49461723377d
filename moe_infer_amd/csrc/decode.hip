// Split-K flash-decoding over the f16 KV cache, for one query token (decode),
// a few query tokens with a causal tail (speculative verify), or a ragged
// batch of independent sequences.
//
// Reference semantics: attention_scores/softmax/values_batched and
// sigmoid_gate_inplace (src/math_util.rs:264-269, 323-383); the split-K
// kernels attn_sdpa_block / attn_sdpa_reduce (src/engine/shaders.metal:
// 1559-1776) dispatched by encode_pre_expert_full (src/engine/qwen35_moe/
// fused_exp2.rs:683-719); the causal bound of attn_sdpa_causal_n
// (shaders.metal:2675-2676: query i sees rows [0, past_pos + i]).
//
// Design (gfx950, wave64):
//  * One workgroup = one (sequence, KV head, chunk of keys).  The eight query
//    heads of the GQA group — times the query tokens for verify — are the
//    columns of one MFMA tile, so each K/V byte is read from HBM once per
//    group rather than once per query head.
//  * S^T = K . Q^T with v_mfma_f32_16x16x32_f16: K rows are the A operand,
//    loaded straight from HBM as 128-bit vectors (each lane streams 128
//    contiguous bytes of one key row); Q^T stays in registers.
//  * O^T += V^T . P^T with the same instruction: the V cache is stored in
//    8-row transposed blocks, so the A operand (eight keys of one value
//    column) is one 128-bit load, and the P^T operand is the S^T
//    accumulator of the same lane (the QK row order is chosen so that it
//    is) — no LDS transpose, no shuffles of P.
//  * Online softmax in base 2 per column; the column max / sum reductions
//    are two cross-lane xor steps (lanes 16 and 32 apart).
//  * The waves of a workgroup merge their (m, l, O) through LDS and write one
//    partial per chunk; attn_combine_kernel merges the chunks, normalises,
//    applies the sigmoid gate and writes f16.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "plan.h"

namespace {

constexpr int D = mi::kHeadDim;
constexpr float kNegBig = -1e30f;

// Most sequences of a ragged batch whose tile offsets the flat split
// computes itself (no plan launch); larger batches run ragged_plan_kernel.
constexpr int kFusedPlan = 256;

struct SplitArgs {
  const _Float16* k;        // K 32-row blocks (mi::k_offset)
  const _Float16* v;        // V blocks, (r,h,i) at v + ((r/8)*G + h)*D*8 + i*8 + r%8
  const int32_t* offsets;   // ragged: first row of sequence s (else null)
  const int32_t* lengths;   // ragged: rows of sequence s (else null)
  int64_t kv_len;           // non-ragged: rows the launch may read
  int64_t lim0;             // non-ragged: rows visible to query token 0
  const _Float16* q;        // [batch][nq][H][D]
  float* part_o;            // [G][nslots][ncols][D], slot = s * max_chunks + chunk
  float* part_ml;           // [G][nslots][ncols][2]  (flat ragged: slot = workgroup + s)
  int64_t nslots;
  int G, H, nq, chunk, max_chunks;
  float scale_log2e;
  // Flat ragged split: tile_off[s] = 32-key tiles of sequences 0..s-1
  // (invalid descriptors count 0), tile_off[batch] = all tiles T; workgroup
  // x < nw = min(gridDim.x, T) takes tiles [x T / nw, (x+1) T / nw) of the
  // concatenation and writes one partial per sequence it touches, in slot
  // x + s.  Null otherwise.
  const int32_t* tile_off;
  // Flat split of up to kFusedPlan sequences: no plan kernel; every
  // workgroup computes the tile offsets into LDS from lengths / offsets, and
  // workgroup (0, 0) also stores them here (= tile_off) for the merge kernel.
  // Null otherwise.
  int32_t* tile_off_out;
  int batch;
  // Optional fused append (decode step, verify): rows [app0, app0 + app_n)
  // of the cache are written from app_k / app_v ([app_n][G*D] token-major)
  // by the workgroup whose key chunk holds them, before it reads them.
  const _Float16* app_k;
  const _Float16* app_v;
  _Float16* kw;
  _Float16* vw;
  int64_t app0;
  int app_n;
  // In-launch merge (single sequence, one query token, one KV head per
  // workgroup): partials m / l at part_ml with a 256-byte stride per slot,
  // then merged inside the launch (merge_tail) and written to out with the
  // gate, instead of by attn_combine_kernel.  Null mcnt: off.
  int* mcnt;          // counters: XCD-local [G][8], then per KV head [G] (256 B apart)
  float* xo;          // per-XCD partials [G][8][8][D]
  float* xml;         // per-XCD (m, l) [G][8][64]
  const _Float16* gate;
  const float* gate32;
  _Float16* out;
};

// Partials are consumed once, by the combine kernel, on any XCD: written
// through to memory (sc0 sc1), so that the end of the split launch has no
// dirty partial lines to write back from the L2s.  Measured at C2 against
// streaming (nontemporal) and default stores, in one process: 19.87-19.91
// against 20.12-20.15 us per step.
__device__ __forceinline__ void store_part(float v, float* p) {
  asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
// A store of more than 64 bits reads its data registers after issue: the
// next instruction may not overwrite them without wait states, which the
// compiler inserts for its own stores but not for asm ones, hence the nops.
__device__ __forceinline__ void store_part(f32x4 v, f32x4* p) {
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n s_nop 1" ::"v"(p), "v"(v) : "memory");
}

// 16-byte streaming load of K/V: read once per launch, so it is not kept in
// the caches (MI_ATTN_TEMPORAL_KV=1 at build time keeps the default policy).
__device__ __forceinline__ f16x8 load16(const _Float16* p) {
#if defined(MI_ATTN_TEMPORAL_KV)
  return *(const f16x8*)p;
#else
  return __builtin_nontemporal_load((const f16x8*)p);
#endif
}

// Fused projection input of the decode step (mi_attn_step_proj): the raw
// q_proj / k / v of one token in f32, normed and rotated inside the split
// kernel.  cos / sin of the rotation angles pos * inv_freq[i] are computed on
// the host (the position is a host value), in f32 like the reference:
// cs[i] = cos, cs[rot_half + i] = sin, i < rot_half.
struct ProjArgs {
  const float* q_proj;  // [H][2*D]: query then gate of each head
  const float* k;       // [G][D]
  const float* v;       // [G][D]
  const uint16_t* q_w;  // bf16 [D]
  const uint16_t* k_w;  // bf16 [D]
  int rot_half;          // host side: selects the Proj<rot_half / 32> kernel
  float eps;
  float cs[MI_ROPE_MAX_DIM];
};
struct NoProj {
  static constexpr int kSH = 0;
};
// ProjArgs with the rotation width as a compile-time constant:
// rot_half = 32 * SH, SH = 0 .. 4.
template <int SH>
struct Proj : ProjArgs {
  static constexpr int kSH = SH;
};
template <class X>
struct is_proj : std::false_type {};
template <int SH>
struct is_proj<Proj<SH>> : std::true_type {};

// The 64*SH cos/sin values spread over the wave: entry 64s + lane in tab[s],
// filled from uniform (scalar) kernel-argument reads.
template <int SH>
struct RopeTab {
  float t[SH > 0 ? SH : 1];
  __device__ __forceinline__ void fill(const ProjArgs& x, int lane) {
#pragma unroll
    for (int s = 0; s < SH; s++) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < 64; k++) v = lane == k ? x.cs[64 * s + k] : v;
      t[s] = v;
    }
  }
  // Entry idx (any lane), read with a cross-lane permute.
  __device__ __forceinline__ float get(int idx) const {
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < SH; s++) {
      const float u = __shfl(t[s], idx & 63, 64);
      v = (idx >> 6) == s ? u : v;
    }
    return v;
  }
};

// Per-head RMS norm + NeoX rotation, one head per TPH = 256 / DPT adjacent
// lanes (aligned within the wave): lane index i = lane % TPH holds columns
// DPT*i .. DPT*i + DPT-1 of the head.  The rotation partner of column
// d < rot_half, d + rot_half, sits rot_half / DPT lanes up.  Split into the
// loads (issued early, ahead of the first K/V tile, so that waiting for
// them does not wait for the tile) and the arithmetic.
template <int DPT>
struct HeadPart {
  float y[DPT];
  uint32_t wb[DPT / 2];  // bf16 pairs
  __device__ __forceinline__ void load(const float* src, const uint16_t* w, int lane) {
    const int i = lane % (D / DPT);
#pragma unroll
    for (int e = 0; e < DPT; e += 4) {
      const float4 f = *(const float4*)(src + DPT * i + e);
      y[e] = f.x;
      y[e + 1] = f.y;
      y[e + 2] = f.z;
      y[e + 3] = f.w;
      const uint2 u = *(const uint2*)(w + DPT * i + e);
      wb[e / 2] = u.x;
      wb[e / 2 + 1] = u.y;
    }
  }
  template <int SH>
  __device__ __forceinline__ void norm_rope(const ProjArgs& x, const RopeTab<SH>& tab, int lane) {
    constexpr int TPH = D / DPT;
    const int i = lane % TPH;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; e++) ss += y[e] * y[e];
#pragma unroll
    for (int m = 1; m < TPH; m <<= 1) ss += __shfl_xor(ss, m, 64);
    const float inv_rms = 1.0f / sqrtf(ss / (float)D + x.eps);
#pragma unroll
    for (int e = 0; e < DPT; e++)
      y[e] = y[e] * inv_rms * mi::bf16_to_f32((uint16_t)(wb[e / 2] >> (16 * (e & 1))));
    if constexpr (SH > 0) {
      constexpr int RH = 32 * SH;
      const int d0 = DPT * i;
      const bool lower = d0 < RH;
      const int partner = lower ? lane + RH / DPT : lane - RH / DPT;
      float pr[DPT];
#pragma unroll
      for (int e = 0; e < DPT; e++) pr[e] = __shfl(y[e], partner & 63, 64);
      const int p0 = lower ? d0 : d0 - RH;
#pragma unroll
      for (int e = 0; e < DPT; e++) {
        const float c = tab.get(p0 + e), sn = tab.get(RH + p0 + e);
        if (d0 < 2 * RH) y[e] = lower ? y[e] * c - pr[e] * sn : pr[e] * sn + y[e] * c;
      }
    }
  }
};

// ---- in-launch merge of the chunk partials (decode of one sequence, one
// query token, one KV head per workgroup).  Workgroup b of the launch runs on
// XCD b % 8 (round-robin dispatch; checked per device when a handle is
// created, else the merge is not used).  The partials of the chunks of one
// KV head whose workgroups share an XCD are merged by the last of them to
// arrive (an XCD-local counter: stores and atomics meet in that XCD's L2,
// so no cache write-back is needed); it writes one partial per XCD through
// to memory, and the last of those (a device-scope counter) merges the
// eight, normalises, applies the gate and writes the output.  Every counter
// is reset by its last user, so the launch can be replayed in a graph.
// Off by default (decode_merge_enabled): in a probe of the protocol alone it
// added 1.9 us to a launch of 256 workgroups, but after a real C2 split the
// chain takes ~5 us, as long as the combine launch.

// Loads the compiler tracks (it places the waits itself: an asm load whose
// result the compiler copied before a separate wait would copy stale
// data).  Within the XCD a plain load: it misses this CU's L1 (which never
// held those lines in this launch; L1 is invalidated at every kernel start)
// and hits the XCD's L2, where the members' stores landed; the barrier
// before the loads keeps them after the arrival count.  Across XCDs,
// system-scope atomic loads (sc0 sc1: past this XCD's L2, from memory, where
// the data was written through).
__device__ __forceinline__ f32x4 ld_xcd4(const float* p) { return *(const f32x4*)p; }
__device__ __forceinline__ float ld_xcd1(const float* p) { return *p; }
__device__ __forceinline__ float ld_dev1(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ f32x4 ld_dev4(const float* p) {
  return f32x4{ld_dev1(p), ld_dev1(p + 1), ld_dev1(p + 2), ld_dev1(p + 3)};
}
__device__ __forceinline__ void st_dev4(float* p, f32x4 v) {  // written through to memory
  // (the nops: as for store_part, the data registers are read after issue)
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n s_nop 1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_dev1(float* p, float v) {
  asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
constexpr int kMergeStride = 64;  // ints between counters (256 bytes)

template <int NT>
__device__ void merge_tail(const SplitArgs& a) {
  static_assert(NT == 512, "one f32x4 of the 8 x 256 outputs per thread");
  const int t = threadIdx.x;
  const int hy = blockIdx.y;  // KV head
  const int mc = a.max_chunks;
  const int x = (blockIdx.x + mc * hy) & 7;  // this workgroup's XCD
  const int ngroups = mc < 8 ? mc : 8;
  // chunks c of this head on XCD x: c = first(x) + 8 j
  auto first_of = [&](int xx) { return ((xx - mc * hy) % 8 + 8) % 8; };
  const int first = first_of(x);
  const int nmem = first < mc ? (mc - first + 7) / 8 : 0;
  const int col = t >> 6, d4 = (t & 63) * 4;  // output column (query head) and values
  __shared__ int s_last;

  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have reached L2
  __syncthreads();
  if (t == 0)
    s_last = __hip_atomic_fetch_add(a.mcnt + (hy * 8 + x) * kMergeStride, 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_WORKGROUP) == nmem - 1;
  __syncthreads();
  if (!s_last) return;

  // XCD level: online merge of the members' (m, l, o), 16 at a time
  float M = kNegBig, L = 0.f;
  f32x4 O = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < nmem; j0 += 16) {
    f32x4 o[16];
    float m[16], l[16];
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const int c = first + 8 * (j0 + u < nmem ? j0 + u : j0);
      const int64_t slot = (int64_t)hy * a.nslots + c;
      o[u] = ld_xcd4(a.part_o + (slot * 8 + col) * D + d4);
      m[u] = ld_xcd1(a.part_ml + slot * 64 + 2 * col);
      l[u] = ld_xcd1(a.part_ml + slot * 64 + 2 * col + 1);
    }
    float mb = M;
#pragma unroll
    for (int u = 0; u < 16; u++)
      if (j0 + u < nmem) mb = fmaxf(mb, m[u]);
    const float r = exp2f(M - mb);
    L *= r;
    O *= r;
#pragma unroll
    for (int u = 0; u < 16; u++)
      if (j0 + u < nmem) {
        const float w = exp2f(m[u] - mb);
        L += l[u] * w;
        O += o[u] * w;
      }
    M = mb;
  }
  st_dev4(a.xo + ((hy * 8 + x) * 8 + col) * D + d4, O);
  if (d4 == 0) {
    st_dev1(a.xml + (hy * 8 + x) * 64 + 2 * col, M);
    st_dev1(a.xml + (hy * 8 + x) * 64 + 2 * col + 1, L);
  }
  __builtin_amdgcn_s_waitcnt(0);  // written through before the arrival is counted
  __syncthreads();
  if (t == 0) {
    __hip_atomic_store(a.mcnt + (hy * 8 + x) * kMergeStride, 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
    int* dc = a.mcnt + (a.G * 8 + hy) * kMergeStride;
    const bool last = __hip_atomic_fetch_add(dc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      ngroups - 1;
    if (last) __hip_atomic_store(dc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;

  // head level: the XCDs that hold chunks of this head
  f32x4 o[8];
  float m[8], l[8];
#pragma unroll
  for (int xx = 0; xx < 8; xx++) {
    o[xx] = ld_dev4(a.xo + ((hy * 8 + xx) * 8 + col) * D + d4);
    m[xx] = ld_dev1(a.xml + (hy * 8 + xx) * 64 + 2 * col);
    l[xx] = ld_dev1(a.xml + (hy * 8 + xx) * 64 + 2 * col + 1);
  }
  float Mh = kNegBig;
#pragma unroll
  for (int xx = 0; xx < 8; xx++)
    if (first_of(xx) < mc) Mh = fmaxf(Mh, m[xx]);
  float Lh = 0.f;
  f32x4 Oh = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int xx = 0; xx < 8; xx++)
    if (first_of(xx) < mc) {
      const float w = exp2f(m[xx] - Mh);
      Lh += l[xx] * w;
      Oh += o[xx] * w;
    }
  // out = O / L (zero when L = 0, math_util.rs:357, 372), then the gate
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  const int hq = hy * 8 + col;
  f16x4 h;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float r = Oh[e] * inv;
    if (a.gate) r = mi::gate_mul(r, (float)a.gate[hq * D + d4 + e]);
    else if (a.gate32) r = mi::gate_mul(r, a.gate32[hq * (2 * D) + D + d4 + e]);
    h[e] = (_Float16)r;
  }
  *(f16x4*)(a.out + hq * D + d4) = h;
}

// Workgroup = GH KV heads x NWH waves per head, over one chunk of keys of one
// sequence (with GH = 2 a workgroup reads one contiguous stretch of both
// heads' K and V blocks).  NCB column blocks of 16 columns (column c = token
// c / 8, query head c % 8 of the group).
// With X = ProjArgs (decode step from projections, one token, NCB = 1) the
// kernel also norms and rotates Q per wave, and the workgroup holding row
// app0 norms, rotates and appends K and appends V.
template <int NWH, int NCB, int GH, typename X, bool FLAT>
__global__ void __launch_bounds__(NWH * GH * 64)
attn_split_kernel(SplitArgs a, X x) {
  constexpr bool kProj = is_proj<X>::value;
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int hw = wv / NWH;   // KV head of this wave within the workgroup
  const int w = wv % NWH;    // wave within the head
  const int g = lane >> 4;   // lane group: k-slot group of the MFMA operands
  const int j = lane & 15;   // column within a column block / A-operand row
  const int chunk_idx = blockIdx.x;
  const int kvh = blockIdx.y * GH + hw;
  int s = blockIdx.z;
  const int G = a.G;
  const int ncols = a.nq * 8;

  constexpr bool flat = FLAT;  // the flat ragged split (a.tile_off)
  int64_t len = 0, row0 = 0, lim0 = 0, key_begin = 0, key_end = 0;
  int64_t t_lo = 0, t_hi = 0;  // flat: this workgroup's tiles of the concatenation
  // flat: the tile offsets, from the plan kernel's table or computed below
  int32_t* const ltoff = (int32_t*)(smem + GH * (NWH * ncols * (D + 4) + 2 * NWH * ncols));
  auto toff = [&](int i) -> int64_t {  // tile_off[i], i wave-uniform in [0, batch]
    return __builtin_amdgcn_readfirstlane(a.tile_off_out ? ltoff[i] : a.tile_off[i]);
  };
  if constexpr (flat) {
    if (a.tile_off_out) {  // uniform
      // Wave 0 scans the tile counts (an invalid descriptor counts 0) of up
      // to kFusedPlan sequences, 64 per step, into LDS; workgroup (0, 0)
      // also stores them for the merge kernel.
      if (wv == 0) {
        int32_t n[kFusedPlan / 64];
#pragma unroll
        for (int c = 0; c < kFusedPlan / 64; c++) {
          const int i = 64 * c + lane;
          n[c] = 0;
          if (i < a.batch) {
            const int32_t len = a.lengths[i], off = a.offsets[i];
            const bool bad = len < 0 || len > a.kv_len || off < 0 || (off & 31);
            n[c] = bad ? 0 : (len + 31) >> 5;
          }
        }
        const bool store = blockIdx.x == 0 && blockIdx.y == 0;
        int32_t carry = 0;
#pragma unroll
        for (int c = 0; c < kFusedPlan / 64; c++) {
          int32_t inc = n[c];
#pragma unroll
          for (int d = 1; d < 64; d <<= 1) {
            const int32_t y = __shfl_up(inc, d, 64);
            if (lane >= d) inc += y;
          }
          const int i = 64 * c + lane;
          if (i < a.batch) {
            ltoff[i] = carry + inc - n[c];
            if (store) a.tile_off_out[i] = carry + inc - n[c];
          }
          carry += __shfl(inc, 63, 64);
        }
        if (lane == 0) {
          ltoff[a.batch] = carry;
          if (store) a.tile_off_out[a.batch] = carry;
        }
      }
      __syncthreads();
    }
    // min(gridDim.x, T) workgroups take the tiles, each at least one
    // (uniform values: kept in scalar registers)
    const int64_t total = toff(a.batch);
    const int64_t nw = min((int64_t)gridDim.x, total);
    if (chunk_idx >= nw) return;  // uniform
    t_lo = (int64_t)chunk_idx * total / nw;
    t_hi = (int64_t)(chunk_idx + 1) * total / nw;
    // the sequence holding tile t_lo: the last s with tile_off[s] <= t_lo
    int lo = 0, hi = a.batch - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (toff(mid) <= t_lo) lo = mid;
      else hi = mid - 1;
    }
    s = lo;
  } else if (a.lengths) {
    len = a.lengths[s];
    row0 = a.offsets[s];
    lim0 = len;
    // invalid descriptors are reported as NaN by the combine kernel
    if (len < 0 || len > a.kv_len || row0 < 0 || (row0 & 31)) return;
  } else {
    len = a.kv_len;
    row0 = 0;
    lim0 = a.lim0;
  }
  if constexpr (!flat) {
    key_begin = (int64_t)chunk_idx * a.chunk;
    // uniform over the workgroup; with the in-launch merge every workgroup
    // takes part (an empty chunk leaves an empty partial)
    if (key_begin >= len && !a.mcnt) return;
    key_end = min(key_begin + (int64_t)a.chunk, len);
  }

  // K operand rows: tile u, A-row j <-> key k0 + 8*(j/4) + 4u + j%4, so that
  // accumulator row 4g+e of tile u is key k0 + 8g + 4u + e.  In the 32-row
  // block layout this operand (chunk 4kk + g of row j, half u) is one
  // 16-byte vector, and the 16 lanes of a group read 256 contiguous bytes.
  // Whole 32-key tiles always lie inside the allocation (cache capacities
  // are multiples of 256 rows; ragged sequences own whole 32-row blocks),
  // so the loads are unconditional and straight-line.  Keys past key_end
  // are masked out of the scores below; their V values are zeroed because
  // stale rows may hold anything (NaN included) and 0 * NaN is NaN.
  // V operand: lane (g, j), value block dblk holds V^T[dblk*16 + j][keys
  // k0+8g .. k0+8g+7] = one 16-byte vector of the block layout.
  auto load_k = [&](int64_t k0, f16x8(&kf)[2][8]) {
    const _Float16* kp =
        a.k + (((row0 + k0) >> 5) * G + kvh) * (int64_t)(32 * D) + g * 128 + j * 8;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int kk = 0; kk < 8; kk++) kf[u][kk] = load16(kp + u * (16 * D) + kk * 512);
  };
  auto load_v = [&](int64_t k0, f16x8(&vf)[16]) {
    const _Float16* vp =
        a.v + (((row0 + k0) >> 3) + g) * G * (int64_t)(D * 8) + kvh * (D * 8) + j * 8;
#pragma unroll
    for (int dblk = 0; dblk < 16; dblk++) vf[dblk] = load16(vp + dblk * 128);
  };
  // LDS: per KV head of the workgroup the merge area (below); with the
  // projection prologue then the normed, rotated f16 query rows of the
  // workgroup's GH*8 heads.
  constexpr int kLdsRow = D + 4;
  constexpr int kQRow = D + 8;
  const int per_head = NWH * ncols * kLdsRow + 2 * NWH * ncols;
  _Float16* qs = (_Float16*)(smem + GH * per_head);  // [GH*8][kQRow]
  // Projection prologue, issue side: this lane's part of the q_proj rows
  // (one query head per kTPH lanes of the workgroup).  The first K/V tile is
  // loaded in the tile loop, after the prologue: issuing it here keeps 128
  // registers live through the norm and rotation, which spills (measured
  // 2 us slower per step).
  constexpr int kTPH = NWH * 8;
  RopeTab<X::kSH> tab;
  HeadPart<kProj ? D / kTPH : 4> qpart;
  f16x8 kf[2][8], vf[16];
  if constexpr (kProj) {
    qpart.load(x.q_proj + ((int64_t)blockIdx.y * GH * 8 + threadIdx.x / kTPH) * (2 * D), x.q_w,
               lane);
    tab.fill(x, lane);
  }

  if constexpr (kProj) {
    const int64_t r = a.app0;
    if (key_begin <= r && r < key_end) {  // workgroup-uniform
      const int h0 = blockIdx.y * GH;
      constexpr int TPH = NWH * 8, DPT = D / TPH;
      if ((int)threadIdx.x < GH * TPH) {  // whole waves
        // K head h0 + t / TPH, columns DPT * (t % TPH) ...
        const int hk = threadIdx.x / TPH;
        HeadPart<DPT> kp;
        kp.load(x.k + (h0 + hk) * D, x.k_w, lane);
        kp.template norm_rope<X::kSH>(x, tab, lane);
        const float(&y)[DPT] = kp.y;
        if constexpr (DPT == 8) {
          f16x8 h;
#pragma unroll
          for (int e = 0; e < 8; e++) h[e] = (_Float16)y[e];
          *(f16x8*)(a.kw + mi::k_offset(r, h0 + hk, DPT * (lane % TPH), G, D)) = h;
        } else {
          f16x4 h;
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = (_Float16)y[e];
          *(f16x4*)(a.kw + mi::k_offset(r, h0 + hk, DPT * (lane % TPH), G, D)) = h;
        }
      }
      for (int it = threadIdx.x; it < GH * D; it += NWH * GH * 64) {
        const int hh = it / D, i = it % D;
        a.vw[mi::v_offset(r, h0 + hh, i, G, D)] = (_Float16)x.v[(h0 + hh) * D + i];
      }
      __syncthreads();  // the row is in L2 before any wave of this group reads it
    }
  } else if (a.app_n > 0) {
    // Fused append of the new rows that fall in this chunk, for this
    // workgroup's GH heads; nothing else reads them in this launch.
    const int64_t r_lo = max(key_begin, a.app0);
    const int64_t r_hi = min(key_end, a.app0 + a.app_n);
    if (r_lo < r_hi) {  // workgroup-uniform
      const int nrow = (int)(r_hi - r_lo);
      const int h0 = blockIdx.y * GH;
      for (int it = threadIdx.x; it < nrow * GH * (D / 8); it += NWH * GH * 64) {
        const int rr = it / (GH * (D / 8)), hh = (it / (D / 8)) % GH, c = it % (D / 8);
        const int64_t r = r_lo + rr;
        *(f16x8*)(a.kw + mi::k_offset(r, h0 + hh, 8 * c, G, D)) =
            *(const f16x8*)(a.app_k + (r - a.app0) * G * D + (h0 + hh) * D + 8 * c);
      }
      for (int it = threadIdx.x; it < nrow * GH * D; it += NWH * GH * 64) {
        const int rr = it / (GH * D), hh = (it / D) % GH, i = it % D;
        const int64_t r = r_lo + rr;
        a.vw[mi::v_offset(r, h0 + hh, i, G, D)] = a.app_v[(r - a.app0) * G * D + (h0 + hh) * D + i];
      }
      __syncthreads();  // the rows are in L2 before any wave of this group reads them
    }
  }


  // One pass per key range: once, or per sequence segment of a flat range.
  for (;;) {
  int64_t pslot = (int64_t)s * a.max_chunks + chunk_idx;  // partial slot
  if constexpr (flat) {
    const int64_t ps = toff(s);
    const int64_t pe = toff(s + 1);
    len = __builtin_amdgcn_readfirstlane(a.lengths[s]);
    row0 = __builtin_amdgcn_readfirstlane(a.offsets[s]);
    lim0 = len;
    key_begin = 32 * (max(t_lo, ps) - ps);
    key_end = min(32 * (min(t_hi, pe) - ps), len);
    pslot = (int64_t)chunk_idx + s;
  }

  // Q^T operand: lane (g, j) holds q[token][head][32kk + 8g + 0..7] for its
  // column j, kk = 0..7 (the column chunk 4kk + g the K operand of the same
  // lane holds).  Padding columns are zero and fully masked.
  f16x8 qf[NCB][8];
  int64_t lim[NCB];
  if constexpr (kProj) {
    static_assert(NCB == 1, "projection input is one query token");
    // Cooperative norm + rotation of the workgroup's GH*8 query heads, one
    // head per kTPH lanes; the result goes to LDS as f16 and comes back as
    // this lane's Q^T operand (column j < 8 = query head kvh*8 + j).
    {
      constexpr int DPT = D / kTPH;
      const int hl = threadIdx.x / kTPH;
      qpart.template norm_rope<X::kSH>(x, tab, lane);
      _Float16* dst = qs + hl * kQRow + DPT * (lane % kTPH);
      if constexpr (DPT == 8) {
        f16x8 h;
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = (_Float16)qpart.y[e];
        *(f16x8*)dst = h;
      } else {
        f16x4 h;
#pragma unroll
        for (int e = 0; e < 4; e++) h[e] = (_Float16)qpart.y[e];
        *(f16x4*)dst = h;
      }
    }
    mi::sync_lds();
    const bool col = j < 8;
    const _Float16* qrow = qs + (hw * 8 + (j & 7)) * kQRow + 8 * g;
#pragma unroll
    for (int kk = 0; kk < 8; kk++) qf[0][kk] = col ? *(const f16x8*)(qrow + 32 * kk) : f16x8{};
    lim[0] = col ? a.lim0 : 0;
  } else {
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) {
    const int c = cb * 16 + j;
    const int tok = c >> 3;
    if (c < ncols) {
      const _Float16* qp =
          a.q + (((int64_t)s * a.nq + tok) * a.H + kvh * 8 + (c & 7)) * D + 8 * g;
#pragma unroll
      for (int kk = 0; kk < 8; kk++) qf[cb][kk] = *(const f16x8*)(qp + 32 * kk);
      lim[cb] = lim0 + tok;
    } else {
#pragma unroll
      for (int kk = 0; kk < 8; kk++) qf[cb][kk] = f16x8{};
      lim[cb] = 0;
    }
  }
  }

  float m[NCB], l[NCB];
  f32x4 acc[NCB][16];
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) {
    m[cb] = kNegBig;
    l[cb] = 0.f;
#pragma unroll
    for (int d = 0; d < 16; d++) acc[cb][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // V rows of the last, partial tile past key_end are zeroed (a
  // wave-uniform branch).  The flat ragged split meets such a tile at the
  // end of every sequence segment, so there the zeroing (which waits for the
  // V loads) comes after the QK MFMAs: C3 312 against 323 us.  For single
  // sequences it stays ahead of them: a build with it after them for every
  // kernel took 15.6 against 14.6 us per C2 split launch.
  auto zero_v_tail = [&](int64_t k0) {
    const int64_t valid = key_end - (k0 + 8 * g);
#pragma unroll
    for (int dblk = 0; dblk < 16; dblk++)
#pragma unroll
      for (int e = 0; e < 8; e++)
        if (e >= valid) vf[dblk][e] = (_Float16)0.f;
  };
  // Wave w of the head takes a contiguous run of the range's 32-key tiles
  // (ceil(tiles / NWH) each).  Against tiles dealt round-robin this took the
  // C2 split from 14.6 to 14.2 us (one tile per wave either way: the loop
  // the compiler makes is what differs); verify and the ragged batch are
  // unchanged.
  const mi::WaveTiles wt = mi::split_wave_tiles(key_begin, key_end, NWH, w);
  for (int64_t k0 = wt.first; k0 < wt.last; k0 += 32) {
    load_k(k0, kf);
    load_v(k0, vf);
    if (!flat && k0 + 32 > key_end) zero_v_tail(k0);

#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      f32x4 st[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        f32x4 c4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 8; kk++)
          c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[u][kk], qf[cb][kk], c4, 0, 0, 0);
        st[u] = c4;
      }
      if (flat && cb == 0 && k0 + 32 > key_end) zero_v_tail(k0);
      // scale into base 2 and mask keys outside this column's window
      float mt = kNegBig;
#pragma unroll
      for (int u = 0; u < 2; u++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int64_t key = k0 + 8 * g + 4 * u + e;
          float sv = st[u][e] * a.scale_log2e;
          sv = (key < lim[cb] && key < key_end) ? sv : -INFINITY;
          st[u][e] = sv;
          mt = fmaxf(mt, sv);
        }
      mt = mi::max_rows(mt);
      const float mnew = fmaxf(m[cb], mt);
      const float alpha = exp2f(m[cb] - mnew);
      float rs = 0.f;
      f16x8 pf;
#pragma unroll
      for (int u = 0; u < 2; u++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          // The row sum adds the f16 weights the PV MFMA uses, so that the
          // normalised weights sum to one.
          const _Float16 ph = (_Float16)exp2f(st[u][e] - mnew);
          rs += (float)ph;
          pf[4 * u + e] = ph;
        }
      rs = mi::sum_rows(rs);
      l[cb] = l[cb] * alpha + rs;
      m[cb] = mnew;
#pragma unroll
      for (int dblk = 0; dblk < 16; dblk++) {
        acc[cb][dblk] *= alpha;
        acc[cb][dblk] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dblk], pf, acc[cb][dblk], 0, 0, 0);
      }
    }
  }

  // ---- merge the NWH waves of each head through LDS.  Per head:
  // O [NWH][ncols][kLdsRow] (row padded by 4 floats so the 16 columns a
  // lane group writes fall in distinct banks), then m, l [NWH][ncols].
  float* so = smem + hw * per_head;
  float* sm = so + NWH * ncols * kLdsRow;
  float* sl = sm + NWH * ncols;
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) {
    const int c = cb * 16 + j;
    if (c < ncols) {
      float* dst = so + (w * ncols + c) * kLdsRow + 4 * g;
#pragma unroll
      for (int dblk = 0; dblk < 16; dblk++) *(f32x4*)(dst + dblk * 16) = acc[cb][dblk];
      if (g == 0) {
        sm[w * ncols + c] = m[cb];
        sl[w * ncols + c] = l[cb];
      }
    }
  }
  __syncthreads();
  // merged O, four columns of d per thread; each thread derives its column's
  // merge weights 2^(m_w - M) from the NWH waves' (m, l) itself (four
  // exponentials), which saves a barrier on the kernel's critical path; the
  // threads of d4 = 0 also store the merged (M, L).
  for (int idx = threadIdx.x; idx < GH * ncols * (D / 4); idx += NWH * GH * 64) {
    const int h2 = idx / (ncols * (D / 4));
    const int c = (idx / (D / 4)) % ncols;
    const int d4 = (idx % (D / 4)) * 4;
    const float* so2 = smem + h2 * per_head;
    const float* sm2 = so2 + NWH * ncols * kLdsRow;
    const float* sl2 = sm2 + NWH * ncols;
    float M = kNegBig;
#pragma unroll
    for (int ww = 0; ww < NWH; ww++) M = fmaxf(M, sm2[ww * ncols + c]);
    float L = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < NWH; ww++) {
      const float sc = exp2f(sm2[ww * ncols + c] - M);
      L += sl2[ww * ncols + c] * sc;
      o += *(const f32x4*)(so2 + (ww * ncols + c) * kLdsRow + d4) * sc;
    }
    const int64_t pb = ((int64_t)(blockIdx.y * GH + h2) * a.nslots + pslot) * ncols + c;
    if (!flat && a.mcnt) {
      // plain stores: the merging workgroup reads them from this XCD's L2
      if (d4 == 0) {
        float* ml = a.part_ml + ((int64_t)(blockIdx.y * GH + h2) * a.nslots + pslot) * 64 + 2 * c;
        ml[0] = M;
        ml[1] = L;
      }
      *(f32x4*)(a.part_o + pb * D + d4) = o;
    } else {
      if (d4 == 0) {
        store_part(M, a.part_ml + pb * 2 + 0);
        store_part(L, a.part_ml + pb * 2 + 1);
      }
      store_part(o, (f32x4*)(a.part_o + pb * D + d4));
    }
  }
  if constexpr (!flat) {
    if constexpr (NWH * GH == 8 && NCB == 1) {  // the forms the host merges in-launch
      if (a.mcnt) merge_tail<NWH * GH * 64>(a);
    }
    break;
  }
  if (toff(s + 1) >= t_hi) break;
  // next sequence with tiles (the range ends inside a later one)
  do s++;
  while (toff(s + 1) == toff(s));
  __syncthreads();  // the LDS merge area is reused
  }
}

struct CombineArgs {
  const int32_t* offsets;  // ragged (else null)
  const int32_t* lengths;  // ragged (else null)
  int64_t kv_len;          // rows (ragged: max_len)
  const float* part_o;
  const float* part_ml;
  const _Float16* gate;    // [batch][nq][H][D] or null
  const float* gate32;     // or the gate halves of q_proj [nq][H][2*D] (else null)
  _Float16* out;           // [batch][nq][H][D]
  int G, H, nq, chunk, max_chunks;
  const int32_t* tile_off;  // flat ragged split (SplitArgs::tile_off), else null
  int nwg, batch;           // flat: the split launch's gridDim.x; sequences
  int64_t nslots;           // partial slots per KV head (SplitArgs::nslots)
};

// Chunk merge.  One workgroup per (column, KV head x slice of S values of
// d, sequence), 256 threads.  Every global load is issued up front: each
// thread's (m_c, l_c) for chunks t, t+256, ... and its partial outputs o_c[d]
// (d = d0 + t%S, chunks congruent to t/S mod 256/S, up to kBatch of them).
// The max and the sum over chunks are wave reductions in DPP followed by one
// LDS exchange each.
// out = sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M), zero when the
// denominator is zero (the reference's `sum > 0` guard and zero-filled
// output, math_util.rs:357, 372), then * sigmoid(gate).
constexpr int kMaxChunks = mi::kMaxSplitChunks;

extern "C" __device__ float __ockl_wfred_max_f32(float);
extern "C" __device__ float __ockl_wfred_add_f32(float);

// S = kCombineSlice values of d per workgroup: 16 for up to 16 columns
// (decode), 32 for the 32-column verify (measured: decode step 18.9 / 19.2 /
// 19.3 us with S = 16 / 32 / 8, verify 33.1 / 32.7 / 34.6 us).
template <int kCombineSlice>
__global__ void __launch_bounds__(256)
attn_combine_kernel(CombineArgs a) {
  constexpr int kCombineGroups = 256 / kCombineSlice;  // chunk groups of a workgroup
  __shared__ float red[2][4];
  __shared__ float wts[kMaxChunks];
  __shared__ float acc_s[kCombineGroups][kCombineSlice + 1];
  const int c = blockIdx.x;
  const int kvh = blockIdx.y / (D / kCombineSlice);
  const int d0 = (blockIdx.y % (D / kCombineSlice)) * kCombineSlice;
  const int s = blockIdx.z;
  const int t = threadIdx.x;
  const int wv = t >> 6;
  const int ncols = a.nq * 8;
  int64_t len = a.kv_len;
  bool bad = false;
  if (a.lengths) {
    len = a.lengths[s];
    const int32_t off = a.offsets[s];
    bad = len < 0 || len > a.kv_len || off < 0 || (off & 31);
    if (bad) len = 0;
  }
  const int nch = (int)((len + a.chunk - 1) / a.chunk);
  const int64_t base = (int64_t)s * a.max_chunks;  // first partial slot of s
  const float* ml = a.part_ml + ((kvh * a.nslots + base) * ncols + c) * 2;  // chunk ch at ml[ch * mstride]
  const int64_t mstride = (int64_t)ncols * 2;
  const int dl = t % kCombineSlice, cg = t / kCombineSlice;
  const float* po = a.part_o + ((kvh * a.nslots + base) * ncols + c) * D + d0 + dl;
  const int64_t ostride = (int64_t)ncols * D;

  float mloc[kMaxChunks / 256], lloc[kMaxChunks / 256];
#pragma unroll
  for (int u = 0; u < kMaxChunks / 256; u++) {
    const int ch = t + 256 * u;
    mloc[u] = ch < nch ? ml[ch * mstride] : kNegBig;
    lloc[u] = ch < nch ? ml[ch * mstride + 1] : 0.f;
  }
  constexpr int kBatch = 16;
  float ov[kBatch];
#pragma unroll
  for (int u = 0; u < kBatch; u++) {
    const int ch = cg + kCombineGroups * u;
    ov[u] = ch < nch ? po[ch * ostride] : 0.f;
  }
  float mx = kNegBig;
#pragma unroll
  for (int u = 0; u < kMaxChunks / 256; u++) mx = fmaxf(mx, mloc[u]);
  mx = __ockl_wfred_max_f32(mx);
  if ((t & 63) == 0) red[0][wv] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float lsum = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxChunks / 256; u++) {
    const int ch = t + 256 * u;
    if (ch < nch) {
      const float wgt = exp2f(mloc[u] - M);
      wts[ch] = wgt;
      lsum += lloc[u] * wgt;
    }
  }
  lsum = __ockl_wfred_add_f32(lsum);
  if ((t & 63) == 0) red[1][wv] = lsum;
  __syncthreads();  // publishes wts[] and the wave sums
  const float L = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  float o = 0.f;
#pragma unroll
  for (int u = 0; u < kBatch; u++) {
    const int ch = cg + kCombineGroups * u;
    if (ch < nch) o += ov[u] * wts[ch];
  }
  for (int ch = cg + kCombineGroups * kBatch; ch < nch; ch += kCombineGroups)
    o += po[ch * ostride] * wts[ch];
  acc_s[cg][dl] = o;
  __syncthreads();
  if (t < kCombineSlice) {
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < kCombineGroups; i++) r += acc_s[i][t];
    r = (L > 0.f) ? r / L : 0.f;
    if (bad) r = __builtin_nanf("");
    const int tok = c >> 3;
    const int hq = kvh * 8 + (c & 7);
    const int64_t oidx = (((int64_t)s * a.nq + tok) * a.H + hq) * D + d0 + t;
    if (a.gate) {
      const float gv = (float)a.gate[oidx];
      r = mi::gate_mul(r, gv);
    } else if (a.gate32) {
      const float gv =
          a.gate32[(((int64_t)s * a.nq + tok) * a.H + hq) * (2 * D) + D + d0 + t];
      r = mi::gate_mul(r, gv);
    }
    a.out[oidx] = (_Float16)r;
  }
}

// Merge for the flat ragged split: a sequence has few partials (its tiles
// span a few workgroups), so one workgroup per (column, KV head, sequence)
// with one thread per d runs a single online-softmax pass over them.
// Workgroup x < nw = min(nwg, T) of the split took tiles [x T / nw,
// (x+1) T / nw), so tile t is in workgroup ceil((t+1) nw / T) - 1 and the
// partials of sequence s are in slots first + s .. last + s.
__global__ void __launch_bounds__(D)
attn_combine_flat_kernel(CombineArgs a) {
  const int c = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z, d = threadIdx.x;
  const int ncols = a.nq * 8;
  const int32_t len = a.lengths[s], off = a.offsets[s];
  const bool bad = len < 0 || len > a.kv_len || off < 0 || (off & 31);
  const int64_t total = a.tile_off[a.batch];
  const int64_t ps = a.tile_off[s], pe = a.tile_off[s + 1];
  int64_t first = 0, nch = 0;
  if (pe > ps) {
    const int64_t nw = min((int64_t)a.nwg, total);
    first = ((ps + 1) * nw + total - 1) / total - 1;
    nch = (pe * nw + total - 1) / total - 1 - first + 1;
  }
  const int64_t slot0 = (kvh * a.nslots + first + s) * ncols + c;
  const float* ml = a.part_ml + slot0 * 2;
  const float* po = a.part_o + slot0 * D + d;
  float M = kNegBig, L = 0.f, o = 0.f;
  constexpr int kB = 8;  // partials loaded per batch, all before their use
  for (int64_t c0 = 0; c0 < nch; c0 += kB) {
    float mb[kB], lb[kB], ob[kB];
#pragma unroll
    for (int k = 0; k < kB; k++) {
      const bool in = c0 + k < nch;
      mb[k] = in ? ml[(c0 + k) * ncols * 2] : kNegBig;
      lb[k] = in ? ml[(c0 + k) * ncols * 2 + 1] : 0.f;
      ob[k] = in ? po[(c0 + k) * ncols * D] : 0.f;
    }
    float mx = M;
#pragma unroll
    for (int k = 0; k < kB; k++) mx = fmaxf(mx, mb[k]);
    const float sc = exp2f(M - mx);  // rescale what has been summed
    L *= sc;
    o *= sc;
    M = mx;
#pragma unroll
    for (int k = 0; k < kB; k++) {
      const float wgt = exp2f(mb[k] - M);
      L += lb[k] * wgt;
      o += ob[k] * wgt;
    }
  }
  float r = (L > 0.f) ? o / L : 0.f;
  if (bad) r = __builtin_nanf("");
  const int hq = kvh * 8 + c;
  const int64_t oidx = ((int64_t)s * a.H + hq) * D + d;
  if (a.gate) r = mi::gate_mul(r, (float)a.gate[oidx]);
  a.out[oidx] = (_Float16)r;
}

// Tile offsets of a ragged batch for the flat split: tile_off[s] = sum over
// r < s of ceil(len_r / 32) (0 for an invalid descriptor), tile_off[batch] =
// the total.  One workgroup, an exclusive scan per 256 sequences.
__global__ void __launch_bounds__(256)
ragged_plan_kernel(const int32_t* lengths, const int32_t* offsets, int batch, int64_t max_len,
                   int32_t* tile_off) {
  __shared__ int32_t scan[256];
  const int t = threadIdx.x;
  int32_t carry = 0;
  for (int b0 = 0; b0 < batch; b0 += 256) {
    const int sq = b0 + t;
    int32_t n = 0;
    if (sq < batch) {
      const int32_t len = lengths[sq], off = offsets[sq];
      const bool bad = len < 0 || len > max_len || off < 0 || (off & 31);
      n = bad ? 0 : (len + 31) >> 5;
    }
    scan[t] = n;
    __syncthreads();
    for (int d = 1; d < 256; d <<= 1) {  // inclusive scan
      const int32_t v = t >= d ? scan[t - d] : 0;
      __syncthreads();
      scan[t] += v;
      __syncthreads();
    }
    if (sq < batch) tile_off[sq] = carry + scan[t] - n;
    carry += scan[255];
    __syncthreads();
  }
  if (t == 0) tile_off[batch] = carry;
}

int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return (e && *e) ? atoi(e) : dflt;
}

// Split-planning knobs, read once per process (measurement aids; the
// defaults are the tuned values): MI_ATTN_SPLIT_GH=2 puts both KV heads of
// a Qwen3.6 layer in one workgroup (default one head per workgroup: at C2
// the same split time with half the partials, 18.8 against 19.5 us per
// step), MI_ATTN_SPLIT_WGS sets the target workgroup count,
// MI_ATTN_SPLIT_CHUNK fixes the keys per chunk.
const mi::SplitKnobs& split_knobs() {
  static const mi::SplitKnobs k{env_int("MI_ATTN_SPLIT_GH", 1),
                                std::max(1, env_int("MI_ATTN_SPLIT_WGS", 256)),
                                std::max(0, env_int("MI_ATTN_SPLIT_CHUNK", 0))};
  return k;
}

using mi::SplitPlan;
SplitPlan plan_split(int64_t max_len, int64_t batch, int G, int nq) {
  return mi::plan_split(max_len, batch, G, nq, split_knobs());
}

template <int NWH, int NCB, int GH, typename X = NoProj, bool FLAT = false>
mi_status launch_split(const SplitArgs& a, int64_t batch, hipStream_t stream, const X& x = X()) {
  const int ncols = a.nq * 8;
  size_t lds = (size_t)GH * (NWH * ncols * (D + 4) + 2 * NWH * ncols) * sizeof(float);
  if constexpr (is_proj<X>::value) lds += (size_t)GH * 8 * (D + 8) * sizeof(_Float16);
  if constexpr (FLAT) lds += (size_t)(kFusedPlan + 1) * sizeof(int32_t);
  static std::atomic<uint64_t> lds_set{0};
  // (below 160 KiB: the kernel also holds a few bytes of static LDS)
  MI_TRY(mi::set_lds_limit((const void*)attn_split_kernel<NWH, NCB, GH, X, FLAT>, 159 * 1024, lds_set));
  dim3 grid(a.max_chunks, a.G / GH, (unsigned)batch);
  MI_HIP(mi::launch("attn_split", attn_split_kernel<NWH, NCB, GH, X, FLAT>, grid,
                    dim3(NWH * GH * 64), lds, stream, a, x));
  return MI_OK;
}

template <int SH>
mi_status launch_proj(const SplitArgs& a, const SplitPlan& plan, hipStream_t stream,
                      const ProjArgs& p) {
  Proj<SH> x;
  static_cast<ProjArgs&>(x) = p;
  if (plan.gh == 2) return launch_split<4, 1, 2>(a, 1, stream, x);
  return launch_split<8, 1, 1>(a, 1, stream, x);
}

size_t split_workspace_bytes(int64_t batch, int G, int max_chunks, int nq) {
  size_t units = (size_t)batch * G * max_chunks * nq * 8;
  return units * (D + 2) * sizeof(float) + 256;
}

// The in-launch merge: partials o as usual, then (m, l) with a 256-byte
// stride per slot (workgroups of neighbouring slots run on different XCDs,
// whose L2s must not share a line); the state in mi_kv::mstate: counters,
// then per-XCD partials [G][8][8][D] and (m, l) [G][8][64].
size_t merge_workspace_bytes(int G, int max_chunks) {
  return (size_t)G * max_chunks * (8 * D + 64) * sizeof(float) + 256;
}
size_t merge_counter_bytes(int G) { return ((size_t)9 * G * kMergeStride * sizeof(int) + 4095) / 4096 * 4096; }
// The workspace a cache decode / verify launch asks for.
size_t attend_workspace_bytes(int G, int max_chunks, int nq) {
  const size_t s = split_workspace_bytes(1, G, max_chunks, nq);
  return nq == 1 ? std::max(s, merge_workspace_bytes(G, max_chunks)) : s;
}
// MI_ATTN_DECODE_MERGE=1 (read at each call) merges single-token decode
// inside the split launch; off by default: at C2 the merge chain after the
// last workgroup (store acknowledgement, XCD-local arrival, merge from L2,
// write-through, device arrival, final merge from memory) takes ~5 us, as
// long as the second launch it replaces (measured: 21.9 against 19.9 us per
// step on one box, 18.5-18.7 against ~18 us for the kernel end).
bool decode_merge_enabled() {
  const char* e = getenv("MI_ATTN_DECODE_MERGE");
  return e && *e && atoi(e) == 1;
}

// Flat ragged split: workgroups per KV-head group (one per CU), and the
// workspace: partials of nwg + batch slots, then the tile offsets.
int ragged_nwg(int G, int gh) { return std::max(1, 256 / std::max(1, G / gh)); }
size_t ragged_workspace_bytes(int64_t batch, int G, int nwg) {
  return split_workspace_bytes(1, G, nwg + (int)batch, 1) + (size_t)(batch + 1) * sizeof(int32_t);
}

// Runs split + combine for nq <= 4 query tokens per sequence.
struct AppendRows {
  const _Float16* k = nullptr;
  const _Float16* v = nullptr;
  int64_t row0 = 0;
  int n = 0;
};

mi_status run_split(const _Float16* k, const _Float16* v, const int32_t* offsets,
                    const int32_t* lengths, int64_t kv_len, int64_t lim0,
                    int64_t max_len, int64_t batch, int H, int G, int nq,
                    const _Float16* q, const _Float16* gate, _Float16* out,
                    void* ws, size_t ws_bytes, hipStream_t stream,
                    const AppendRows& app = AppendRows(), const ProjArgs* proj = nullptr,
                    const mi_kv* kv = nullptr) {
  const SplitPlan plan = plan_split(max_len, batch, G, nq);
  SplitArgs a;
  a.mcnt = nullptr;
  a.k = k;
  a.v = v;
  a.offsets = offsets;
  a.lengths = lengths;
  a.kv_len = kv_len;
  a.lim0 = lim0;
  a.q = q;
  a.G = G;
  a.H = H;
  a.nq = nq;
  a.chunk = plan.chunk;
  a.max_chunks = plan.max_chunks;
  a.scale_log2e = mi::kLog2e / sqrtf((float)D);
  a.app_k = app.k;
  a.app_v = app.v;
  a.kw = const_cast<_Float16*>(k);
  a.vw = const_cast<_Float16*>(v);
  a.app0 = app.row0;
  a.app_n = app.n;
  a.tile_off = nullptr;
  a.tile_off_out = nullptr;
  a.batch = (int)batch;
  const int nwg = ragged_nwg(G, plan.gh);
  const size_t need = lengths ? ragged_workspace_bytes(batch, G, nwg)
                              : split_workspace_bytes(batch, G, a.max_chunks, nq);
  if (ws_bytes < need)
    return mi::fail(MI_ERR_INVALID_ARG, "workspace %zu bytes < %zu needed", ws_bytes, need);
  const size_t slots = lengths ? (size_t)nwg + batch : (size_t)batch * a.max_chunks;
  a.part_o = (float*)ws;
  a.part_ml = a.part_o + slots * G * nq * 8 * D;
  a.nslots = (int64_t)slots;
  if (lengths) {
    // flat split over the concatenated sequences (one nq = 1 token each)
    if (nq != 1) return mi::fail(MI_ERR_INVALID_ARG, "ragged batches take one query token");
    if ((int64_t)batch * ((max_len + 31) / 32) >= ((int64_t)1 << 31))
      return mi::fail(MI_ERR_UNSUPPORTED, "batch * max_len / 32 beyond 2^31 tiles");
    int32_t* tile_off = (int32_t*)(a.part_ml + slots * G * nq * 8 * 2);
    if (batch <= kFusedPlan) {
      a.tile_off_out = tile_off;  // the split launch computes and stores them
    } else {
      MI_HIP(mi::launch("ragged_plan", ragged_plan_kernel, dim3(1), dim3(256), 0, stream, lengths,
                        offsets, (int)batch, kv_len, tile_off));
    }
    a.tile_off = tile_off;
    a.max_chunks = nwg;
    a.chunk = 0;
  }
  // In-launch merge: one sequence, one query token, one KV head per
  // workgroup, 8 waves (the launch_split<8, 1, 1> forms), on a device that
  // dispatches round-robin over 8 XCDs, with room for the padded (m, l).
  const bool merge = kv && kv->merge_ok && kv->mstate && !lengths && batch == 1 && nq == 1 &&
                     plan.gh == 1 && plan.ncb == 1 && plan.nwh == 8 && decode_merge_enabled() &&
                     ws_bytes >= merge_workspace_bytes(G, a.max_chunks);
  if (merge) {
    a.mcnt = (int*)kv->mstate;
    a.xo = (float*)((char*)kv->mstate + merge_counter_bytes(G));
    a.xml = a.xo + (size_t)G * 8 * 8 * D;
    a.gate = gate;
    a.gate32 = proj ? proj->q_proj : nullptr;
    a.out = out;
  }
  mi_status st;
  if (proj) {
    if (nq != 1 || batch != 1) return mi::fail(MI_ERR_INVALID_ARG, "projection input: one token");
    switch (proj->rot_half / 32) {
      case 0: st = launch_proj<0>(a, plan, stream, *proj); break;
      case 1: st = launch_proj<1>(a, plan, stream, *proj); break;
      case 2: st = launch_proj<2>(a, plan, stream, *proj); break;
      case 3: st = launch_proj<3>(a, plan, stream, *proj); break;
      case 4: st = launch_proj<4>(a, plan, stream, *proj); break;
      default: return mi::fail(MI_ERR_UNSUPPORTED, "rot_half=%d", proj->rot_half);
    }
  } else if (lengths) {
    st = plan.gh == 2 ? launch_split<4, 1, 2, NoProj, true>(a, 1, stream)
                      : launch_split<8, 1, 1, NoProj, true>(a, 1, stream);
  } else if (plan.ncb == 2)
    st = launch_split<4, 2, 1>(a, batch, stream);
  else if (plan.gh == 2)
    st = launch_split<4, 1, 2>(a, batch, stream);
  else
    st = launch_split<8, 1, 1>(a, batch, stream);
  MI_TRY(st);
  if (merge) return MI_OK;  // merged and written by the split launch
  CombineArgs c;
  c.offsets = offsets;
  c.lengths = lengths;
  c.kv_len = kv_len;
  c.part_o = a.part_o;
  c.part_ml = a.part_ml;
  c.gate = gate;
  c.gate32 = proj ? proj->q_proj : nullptr;
  c.out = out;
  c.G = G;
  c.H = H;
  c.nq = nq;
  c.chunk = a.chunk;
  c.max_chunks = a.max_chunks;
  c.tile_off = a.tile_off;
  c.nslots = a.nslots;
  c.nwg = nwg;
  c.batch = (int)batch;
  if (lengths) {
    MI_HIP(mi::launch("attn_combine", attn_combine_flat_kernel, dim3(8, G, (unsigned)batch),
                      dim3(D), 0, stream, c));
    return MI_OK;
  }
  if (nq > 2) {
    MI_HIP(mi::launch("attn_combine", attn_combine_kernel<32>, dim3(nq * 8, G * (D / 32), (unsigned)batch),
                      dim3(256), 0, stream, c));
  } else {
    MI_HIP(mi::launch("attn_combine", attn_combine_kernel<16>, dim3(nq * 8, G * (D / 16), (unsigned)batch),
                      dim3(256), 0, stream, c));
  }
  return MI_OK;
}

// Merge of a few chunks (at most kColsChunks) for many columns: one thread
// per output value, one workgroup of D threads per (column, KV head).  The
// wide verify's partials for many tokens come in few chunks, where
// attn_combine_kernel's workgroup per column and 32-value slice (chunks
// spread over its threads) would launch 16 workgroups per column.
constexpr int kColsChunks = 16;
__global__ void __launch_bounds__(D) attn_combine_cols_kernel(CombineArgs a) {
  const int c = blockIdx.x, kvh = blockIdx.y, d = threadIdx.x;
  const int ncols = a.nq * 8;
  const int nch = (int)((a.kv_len + a.chunk - 1) / a.chunk);
  float m[kColsChunks], l[kColsChunks], o[kColsChunks];
#pragma unroll
  for (int ch = 0; ch < kColsChunks; ch++) {
    m[ch] = kNegBig;
    l[ch] = 0.f;
    o[ch] = 0.f;
    if (ch < nch) {
      const int64_t slot = ((int64_t)kvh * a.nslots + ch) * ncols + c;
      m[ch] = a.part_ml[slot * 2];
      l[ch] = a.part_ml[slot * 2 + 1];
      o[ch] = a.part_o[slot * D + d];
    }
  }
  float M = kNegBig;
#pragma unroll
  for (int ch = 0; ch < kColsChunks; ch++) M = fmaxf(M, m[ch]);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int ch = 0; ch < kColsChunks; ch++) {
    const float w = exp2f(m[ch] - M);
    L += l[ch] * w;
    O += o[ch] * w;
  }
  // out = O / L (zero when L = 0, math_util.rs:357, 372), then the gate
  float r = (L > 0.f) ? O / L : 0.f;
  const int tok = c >> 3, hq = kvh * 8 + (c & 7);
  const int64_t oidx = ((int64_t)tok * a.H + hq) * D + d;
  if (a.gate) r = mi::gate_mul(r, (float)a.gate[oidx]);
  a.out[oidx] = (_Float16)r;
}

// Wide verify for more than 4 query tokens (MI_ATTN_VERIFY_WIDE=0, read at
// each call, turns it off): one split pass that reads every K/V tile once
// per 16 tokens (attn_prefill64_kernel's MFMA tiles over key chunks), then
// the combine, instead of one split-K launch pair per 4-token group.
bool verify_wide_enabled() {
  const char* e = getenv("MI_ATTN_VERIFY_WIDE");
  return !(e && *e && atoi(e) == 0);
}

// The wide verify's plan (mi::wide_plan) and the workspace its partials
// (O, m, l) take.
struct WideLaunch {
  int64_t chunk;
  int nchunks;
  size_t ws_bytes;
};
WideLaunch wide_launch(int G, int64_t past, int32_t n) {
  const mi::WidePlan w = mi::wide_plan(G, past, n);
  WideLaunch p;
  p.chunk = w.chunk;
  p.nchunks = w.nchunks;
  p.ws_bytes = (size_t)G * p.nchunks * 8 * n * (D + 2) * sizeof(float) + 256;
  return p;
}

mi_status wide_attend(mi_kv* kv, int32_t layer, const _Float16* q, const _Float16* gate,
                      _Float16* out, int64_t past_pos, int32_t n, hipStream_t stream,
                      const _Float16* k_new, const _Float16* v_new) {
  const int G = kv->G;
  const int64_t rows = past_pos + n;
  const WideLaunch wp = wide_launch(G, past_pos, n);
  const int64_t chunk = wp.chunk;
  const int nchunks = wp.nchunks;
  const int ncols = 8 * n;
  const size_t units = (size_t)G * nchunks * ncols;
  void* ws;
  MI_TRY(mi::kv_workspace(kv, wp.ws_bytes, stream, &ws));
  float* part_o = (float*)ws;
  float* part_ml = part_o + units * D;
  if (k_new) MI_TRY(mi::kv_append_rows(kv, layer, k_new, v_new, past_pos, n, stream));
  MI_TRY(mi::verify_wide_split(kv, layer, q, past_pos, n, chunk, nchunks, part_o, part_ml,
                               stream));
  CombineArgs c{};
  c.kv_len = rows;
  c.part_o = part_o;
  c.part_ml = part_ml;
  c.gate = gate;
  c.out = out;
  c.G = G;
  c.H = kv->H;
  c.nq = n;
  c.chunk = (int)chunk;
  c.max_chunks = nchunks;
  c.batch = 1;
  c.nslots = nchunks;
  if (nchunks <= kColsChunks)
    MI_HIP(mi::launch("attn_combine", attn_combine_cols_kernel, dim3(n * 8, G), dim3(D), 0,
                      stream, c));
  else
    MI_HIP(mi::launch("attn_combine", attn_combine_kernel<32>, dim3(n * 8, G * (D / 32), 1),
                      dim3(256), 0, stream, c));
  return MI_OK;
}

// Verify / decode over the cache: n query tokens at positions past_pos ..
// past_pos+n-1, rows [0, past_pos+n) already in the cache.
// With k_new / v_new, the n new rows [past_pos, past_pos + n) are appended
// by the split kernels themselves (each token group appends its own rows,
// which precede every read of them; the wide form appends them all in a
// launch of their own first); the caller has grown the cache.
mi_status cache_attend(mi_kv* kv, int32_t layer, const _Float16* q, const _Float16* gate,
                       _Float16* out, int64_t past_pos, int32_t n, hipStream_t stream,
                       const _Float16* k_new = nullptr, const _Float16* v_new = nullptr) {
  if (n > 4 && verify_wide_enabled())
    return wide_attend(kv, layer, q, gate, out, past_pos, n, stream, k_new, v_new);
  const int64_t lim0 = past_pos + 1;
  // The workspace is grown once, to the largest group's need, before any
  // launch: a growth refused under graph capture then leaves nothing of
  // this call half-recorded.
  size_t need = 0;
  for (int32_t t0 = 0; t0 < n; t0 += 4) {
    const int nq = (n - t0) < 4 ? (n - t0) : 4;
    const SplitPlan plan = plan_split(past_pos + t0 + nq, 1, kv->G, nq);
    need = std::max(need, attend_workspace_bytes(kv->G, plan.max_chunks, nq));
  }
  void* ws;
  MI_TRY(mi::kv_workspace(kv, need, stream, &ws));
  for (int32_t t0 = 0; t0 < n; t0 += 4) {
    const int nq = (n - t0) < 4 ? (n - t0) : 4;
    const int64_t rows = past_pos + t0 + nq;  // rows the last token of this group sees
    const int64_t qoff = (int64_t)t0 * kv->H * D;
    AppendRows app;
    if (k_new) {
      app.k = k_new + (int64_t)t0 * kv->G * D;
      app.v = v_new + (int64_t)t0 * kv->G * D;
      app.row0 = past_pos + t0;
      app.n = nq;
    }
    MI_TRY(run_split(kv->k[layer], kv->v[layer], nullptr, nullptr, rows, lim0 + t0,
                     rows, 1, kv->H, kv->G, nq, q + qoff, gate ? gate + qoff : nullptr,
                     out + qoff, ws, kv->ws_bytes, stream, app, nullptr, kv));
  }
  return MI_OK;
}

}  // namespace

namespace {
// Records the XCD each workgroup runs on (HW_REG_XCC_ID).
__global__ void xcc_probe_kernel(int* out) {
  if (threadIdx.x == 0) {
    int v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    out[blockIdx.x] = v;
  }
}
}  // namespace

namespace mi {
size_t merge_state_bytes(int G) {
  return merge_counter_bytes(G) + (size_t)G * 8 * (8 * D + 64) * sizeof(float);
}

bool xcd_round_robin() {
  static std::atomic<int> known[64];  // per device: 0 unknown, 1 yes, 2 no
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  const int k = known[dev].load(std::memory_order_acquire);
  if (k) return k == 1;
  constexpr int kN = 2048;
  int* d = nullptr;
  bool ok = hipMalloc(&d, kN * sizeof(int)) == hipSuccess;
  std::vector<int> h(kN, -1);
  if (ok) {
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(kN), dim3(64), 0, 0, d);
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpy(h.data(), d, kN * sizeof(int), hipMemcpyDeviceToHost) == hipSuccess;
  }
  if (d) (void)hipFree(d);
  for (int b = 0; ok && b < kN; b++) ok = h[b] == b % 8;
  known[dev].store(ok ? 1 : 2, std::memory_order_release);
  return ok;
}

mi_status attend_cache(mi_kv* kv, int32_t layer, const _Float16* q, const _Float16* gate,
                       _Float16* out, int64_t past_pos, int32_t n, hipStream_t stream) {
  return cache_attend(kv, layer, q, gate, out, past_pos, n, stream);
}

mi_status attend_wide(mi_kv* kv, int32_t layer, const _Float16* q, const _Float16* gate,
                      _Float16* out, int64_t past, int32_t n, hipStream_t stream) {
  return wide_attend(kv, layer, q, gate, out, past, n, stream, nullptr, nullptr);
}

size_t wide_workspace_bytes(int G, int64_t past, int32_t n) {
  return wide_launch(G, past, n).ws_bytes;
}
}  // namespace mi

extern "C" mi_status mi_attn_decode(mi_kv* kv, int32_t layer, const mi_f16* q,
                                    const mi_f16* gate, mi_f16* out, int64_t seq_len,
                                    mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!q || !out) return mi::fail(MI_ERR_INVALID_ARG, "null q/out");
  if (seq_len < 0 || seq_len > kv->cap)
    return mi::fail(MI_ERR_OUT_OF_RANGE, "seq_len %lld outside [0, capacity %lld]",
                    (long long)seq_len, (long long)kv->cap);
  // seq_len == 0 runs no split work; the combine writes zeros (times the gate).
  return cache_attend(kv, layer, (const _Float16*)q, (const _Float16*)gate, (_Float16*)out,
                      seq_len - 1, 1, (hipStream_t)stream);
}

extern "C" mi_status mi_attn_step(mi_kv* kv, int32_t layer, const mi_f16* q,
                                  const mi_f16* k, const mi_f16* v, const mi_f16* gate,
                                  mi_f16* out, int64_t pos, mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!q || !k || !v || !out) return mi::fail(MI_ERR_INVALID_ARG, "null q/k/v/out");
  if (pos < 0) return mi::fail(MI_ERR_OUT_OF_RANGE, "pos=%lld", (long long)pos);
  MI_TRY(mi::kv_grow(kv, pos + 1, (hipStream_t)stream));
  MI_TRY(cache_attend(kv, layer, (const _Float16*)q, (const _Float16*)gate, (_Float16*)out, pos,
                      1, (hipStream_t)stream, (const _Float16*)k, (const _Float16*)v));
  kv->len[layer] = pos + 1;
  return MI_OK;
}

extern "C" mi_status mi_attn_verify(mi_kv* kv, int32_t layer, const mi_f16* q,
                                    const mi_f16* k, const mi_f16* v, const mi_f16* gate,
                                    mi_f16* out, int64_t past_pos, int32_t n,
                                    mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!q || !out) return mi::fail(MI_ERR_INVALID_ARG, "null q/out");
  if (!k != !v) return mi::fail(MI_ERR_INVALID_ARG, "k and v must both be given or both NULL");
  if (n <= 0) return mi::fail(MI_ERR_INVALID_ARG, "n=%d", n);
  if (past_pos < 0) return mi::fail(MI_ERR_OUT_OF_RANGE, "past_pos=%lld", (long long)past_pos);
  if (!k && past_pos + n > kv->len[layer])
    return mi::fail(MI_ERR_OUT_OF_RANGE, "k = v = NULL but rows [%lld, %lld) are not in the "
                    "cache (len %lld)", (long long)past_pos, (long long)(past_pos + n),
                    (long long)kv->len[layer]);
  MI_TRY(mi::kv_grow(kv, past_pos + n, (hipStream_t)stream));
  MI_TRY(cache_attend(kv, layer, (const _Float16*)q, (const _Float16*)gate, (_Float16*)out,
                      past_pos, n, (hipStream_t)stream, (const _Float16*)k, (const _Float16*)v));
  kv->len[layer] = past_pos + n;
  return MI_OK;
}

extern "C" size_t mi_attn_ragged_workspace_size(int32_t batch, int32_t max_len,
                                                int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim) {
  if (batch <= 0 || max_len <= 0 || num_kv_heads <= 0) return 256;
  (void)num_q_heads;
  (void)head_dim;
  const SplitPlan plan = plan_split(max_len, batch, num_kv_heads, 1);
  return ragged_workspace_bytes(batch, num_kv_heads, ragged_nwg(num_kv_heads, plan.gh));
}

extern "C" mi_status mi_attn_decode_ragged(const mi_f16* k_rows, const mi_f16* v_rows,
                                           const int32_t* offsets, const int32_t* lengths,
                                           int32_t batch, int32_t max_len,
                                           int32_t num_q_heads, int32_t num_kv_heads,
                                           int32_t head_dim, const mi_f16* q,
                                           const mi_f16* gate, mi_f16* out, void* workspace,
                                           size_t workspace_bytes, mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_shape(num_q_heads, num_kv_heads, head_dim));
  if (!k_rows || !v_rows || !offsets || !lengths || !q || !out || !workspace)
    return mi::fail(MI_ERR_INVALID_ARG, "null pointer argument");
  if (batch <= 0 || max_len < 0)
    return mi::fail(MI_ERR_INVALID_ARG, "batch=%d max_len=%d", batch, max_len);
  if (batch > 65535)  // the merge launch has one grid row per sequence
    return mi::fail(MI_ERR_UNSUPPORTED, "batch=%d above 65535 sequences", batch);
  const int64_t ml = max_len > 0 ? max_len : 1;
  return run_split((const _Float16*)k_rows, (const _Float16*)v_rows, offsets, lengths, ml, 0,
                   ml, batch, num_q_heads, num_kv_heads, 1, (const _Float16*)q,
                   (const _Float16*)gate, (_Float16*)out, workspace, workspace_bytes,
                   (hipStream_t)stream);
}

extern "C" mi_status mi_attn_step_proj(mi_kv* kv, int32_t layer, const float* q_proj,
                                       const float* k, const float* v,
                                       const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                       int32_t rotary_dim, float rope_theta, float eps,
                                       mi_f16* out, int64_t pos, mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!q_proj || !k || !v || !q_norm_w || !k_norm_w || !out)
    return mi::fail(MI_ERR_INVALID_ARG, "null pointer argument");
  if (pos < 0) return mi::fail(MI_ERR_OUT_OF_RANGE, "pos=%lld", (long long)pos);
  MI_TRY(mi::check_rope(kv, rotary_dim, rope_theta, eps));
  if (rotary_dim % 64)
    return mi::fail(MI_ERR_UNSUPPORTED,
                    "rotary_dim=%d: the fused step rotates whole 64-column slices; use "
                    "mi_qk_norm_rope_append + mi_attn_decode",
                    rotary_dim);
  MI_TRY(mi::kv_grow(kv, pos + 1, (hipStream_t)stream));
  ProjArgs x{};
  x.q_proj = q_proj;
  x.k = k;
  x.v = v;
  x.q_w = q_norm_w;
  x.k_w = k_norm_w;
  x.rot_half = rotary_dim / 2;
  x.eps = eps;
  float inv_freq[MI_ROPE_MAX_DIM / 2];
  mi::rope_inv_freq(rope_theta, rotary_dim, inv_freq);
  const float fpos = (float)pos;
  for (int i = 0; i < x.rot_half; i++) {
    const float theta = fpos * inv_freq[i];
    x.cs[i] = cosf(theta);
    x.cs[x.rot_half + i] = sinf(theta);
  }
  const int64_t rows = pos + 1;
  const SplitPlan plan = plan_split(rows, 1, kv->G, 1);
  void* ws;
  MI_TRY(mi::kv_workspace(kv, attend_workspace_bytes(kv->G, plan.max_chunks, 1), (hipStream_t)stream, &ws));
  AppendRows app;
  app.row0 = pos;
  app.n = 1;
  MI_TRY(run_split(kv->k[layer], kv->v[layer], nullptr, nullptr, rows, rows, rows, 1, kv->H,
                   kv->G, 1, nullptr, nullptr, (_Float16*)out, ws, kv->ws_bytes,
                   (hipStream_t)stream, app, &x, kv));
  kv->len[layer] = pos + 1;
  return MI_OK;
}

// ------------------------------------------- allocation-free ragged decode --
//
// The ragged decode's workspace (split partials + tile offsets) as a
// file-scope device array, for callers that cannot allocate.  Each device
// the library runs on holds its own copy until the process ends; host code
// reaches it only through the address hipGetSymbolAddress returns for the
// current device (the array's name in host code is not a device address).
// Nothing in it has to start at zero: the plan kernel (or, for up to
// kFusedPlan sequences, the split launch itself) writes every tile offset
// and the split kernel writes every partial slot the merge reads.
static __device__ __align__(256) unsigned char scratch[MI_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`, looked up once per device.  The
// launch stream must belong to the current device: the copy is per device.
mi_status scratch_ptr(hipStream_t stream, void** out) {
  int dev = 0;
  MI_HIP(hipGetDevice(&dev));
  if (stream) {
    int sdev = 0;
    MI_HIP(hipStreamGetDevice(stream, &sdev));
    if (sdev != dev)
      return mi::fail(MI_ERR_INVALID_ARG, "stream on device %d, current device %d", sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices)
    return mi::fail(MI_ERR_UNSUPPORTED, "device %d beyond the %d the library tracks", dev,
                    kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    MI_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return MI_OK;
}
}  // namespace

extern "C" mi_status mi_attn_decode_ragged_noalloc(
    const mi_f16* k_rows, const mi_f16* v_rows, const int32_t* offsets, const int32_t* lengths,
    int32_t batch, int32_t max_len, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, const mi_f16* q, const mi_f16* gate, mi_f16* out, mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_shape(num_q_heads, num_kv_heads, head_dim));
  if (batch <= 0 || max_len < 0)
    return mi::fail(MI_ERR_INVALID_ARG, "batch=%d max_len=%d", batch, max_len);
  const size_t need =
      mi_attn_ragged_workspace_size(batch, max_len, num_q_heads, num_kv_heads, head_dim);
  if (need > (size_t)MI_NOALLOC_SCRATCH_BYTES)
    return mi::fail(MI_ERR_UNSUPPORTED,
                    "batch=%d needs %zu bytes of scratch; the static scratch holds %zu "
                    "(use mi_attn_decode_ragged with a workspace)",
                    batch, need, (size_t)MI_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  MI_TRY(scratch_ptr((hipStream_t)stream, &ws));
  return mi_attn_decode_ragged(k_rows, v_rows, offsets, lengths, batch, max_len, num_q_heads,
                               num_kv_heads, head_dim, q, gate, out, ws,
                               (size_t)MI_NOALLOC_SCRATCH_BYTES, stream);
}
