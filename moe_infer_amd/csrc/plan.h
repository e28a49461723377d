// Launch plans shared by the kernels, their host launchers and the CPU
// model of their memory accesses (tests/copy_bounds_model.cc compiles this
// header with g++): the causal prefill's per-wave tile schedule and the
// split-K decode's chunking.  Plain C++ with no HIP dependency.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define MI_HD __host__ __device__
#else
#define MI_HD
#endif

namespace mi {

// ------------------------------------------------------------- prefill --

constexpr int kPrefillBQ = 128;  // queries per workgroup (4 waves of 32)
constexpr int kPrefillBK = 64;   // keys per LDS tile

// The key-tile range of one wave of the causal prefill: the wave owns
// queries q0 + 32 w .. + 31 of query tile `qtile` (positions past + i), and
// its workgroup walks key tiles 0 .. nt-1 (64 keys each) up to the last
// key any of its queries sees.  Positions are 32-bit (the host checks
// past + n + 2 * kPrefillBK < 2^31).
struct PrefillWave {
  int first;   // smallest query position of the wave
  int last;    // largest query position of the wave (may be >= kv_len: padding)
  int kv_len;  // rows in the cache after the append: past + n
  int nt;      // key tiles the workgroup walks
};

MI_HD inline PrefillWave prefill_wave(int past, int n, int qtile, int w) {
  PrefillWave p;
  const int q0 = qtile * kPrefillBQ;
  p.first = past + q0 + 32 * w;
  p.last = p.first + 31;
  p.kv_len = past + n;
  const int end = past + q0 + kPrefillBQ < p.kv_len ? past + q0 + kPrefillBQ : p.kv_len;
  p.nt = (end + kPrefillBK - 1) / kPrefillBK;
  return p;
}

// Tile t of the wave's walk: does the wave attend it (some query sees a key
// of it), is it on the wave's diagonal (needs the causal mask), and does it
// take the steady-state schedule?  The steady schedule copies K(t+1) into
// LDS unconditionally, so it is taken only when t + 1 < nt: a wave whose
// queries all lie past n (padding of the last query tile) has its diagonal
// beyond the last tile, so "not diagonal" alone would let it copy K(nt),
// 64 rows past kv_len and possibly past the allocation.  Every other tile
// copies K(t+1) only when t + 1 < nt, and V(t).
MI_HD inline bool prefill_active(const PrefillWave& p, int t) {
  return t * kPrefillBK <= p.last;
}
MI_HD inline bool prefill_diag(const PrefillWave& p, int t) {
  return t * kPrefillBK + kPrefillBK - 1 > p.first;
}
MI_HD inline bool prefill_steady(const PrefillWave& p, int t, bool pending) {
  return prefill_active(p, t) && pending && !prefill_diag(p, t) && t + 1 < p.nt;
}

// The 64-queries-per-wave form (attn_prefill64_kernel): wave (qb, kp) owns
// queries q0 + 64 qb .. + 63 and keys 32 kp .. 32 kp + 31 of every 64-key
// tile; the workgroup walks the same nt tiles as above.
struct PrefillWave64 {
  int first, last, kv_len, nt;
  int koff;  // 32 kp: the wave's key half of a tile
};

MI_HD inline PrefillWave64 prefill_wave64(int past, int n, int qtile, int qb, int kp) {
  PrefillWave64 p;
  const int q0 = qtile * kPrefillBQ;
  p.first = past + q0 + 64 * qb;
  p.last = p.first + 63;
  p.kv_len = past + n;
  const int end = past + q0 + kPrefillBQ < p.kv_len ? past + q0 + kPrefillBQ : p.kv_len;
  p.nt = (end + kPrefillBK - 1) / kPrefillBK;
  p.koff = 32 * kp;
  return p;
}
// The wide verify's form of the same: the workgroup's keys are chunk
// [kbeg, kbeg + chunk) of [0, past + n), positions relative to kbeg; its
// row block holds tokens tok0 .. tok0 + 15, rows 64 qb .. + 63 being tokens
// tok0 + 8 qb .. + 7 (each with the group's eight heads), token i seeing
// keys up to past + i.  A chunk past every key its tokens see keeps one
// tile, fully masked (empty partials).
MI_HD inline PrefillWave64 verify_wave64(int64_t past, int n, int64_t kbeg, int64_t chunk,
                                         int tok0, int qb, int kp) {
  PrefillWave64 p;
  p.first = (int)(past - kbeg) + tok0 + 8 * qb;
  p.last = p.first + 7;
  const int tend = n < tok0 + 16 ? n : tok0 + 16;  // the block's tokens
  int64_t end = past + tend - kbeg;                 // keys they see in the chunk
  if (end > chunk) end = chunk;
  if (end < 1) end = 1;
  p.kv_len = (int)end;
  p.nt = (p.kv_len + kPrefillBK - 1) / kPrefillBK;
  p.koff = 32 * kp;
  return p;
}
MI_HD inline bool prefill64_active(const PrefillWave64& p, int t) {
  return t * kPrefillBK + p.koff <= p.last;
}
MI_HD inline bool prefill64_diag(const PrefillWave64& p, int t) {
  return t * kPrefillBK + p.koff + 31 > p.first;
}
// As prefill_steady: the steady schedule copies K(t+1), so t + 1 < nt.
MI_HD inline bool prefill64_steady(const PrefillWave64& p, int t, bool pending) {
  return prefill64_active(p, t) && pending && !prefill64_diag(p, t) && t + 1 < p.nt;
}

// ----------------------------------------------------------- split-K --

// The 32-key tiles wave w of nwh reads in a chunk [begin, end): a
// contiguous run of ceil(tiles / nwh) tiles from first, while k0 < last.
struct WaveTiles {
  int64_t first, last;
};
MI_HD inline WaveTiles split_wave_tiles(int64_t begin, int64_t end, int nwh, int w) {
  const int64_t per = ((end - begin + 31) / 32 + nwh - 1) / nwh;
  WaveTiles r;
  r.first = begin + 32 * per * w;
  const int64_t e = begin + 32 * per * (w + 1);
  r.last = e < end ? e : end;
  return r;
}

// Most chunks (partials) per sequence of one split launch.
constexpr int kMaxSplitChunks = 1024;

// Chunking of the wide verify / split-K prefill (attn_verify_wide_kernel):
// about 256 workgroups of (row block of 16 tokens, chunk, KV head) over rows
// [0, past + n); whole 64-key tiles; at most kMaxSplitChunks chunks (the
// merge kernels' limit).
struct WidePlan {
  int64_t chunk;
  int nchunks;
};
inline WidePlan wide_plan(int G, int64_t past, int n) {
  const int64_t rows = past + n;
  const int64_t nrb = (n + 15) / 16;
  int64_t target = (256 + G * nrb - 1) / (G * nrb);
  if (target < 1) target = 1;
  int64_t chunk = (rows + target - 1) / target;
  const int64_t min_chunk = (rows + kMaxSplitChunks - 1) / kMaxSplitChunks;
  if (chunk < min_chunk) chunk = min_chunk;
  chunk = (chunk + kPrefillBK - 1) / kPrefillBK * kPrefillBK;
  WidePlan p;
  p.chunk = chunk;
  p.nchunks = (int)((rows + chunk - 1) / chunk);
  return p;
}

struct SplitKnobs {
  int gh;     // KV heads per workgroup (2, or 1 when set to 1)
  int wgs;    // target workgroup count
  int chunk;  // fixed keys per chunk (0: planned)
};

struct SplitPlan {
  int nwh, gh, ncb, chunk, max_chunks;
};

// Kernel variant and chunking of one split launch over sequences of at
// most max_len rows.  Keys per chunk (per head): enough workgroups to
// cover 256 CUs about once (K/V of one key and head is 1 KiB, so a 128-key
// chunk of two heads moves 256 KiB and leaves one 8 KiB partial per head and
// query token), at least one 32-key tile, at most 2048 keys (ragged batches
// balance better with more workgroups), and at most kMaxSplitChunks chunks.
// Chunks are whole 32-key tiles; the waves of a workgroup take its tiles
// round-robin.  Decode rounds chunks to 32 keys: rounding up to 32 * NWH
// would leave up to half the CUs idle just above a power of two (ctx 32769:
// 129 workgroups instead of 256, 21.0 against 18.1 us per call).  The
// 32-column verify (nq > 2) keeps whole wave rounds (measured ~1 us faster
// at 65540 rows: 206 workgroups of 20 tiles against 242 of 17).
inline SplitPlan plan_split(int64_t max_len, int64_t batch, int G, int nq, const SplitKnobs& k) {
  SplitPlan p;
  p.ncb = nq <= 2 ? 1 : 2;
  if (p.ncb == 2) {  // 32 columns: 4 waves, one head (registers and LDS)
    p.nwh = 4;
    p.gh = 1;
  } else if (G % 2 == 0 && k.gh == 2) {
    p.nwh = 4;
    p.gh = 2;
  } else {
    p.nwh = 8;
    p.gh = 1;
  }
  const int64_t step = 32 * p.nwh;
  const int64_t target_wgs = k.wgs > 0 ? k.wgs : 1;
  int64_t chunk = k.chunk;
  if (chunk <= 0) {
    chunk = (batch * G * max_len + p.gh * target_wgs - 1) / (p.gh * target_wgs);
    if (chunk > 2048) chunk = 2048;
  }
  const int64_t min_chunk = (max_len + kMaxSplitChunks - 1) / kMaxSplitChunks;
  if (chunk < min_chunk) chunk = min_chunk;
  const int64_t gran = p.ncb == 2 ? step : 32;
  chunk = (chunk + gran - 1) / gran * gran;
  if (chunk < gran) chunk = gran;  // also for max_len == 0
  p.chunk = (int)chunk;
  p.max_chunks = (int)((max_len + chunk - 1) / chunk);
  if (p.max_chunks < 1) p.max_chunks = 1;
  return p;
}

}  // namespace mi
