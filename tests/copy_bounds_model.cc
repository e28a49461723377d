// CPU model of the rows the attention kernels read, over the launch plans of
// moe_infer_amd/csrc/plan.h (the same header the kernels and their launchers
// use).  Built and run by tests/test_copy_bounds.py; prints one line per
// check: "<name> <cases> <violations>".
//
// Prefill (attn_prefill_kernel): every wave copies K tile 0 before its loop;
// at tile t the steady schedule (mi::prefill_steady) copies K(t+1) and V(t),
// any other tile copies K(t+1) when t + 1 < nt, and V(t).  A tile is rows
// [64 T, 64 T + 64) of both K and V; the cache holds round_cap(past + n) rows
// at least (capacities are multiples of 256 rows).  The same walk with the
// steady condition lacking "t + 1 < nt" is checked too, and must find
// violations: it is the copy past the allocation that faulted before the
// condition was added.
//
// Split-K decode / verify (attn_split_kernel, non-ragged): chunk c covers
// keys [c * chunk, min((c+1) * chunk, len)); wave w of NWH reads the whole
// 32-key tiles of mi::split_wave_tiles (the kernel calls the same helper):
// k0 = begin + 32 (P w + i), i = 0 .. P-1, P = ceil(tiles / NWH), while
// k0 < end.  Each tile must be 32-aligned and lie inside
// round_cap(len) rows, every key of the chunk must be read by exactly one
// wave, and chunks must number at most kMaxSplitChunks (the combine kernel
// merges at most that many).
#include <cstdio>
#include <initializer_list>

#include "plan.h"

static long long round_cap(long long rows) {
  if (rows < 256) rows = 256;
  return (rows + 255) / 256 * 256;
}

// Walks one (past, n) prefill; returns the number of tile copies that leave
// `cap` rows.  old_rule: the steady condition without "t + 1 < nt".
static long long prefill_violations(int past, int n, long long cap, bool old_rule) {
  long long bad = 0;
  auto copy = [&](int T) {
    if ((long long)T * mi::kPrefillBK + mi::kPrefillBK > cap) bad++;
  };
  const int ntiles = (n + mi::kPrefillBQ - 1) / mi::kPrefillBQ;
  for (int qt = 0; qt < ntiles; qt++)
    for (int w = 0; w < 4; w++) {
      const mi::PrefillWave p = mi::prefill_wave(past, n, qt, w);
      copy(0);
      bool pending = false;
      for (int t = 0; t < p.nt; t++) {
        const bool active = mi::prefill_active(p, t);
        bool steady = mi::prefill_steady(p, t, pending);
        if (old_rule) steady = active && pending && !mi::prefill_diag(p, t);
        if (steady) {
          copy(t + 1);
        } else if (t + 1 < p.nt) {
          copy(t + 1);
        }
        copy(t);  // V(t)
        pending = active;
      }
    }
  return bad;
}

// The same for attn_prefill64_kernel: every pass (the walk, and after an
// overflow the max pass and the walk again) copies K(0) first; tile 0's asm
// block copies K(min(1, nt - 1)) and V(0); at tile t >= 1 an active wave
// (mi::prefill64_active) copies K(min(t + 1, nt - 1)) in its asm block and
// V(t) from its PV phase, any other copies K(t + 1) when t + 1 < nt, and
// V(t) (the max pass: K only).  Both passes are walked.
static long long prefill64_violations(int past, int n, long long cap) {
  long long bad = 0;
  auto copy = [&](int T) {
    if ((long long)T * mi::kPrefillBK + mi::kPrefillBK > cap) bad++;
  };
  const int ntiles = (n + mi::kPrefillBQ - 1) / mi::kPrefillBQ;
  for (int qt = 0; qt < ntiles; qt++)
    for (int w = 0; w < 4; w++) {
      const mi::PrefillWave64 p = mi::prefill_wave64(past, n, qt, w & 1, w >> 1);
      const int nt = p.nt;
      for (int pass = 0; pass < 2; pass++) {  // 0: walk, 1: max pass
        copy(0);
        for (int t = 0; t < nt; t++) {
          const int tk = t + 1 < nt ? t + 1 : t;
          if (t == 0 || mi::prefill64_active(p, t)) {
            copy(tk);
            if (pass == 0) copy(t);  // V(t)
          } else {
            if (t + 1 < nt) copy(t + 1);
            if (pass == 0) copy(t);
          }
        }
      }
    }
  return bad;
}

// The wide verify / split-K prefill (attn_verify_wide_kernel): plan
// mi::wide_plan (two KV heads); workgroup (row block rb of 16 tokens, chunk
// c): keys from kbeg = c * chunk, wave (qb, kp) walking mi::verify_wave64's
// tiles with the 64-query kernel's copies (K(0) first; then K(min(t + 1,
// nt - 1)) and V(t) at tile 0 and on active tiles, else K(t + 1) when
// t + 1 < nt and V(t); the max pass copies K only), tile T being rows
// [kbeg + 64 T, + 64).  Every copy must lie inside `cap` rows, the chunks
// must be whole tiles, at most kMaxSplitChunks, and cover [0, past + n),
// and each token's visible keys within a chunk must lie inside the tiles
// its workgroup walks.
static long long wide_violations(long long past, int n, long long cap) {
  const mi::WidePlan wp = mi::wide_plan(2, past, n);
  long long bad = 0;
  if (wp.chunk % mi::kPrefillBK || wp.nchunks > mi::kMaxSplitChunks ||
      (long long)wp.nchunks * wp.chunk < past + n)
    bad++;
  const int nrb = (n + 15) / 16;
  for (int rb = 0; rb < nrb; rb++)
    for (int c = 0; c < wp.nchunks; c++) {
      const long long kbeg = (long long)c * wp.chunk;
      auto copy = [&](int T) {
        if (kbeg + (long long)T * mi::kPrefillBK + mi::kPrefillBK > cap) bad++;
      };
      for (int w = 0; w < 4; w++) {
        const mi::PrefillWave64 p = mi::verify_wave64(past, n, kbeg, wp.chunk, 16 * rb, w & 1, w >> 1);
        const int nt = p.nt;
        for (int pass = 0; pass < 2; pass++) {
          copy(0);
          for (int t = 0; t < nt; t++) {
            const int tk = t + 1 < nt ? t + 1 : t;
            if (t == 0 || mi::prefill64_active(p, t)) {
              copy(tk);
              if (pass == 0) copy(t);
            } else {
              if (t + 1 < nt) copy(t + 1);
              if (pass == 0) copy(t);
            }
          }
        }
        // tokens of this wave's rows: tok0 + 8 qb .. + 7
        for (int i = 16 * rb + 8 * (w & 1); i < 16 * rb + 8 * (w & 1) + 8 && i < n; i++) {
          long long vis_end = past + i + 1;  // keys [0, past + i]
          if (vis_end > kbeg + wp.chunk) vis_end = kbeg + wp.chunk;
          if (vis_end > kbeg && vis_end > kbeg + p.kv_len) bad++;
        }
      }
    }
  return bad;
}

// Tiles of one split launch over `len` rows with `nq` query tokens.
static long long split_violations(long long len, int nq, const mi::SplitKnobs& k) {
  const mi::SplitPlan p = mi::plan_split(len, 1, 2, nq, k);
  long long bad = 0;
  if (p.max_chunks > mi::kMaxSplitChunks || p.chunk % 32) bad++;
  const long long cap = round_cap(len);
  for (long long c = 0; c < p.max_chunks; c++) {
    const long long b = c * p.chunk;
    if (b >= len) continue;
    const long long e = b + p.chunk < len ? b + p.chunk : len;
    long long covered = 0;
    for (int w = 0; w < p.nwh; w++) {
      const mi::WaveTiles wt = mi::split_wave_tiles(b, e, p.nwh, w);
      for (long long k0 = wt.first; k0 < wt.last; k0 += 32) {
        if (k0 % 32 || k0 + 32 > cap) bad++;
        covered += (k0 + 32 < e ? k0 + 32 : e) - k0;
      }
    }
    if (covered != e - b) bad++;
  }
  if ((long long)p.max_chunks * p.chunk < len) bad++;  // every key covered
  return bad;
}

int main() {
  long long cases = 0, bad_new = 0, bad_old = 0, bad64 = 0;
  for (int past = 0; past < 700; past++)
    for (int n = 1; n < 700; n++) {
      const long long cap = round_cap((long long)past + n);
      bad_new += prefill_violations(past, n, cap, false);
      bad_old += prefill_violations(past, n, cap, true);
      bad64 += prefill64_violations(past, n, cap);
      cases++;
    }
  std::printf("prefill %lld %lld\n", cases, bad_new);
  std::printf("prefill_without_last_tile_rule %lld %lld\n", cases, bad_old);
  std::printf("prefill64 %lld %lld\n", cases, bad64);
  // long pasts and C4-adjacent sizes
  long long c2 = 0, b2 = 0;
  for (int past : {0, 32768, 65000, 65535, 131071})
    for (int n : {1, 127, 128, 129, 257, 1000, 4095, 4096, 4097}) {
      b2 += prefill_violations(past, n, round_cap((long long)past + n), false);
      b2 += prefill64_violations(past, n, round_cap((long long)past + n));
      c2++;
    }
  std::printf("prefill_long %lld %lld\n", c2, b2);

  const mi::SplitKnobs knobs[] = {{2, 256, 0}, {1, 256, 0}, {2, 1000, 0}, {2, 7, 0}, {2, 256, 100}};
  long long cs = 0, bs = 0;
  for (const auto& k : knobs)
    for (int nq = 1; nq <= 4; nq++) {
      for (long long len = 1; len <= 5000; len++) {
        bs += split_violations(len, nq, k);
        cs++;
      }
      for (long long len : {32767LL, 32768LL, 32769LL, 65536LL, 65540LL, 262144LL, 262161LL,
                            1000000LL, 2097152LL, 4194304LL}) {
        bs += split_violations(len, nq, k);
        cs++;
      }
    }
  std::printf("split %lld %lld\n", cs, bs);

  long long cw = 0, bw = 0;
  for (long long past : {0LL, 1LL, 63LL, 64LL, 65LL, 700LL, 2048LL, 4096LL, 20000LL, 65536LL,
                         131071LL})
    for (int n = 1; n <= 1100; n += (n < 40 ? 1 : 37)) {
      bw += wide_violations(past, n, round_cap(past + n));
      cw++;
    }
  std::printf("wide %lld %lld\n", cw, bw);
  return 0;
}
