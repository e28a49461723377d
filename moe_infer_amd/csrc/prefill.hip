// Causal batched prefill: flash-attention forward on gfx950 MFMA.
//
// Reference semantics: op1_full_batched (src/engine/qwen35_moe/batched.rs:
// 233-260): kv_cache_append_n of the n new rows at past_pos, then
// attn_sdpa_causal_n (src/engine/shaders.metal:2656-2769) where query i
// attends rows [0, past_pos + i] inclusive, then sigmoid_gate per token.
//
// Design:
//  * Workgroup = 4 waves = 128 queries of one query head; wave w owns 32
//    queries.  Grid order is heaviest query tile first, and the eight heads
//    of a GQA group on the same query tile are placed on one XCD so that
//    their identical K/V tile reads share that XCD's L2.
//  * K/V tiles of 64 keys are staged in LDS (double-buffered, one barrier per
//    tile); global loads of tile t+1 are in flight while tile t computes.
//  * S^T = K . Q^T with v_mfma_f32_32x32x16_f16 (A = K rows from LDS,
//    B = Q^T held in registers for the whole kernel); the online softmax is
//    per lane column (one query per lane column), so row statistics need a
//    single cross-lane step (lanes 32 apart).
//  * O^T += V^T . P^T: the V tile is kept in the cache's 8-row transposed
//    block layout, so the A operand is one 128-bit LDS read, and the QK row
//    order is chosen so that P^T is the lane's own S^T accumulator.
//  * Epilogue: divide by the row sum, multiply by sigmoid(gate), write f16.
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "plan.h"

namespace {

constexpr int D = mi::kHeadDim;
constexpr int BQ = mi::kPrefillBQ;  // queries per workgroup
constexpr int BK = mi::kPrefillBK;  // keys per LDS tile
// K tile in LDS: two 32-key blocks copied verbatim from the cache layout
// (mi::k_offset), unpadded.  An A-operand read then hits each LDS bank once
// per 16-byte slot (rocprofv3 SQ_LDS_BANK_CONFLICT: 0); with the two row
// halves u of a block 128 bytes out of step, half of that read's LDS cycles
// were bank conflicts on gfx950.
constexpr int KU = 16 * D;                  // one u half (halves)
constexpr int KSUB = 2 * KU;                // one 32-key block
constexpr int K_TILE_HALVES = 2 * KSUB;
constexpr int V_TILE_HALVES = BK * D;  // 8 blocks of [D][8]
// LDS: K tiles double-buffered at [0, 2*K_TILE_HALVES), V tiles after them.
constexpr int LDS_HALVES = 2 * (K_TILE_HALVES + V_TILE_HALVES);
// Epilogue staging of O (f32, one padded row of D per query of the 4 waves),
// over the tile buffers once every wave has finished its last tile.
constexpr int O_ROW = D + 4;
constexpr int LDS_BYTES = LDS_HALVES * 2 > 4 * 32 * O_ROW * 4 ? LDS_HALVES * 2 : 4 * 32 * O_ROW * 4;
constexpr float kNegBig = -1e30f;
// attn_prefill64_kernel's restart flag (one int), past the tile buffers.
constexpr int LDS_FLAG_OFF = (LDS_BYTES + 1024) / 2;  // in halves
constexpr int LDS64_BYTES = LDS_BYTES + 1024 + 16;

struct PrefillArgs {
  const _Float16* q;      // [n][H][D]
  const _Float16* k;      // cache K, token-major [cap][G*D]
  const _Float16* v;      // cache V blocks
  const _Float16* gate;   // [n][H][D] or null
  _Float16* out;          // [n][H][D]
  int64_t past;           // past_pos
  int n, H, G, ntiles, work;
  float scale_log2e;
};

// Wide verify (attn_verify_wide_kernel): workgroup = (key chunk, KV head);
// rows are (token, query head of the group) pairs, row = 8 token + head;
// keys [c chunk, (c + 1) chunk) of [0, past + n); unnormalised partials
// (O, m, l) go to part_o [G][nslots][ncols][D] / part_ml [..][2] for the
// combine kernel (ncols = 8 n).
struct VerifyArgs {
  int64_t chunk;
  int nchunks, ncols;
  int64_t nslots;
  float* part_o;
  float* part_ml;
};

// Row m of a 32-key QK tile holds key swap_bits_2_3(m): then accumulator
// element e of lane half hl (row 8*(e/4) + 4*hl + e%4) is key
// 16*(e/8) + 8*hl + e%8, i.e. the PV step e/8 sees eight consecutive keys
// per lane half — one V block.
__device__ __forceinline__ int qk_row_key(int m) {
  return (m & 0x13) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Buffer resource over a wave-uniform base: no stride, 2^31-1 bytes,
// dword3 0x00020000 (32-bit data format, the value raw untyped buffer loads
// take on CDNA).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

// blockIdx -> (KV head, head in group, query tile), heaviest query tile
// first.  Dispatch is round-robin over the 8 XCDs (bid % 8), and the eight
// query heads of one (query tile, KV head) go to one XCD, so that their
// identical K/V tile reads share its L2.  With two KV heads, XCDs 0-3 take
// KV head 0 and XCDs 4-7 KV head 1, so an XCD's L2 holds one head's K/V
// (4 MiB at 4096 rows) rather than both; the query tiles of a KV head are
// dealt to its four XCDs in a snake (block j of 4 tiles: XCD i takes tile
// rank 4j + i for even j, 4j + 3 - i for odd j), which gives every XCD the
// same causal work.  Other head counts deal (query tile, KV head) groups
// over all 8 XCDs in the same snake.  The grid is (8 heads x ntiles x G)
// rounded up to 64 workgroups; returns false for its padding.
__device__ __forceinline__ bool prefill_item(int bid, const PrefillArgs& a, int& kvh, int& hg,
                                             int& qtile) {
  const int xcd = bid & 7, r = bid >> 3;
  hg = r & 7;
  const int jb = r >> 3;
  int rank;
  if (a.G == 2) {
    const int xi = xcd & 3;
    kvh = xcd >> 2;
    rank = 4 * jb + ((jb & 1) ? 3 - xi : xi);
  } else {
    const int grp = 8 * jb + ((jb & 1) ? 7 - xcd : xcd);
    kvh = grp % a.G;
    rank = grp / a.G;
  }
  qtile = a.ntiles - 1 - rank;
  return rank < a.ntiles;
}

__global__ void __launch_bounds__(256, 1)
attn_prefill_kernel(PrefillArgs a) {
  extern __shared__ _Float16 lds[];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hl = lane >> 5;   // lane half
  const int col = lane & 31;  // query column of this lane

  int kvh, hg, qtile;
  if (!prefill_item(blockIdx.x, a, kvh, hg, qtile)) return;
  const int hq = kvh * 8 + hg;
  const int q0 = qtile * BQ;

  // Q^T operand for this lane's query: 16 k-steps of 8 halves.
  const int qi = q0 + 32 * w + col;
  f16x8 qf[16];
  if (qi < a.n) {
    const _Float16* qp = a.q + ((int64_t)qi * a.H + hq) * D + 8 * hl;
#pragma unroll
    for (int ks = 0; ks < 16; ks++) qf[ks] = *(const f16x8*)(qp + 16 * ks);
  } else {
#pragma unroll
    for (int ks = 0; ks < 16; ks++) qf[ks] = f16x8{};
  }
  // In-kernel positions are 32-bit (the host checks past + n < 2^31).
  const int past = (int)a.past;
  const int qpos = past + qi;  // this lane's query position
  const mi::PrefillWave pw = mi::prefill_wave(past, a.n, qtile, w);
  const int kv_len = pw.kv_len;
  const int nt = pw.nt;
  const float c2 = a.scale_log2e;

  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = f32x16{};
  float m = kNegBig, l = 0.f;

  // Tiles move global -> LDS directly (buffer_load_dwordx4 ... lds: each
  // lane's 16 bytes land at the wave's LDS base + 16 * lane), no staging
  // registers.  The buffer (MUBUF) form rather than global_load_lds: the
  // compiler counts a global_load_lds as a possible LDS-counter event, and
  // while one is pending it turns every LDS wait of the block into
  // lgkmcnt(0), so the K/V fragment reads could not stay in flight across
  // MFMAs.  Buffer bases are per tile (wave-uniform), offsets 32-bit.
  // A tile is 32 one-KiB pieces of K (two 32-key blocks of 16 KiB, each
  // block's two row halves u, KU apart) and 32 pieces of V (eight 4 KiB
  // 8-key blocks, contiguous); wave w moves pieces 8w .. 8w+7 of each.
  const int lane16 = lane * 8;  // halves
  // The wave index as a scalar, so that the copies' LDS addresses (M0) are
  // computed on the scalar unit.
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const _Float16* kg = a.k + (int64_t)kvh * (32 * D);
  const _Float16* vg = a.v + (int64_t)kvh * (D * 8);
  const int64_t kblk_stride = (int64_t)a.G * (32 * D);  // one 32-key block, all heads
  const int64_t vblk_stride = (int64_t)a.G * (D * 8);   // one 8-key block, all heads
  _Float16* const kbuf0 = lds;
  _Float16* const vbuf0 = lds + 2 * K_TILE_HALVES;
  auto load_k_piece = [&](int t, int pi) {
    const _Float16* kt = kg + (int64_t)(t * 2) * kblk_stride;
    _Float16* ks = kbuf0 + (t & 1) * K_TILE_HALVES;
    const int i = 8 * wu + pi;
    const int b = i >> 4, u = (i >> 3) & 1, pc = i & 7;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        buf_rsrc(kt), (__attribute__((address_space(3))) void*)(ks + b * KSUB + u * KU + pc * 512), 16,
        2 * (lane16 + b * (int)kblk_stride + (u * 8 + pc) * 512), 0, 0, 0);
  };
  auto load_v_piece = [&](int t, int pi) {
    const _Float16* vt = vg + (int64_t)(t * 8) * vblk_stride;
    _Float16* vs = vbuf0 + (t & 1) * V_TILE_HALVES;
    const int i = 8 * wu + pi;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        buf_rsrc(vt), (__attribute__((address_space(3))) void*)(vs + i * 512), 16,
        2 * (lane16 + (i >> 2) * (int)vblk_stride + (i & 3) * 512), 0, 0, 0);
  };
  auto load_k = [&](int t) {
    const _Float16* kt = kg + (int64_t)(t * 2) * kblk_stride;
    _Float16* ks = kbuf0 + (t & 1) * K_TILE_HALVES;
#pragma unroll
    for (int pi = 0; pi < 8; pi++) {
      const int i = 8 * wu + pi;
      const int b = i >> 4, u = (i >> 3) & 1, pc = i & 7;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          buf_rsrc(kt), (__attribute__((address_space(3))) void*)(ks + b * KSUB + u * KU + pc * 512), 16,
          2 * (lane16 + b * (int)kblk_stride + (u * 8 + pc) * 512), 0, 0, 0);
    }
  };
  auto load_v = [&](int t) {
    const _Float16* vt = vg + (int64_t)(t * 8) * vblk_stride;
    _Float16* vs = vbuf0 + (t & 1) * V_TILE_HALVES;
#pragma unroll
    for (int pi = 0; pi < 8; pi++) {
      const int i = 8 * wu + pi;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          buf_rsrc(vt), (__attribute__((address_space(3))) void*)(vs + i * 512), 16,
          2 * (lane16 + (i >> 2) * (int)vblk_stride + (i & 3) * 512), 0, 0, 0);
    }
  };
  // Rows of the last tile past kv_len may hold stale data (NaN included):
  // zero their V entries in LDS once the tile has landed.  Thread t owns
  // value column t of every 8-key block.
  auto zero_v_tail = [&](int t) {
    _Float16* vs = vbuf0 + (t & 1) * V_TILE_HALVES;
    for (int b = 0; b < 8; b++) {
      const int valid = kv_len - (t * BK + 8 * b);
      if (valid >= 8) continue;
      _Float16* col8 = vs + (b * D + threadIdx.x) * 8;
#pragma unroll
      for (int e = 0; e < 8; e++)
        if (e >= valid) col8[e] = (_Float16)0.f;
    }
  };

  const bool tail_tile = (kv_len % BK) != 0;  // the last tile has rows past kv_len

  // A-operand row `col` of each 32-key block is key qk_row_key(col); its
  // chunk 2k + hl sits at (u, j) of the block layout.
  const int krow = qk_row_key(col);
  const int k_lds_off = ((krow >> 2) & 1) * KU + hl * 128 + (((krow >> 3) << 2) | (krow & 3)) * 8;

  // P . V of one tile: O^T += V^T P^T over its 64 keys, in 4 steps of 16
  // keys (V block sub*4 + 2*stp + hl holds keys sub*32 + 16*stp + 8*hl ..
  // +7); the 8 fragments of step s+1 are read while step s's MFMAs run.
  auto pv = [&](int t, const f16x8 (&pf)[2][2]) {
    const _Float16* vs = vbuf0 + (t & 1) * V_TILE_HALVES + hl * (D * 8) + col * 8;
    f16x8 vf[2][8];
#pragma unroll
    for (int i = 0; i < 8; i++) vf[0][i] = *(const f16x8*)(vs + i * 32 * 8);
#pragma unroll
    for (int st4 = 0; st4 < 4; st4++) {
      if (st4 + 1 < 4) {
        const _Float16* vb = vs + 2 * (st4 + 1) * (D * 8);  // block sub*4 + 2*stp = 2*step
#pragma unroll
        for (int i = 0; i < 8; i++) vf[(st4 + 1) & 1][i] = *(const f16x8*)(vb + i * 32 * 8);
      }
#pragma unroll
      for (int i = 0; i < 8; i++)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[st4 & 1][i], pf[st4 >> 1][st4 & 1],
                                                        acc[i], 0, 0, 0);
    }
  };

  // Software pipeline over tiles: iteration t issues QK(t), then the PV
  // MFMAs of tile t-1 (independent of QK(t)) run while the softmax of tile
  // t executes on the VALU.  K runs one tile ahead of V: iteration t loads
  // K(t+1) and V(t), so K and V each need only a double buffer.  After
  // iteration t, acc = alpha_t * O_{t-1}; the epilogue adds P_{nt-1} V_{nt-1}.
  load_k(0);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): this wave's pieces have landed
  __syncthreads();

  f16x8 pprev[2][2];
  bool pending = false;  // PV of the previous tile still to do
  // QK^T of tile t (outside the steady state): two 32-key sub-tiles, 16
  // k-steps each, the two chains interleaved.
  auto qk = [&](int t, f32x16 (&st)[2]) {
    const _Float16* ks = kbuf0 + (t & 1) * K_TILE_HALVES;
    const _Float16* kr0 = ks + k_lds_off;
    const _Float16* kr1 = ks + KSUB + k_lds_off;
    f32x16 c0 = f32x16{}, c1 = f32x16{};
    // K fragments are read kAhead k-steps before their MFMA (LDS latency).
    constexpr int kAhead = 4;
    f16x8 ka[16], kb[16];
#pragma unroll
    for (int k = 0; k < kAhead; k++) {
      ka[k] = *(const f16x8*)(kr0 + 256 * k);
      kb[k] = *(const f16x8*)(kr1 + 256 * k);
    }
#pragma unroll
    for (int k = 0; k < 16; k++) {
      if (k + kAhead < 16) {
        ka[k + kAhead] = *(const f16x8*)(kr0 + 256 * (k + kAhead));
        kb[k + kAhead] = *(const f16x8*)(kr1 + 256 * (k + kAhead));
      }
      c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[k], qf[k], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb[k], qf[k], c1, 0, 0, 0);
    }
    st[0] = c0;
    st[1] = c1;
  };
  // Online softmax of one tile's raw scores: reference max, alpha, P (f16),
  // l.  The scale (1/sqrt(D) * log2 e > 0) is folded into the exponent, so
  // the row max is taken on raw scores.  The reference max m of a row moves
  // only when the tile's max exceeds it by more than kLazy (base-2 units):
  // P = 2^(s - m) then stays below 2^kLazy (well inside f16 and f32), the
  // final normalisation divides by l accumulated against the same m, and
  // the O rescale (alpha != 1) becomes rare.  The row sum adds the f16
  // weights the PV MFMA uses (v_dot2_f32_f16 against (1, 1), f32
  // accumulation), so that the normalised weights sum to one.
  constexpr float kLazy = 8.f;
  auto softmax = [&](f32x16 (&st)[2], float& alpha) {
    float mt = st[0][0];
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int e = 0; e < 16; e++) mt = fmaxf(mt, st[sub][e]);
    mt = mi::max_xor32(mt) * c2;
    const float mnew = (mt > m + kLazy) ? mt : m;
    alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    float rs = 0.f;
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const f16x2 ph = {(_Float16)__builtin_amdgcn_exp2f(fmaf(st[sub][e], c2, -mnew)),
                          (_Float16)__builtin_amdgcn_exp2f(fmaf(st[sub][e + 1], c2, -mnew))};
        rs = __builtin_amdgcn_fdot2(ph, f16x2{1.f16, 1.f16}, rs, false);
        pprev[sub][e >> 3][e & 7] = ph[0];
        pprev[sub][e >> 3][(e & 7) + 1] = ph[1];
      }
    rs = mi::sum_xor32(rs);
    l = l * alpha + rs;
  };
  // Steady-state tile, one basic block in a fixed issue order (each slot
  // closed by a scheduling barrier, so the compiler keeps it):
  //  * QK(t): 16 k-steps of two MFMAs; K fragments are read from LDS
  //    kRing k-steps ahead through a ring of registers (~8 reads in flight),
  //    and one global -> LDS piece of the next tiles (K(t+1) piece k/2 on
  //    even steps, V(t) piece k/2 on odd ones) is issued per step.  The last
  //    four k-steps read the V fragments of PV step 0.
  //  * PV(t-1): 4 steps of 8 MFMAs; after each MFMA the same ring slot is
  //    refilled with the next step's fragment.  Tile t's softmax runs in
  //    chunks between these MFMAs (it needs only QK(t), not PV(t-1)), and
  //    writes P(t) into pprev once PV(t-1) has consumed the old P.
  auto steady = [&](int t, float& alpha) {
    const _Float16* ks = kbuf0 + (t & 1) * K_TILE_HALVES;
    const _Float16* kr0 = ks + k_lds_off;
    const _Float16* kr1 = ks + KSUB + k_lds_off;
    const _Float16* vs = vbuf0 + ((t - 1) & 1) * V_TILE_HALVES + hl * (D * 8) + col * 8;
    constexpr int kRing = 4;
    f16x8 ka[kRing], kb[kRing], vf[8];
    f32x16 c0 = f32x16{}, c1 = f32x16{};
#pragma unroll
    for (int k = 0; k < kRing; k++) {
      ka[k] = *(const f16x8*)(kr0 + 256 * k);
      kb[k] = *(const f16x8*)(kr1 + 256 * k);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 16; k++) {
      c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[k % kRing], qf[k], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb[k % kRing], qf[k], c1, 0, 0, 0);
      if (k + kRing < 16) {
        ka[k % kRing] = *(const f16x8*)(kr0 + 256 * (k + kRing));
        kb[k % kRing] = *(const f16x8*)(kr1 + 256 * (k + kRing));
      }
      if (k >= 12) {
        const int i0 = 2 * (k - 12);
        vf[i0] = *(const f16x8*)(vs + i0 * 256);
        vf[i0 + 1] = *(const f16x8*)(vs + (i0 + 1) * 256);
      }
      if ((k & 1) == 0) load_k_piece(t + 1, k >> 1);
      else load_v_piece(t, k >> 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    f16x8 pnew[2][2];
    // The weights use the running reference max m as it stands: no row max
    // is taken in the steady state.  They are valid while none reaches 2^15
    // (f16 range; each weight is at most its lane's sum); otherwise, rarely,
    // the tile is redone below with the new row max.
    float rs = 0.f;
    bool ovf = false;
#pragma unroll
    for (int st4 = 0; st4 < 4; st4++) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i], pprev[st4 >> 1][st4 & 1], acc[i], 0, 0, 0);
        if (st4 + 1 < 4) vf[i] = *(const f16x8*)(vs + 2 * (st4 + 1) * (D * 8) + i * 256);
        const int slot = st4 * 8 + i;
        if (slot >= 2 && slot < 18) {
          const int e0 = 2 * (slot - 2);  // scores e0, e0 + 1 of the 32
          const int sub = e0 >> 4, ee = e0 & 15;
          const float sa = sub ? c1[ee] : c0[ee], sb = sub ? c1[ee + 1] : c0[ee + 1];
          const f16x2 ph = {(_Float16)__builtin_amdgcn_exp2f(fmaf(sa, c2, -m)),
                            (_Float16)__builtin_amdgcn_exp2f(fmaf(sb, c2, -m))};
          rs = __builtin_amdgcn_fdot2(ph, f16x2{1.f16, 1.f16}, rs, false);
          pnew[sub][ee >> 3][ee & 7] = ph[0];
          pnew[sub][ee >> 3][(ee & 7) + 1] = ph[1];
        } else if (slot == 18) {
          ovf = !(rs < 32768.f);  // also inf / NaN
          rs = mi::sum_xor32(rs);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (__ballot(ovf)) {  // wave-uniform: a row max moved up by 15 or more
      float mt = c0[0];
#pragma unroll
      for (int e = 1; e < 16; e++) mt = fmaxf(mt, c0[e]);
#pragma unroll
      for (int e = 0; e < 16; e++) mt = fmaxf(mt, c1[e]);
      mt = mi::max_xor32(mt) * c2;
      const float mnew = fmaxf(m, mt);
      alpha = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      rs = 0.f;
#pragma unroll
      for (int e = 0; e < 32; e += 2) {
        const int sub = e >> 4, ee = e & 15;
        const float sa = sub ? c1[ee] : c0[ee], sb = sub ? c1[ee + 1] : c0[ee + 1];
        const f16x2 ph = {(_Float16)__builtin_amdgcn_exp2f(fmaf(sa, c2, -m)),
                          (_Float16)__builtin_amdgcn_exp2f(fmaf(sb, c2, -m))};
        rs = __builtin_amdgcn_fdot2(ph, f16x2{1.f16, 1.f16}, rs, false);
        pnew[sub][ee >> 3][ee & 7] = ph[0];
        pnew[sub][ee >> 3][(ee & 7) + 1] = ph[1];
      }
      rs = mi::sum_xor32(rs);
    }
    l = l * alpha + rs;
#pragma unroll
    for (int a2 = 0; a2 < 2; a2++)
#pragma unroll
      for (int b2 = 0; b2 < 2; b2++) pprev[a2][b2] = pnew[a2][b2];
  };
  for (int t = 0; t < nt; t++) {
    const int key0 = t * BK;
    const bool active = mi::prefill_active(pw, t);
    const bool diag = mi::prefill_diag(pw, t);
    float alpha = 1.f;
    f32x16 st[2];
    // Steady state: not the wave's first or diagonal tile, and not the last
    // tile (the steady schedule copies K(t+1); mi::prefill_steady).
    if (mi::prefill_steady(pw, t, pending)) {
      steady(t, alpha);
    } else {
      if (t + 1 < nt) load_k(t + 1);
      load_v(t);
      if (active) qk(t, st);
      if (pending) pv(t - 1, pprev);
      if (active) {
        if (diag) {  // causal mask: key (key0 + 16 s2 + 8 hl + e7) <= qpos
          const int rel = qpos - key0 - 8 * hl;
#pragma unroll
          for (int sub = 0; sub < 2; sub++)
#pragma unroll
            for (int e = 0; e < 16; e++)
              if (sub * 32 + 16 * (e >> 3) + (e & 7) > rel) st[sub][e] = -INFINITY;
        }
        softmax(st, alpha);
      }
    }
    // Rescale only when some row max moved (wave-uniform branch); after the
    // first tiles this is rare.
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < 8; i++) acc[i] *= alpha;
    }
    pending = active;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tail_tile && t + 1 == nt) {
      zero_v_tail(t);
      __syncthreads();
    }
  }
  if (pending) pv(nt - 1, pprev);

  // Epilogue: O / l goes to LDS as f32 rows (query-major), then every query
  // row of D outputs is written by 32 lanes with 16-byte stores (two rows per
  // wave instruction), the gate read the same way; the accumulator layout
  // would otherwise make each lane store 8 bytes into 32 rows 8 KiB apart.
  __syncthreads();  // every wave is done with the K/V tiles
  // The gate rows are loaded first, so that their latency overlaps the
  // staging of O (lane: columns dc .. dc+7 of rows 2 st + hl).
  const int dc = 8 * (lane & 31);  // this lane's 8 columns of a row
  f16x8 gv[16];
  if (a.gate) {
#pragma unroll
    for (int st = 0; st < 16; st++) {
      const int qr = q0 + 32 * w + 2 * st + hl;
      gv[st] = qr < a.n ? *(const f16x8*)(a.gate + ((int64_t)qr * a.H + hq) * D + dc) : f16x8{};
    }
  }
  float* ob = (float*)lds + w * 32 * O_ROW;
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int e4 = 0; e4 < 4; e4++) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = acc[i][4 * e4 + e] * inv;
      *(f32x4*)(ob + col * O_ROW + i * 32 + 8 * e4 + 4 * hl) = o;
    }
  mi::sync_lds();
#pragma unroll
  for (int st = 0; st < 16; st++) {
    const int r = 2 * st + hl;  // query row of the wave
    const int qr = q0 + 32 * w + r;
    if (qr >= a.n) continue;
    const float* src = ob + r * O_ROW + dc;
    const f32x4 x0 = *(const f32x4*)src, x1 = *(const f32x4*)(src + 4);
    const int64_t obase = ((int64_t)qr * a.H + hq) * D + dc;
    f16x8 y;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      y[e] = (_Float16)x0[e];
      y[4 + e] = (_Float16)x1[e];
    }
    if (a.gate) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        y[e] = (_Float16)mi::gate_mul(x0[e], (float)gv[st][e]);
        y[4 + e] = (_Float16)mi::gate_mul(x1[e], (float)gv[st][4 + e]);
      }
    }
    *(f16x8*)(a.out + obase) = y;
  }
}


// ---------------------------------------------------------------------------
// 64 queries per wave.  Workgroup = 4 waves over the same 128 queries of one
// query head as attn_prefill_kernel, with the same LDS tiles and copy
// schedule; wave w owns query rows 64 (w & 1) .. + 63 (two 32-query MFMA
// column blocks) and the key half kp = w >> 1 of every 64-key tile (32
// keys).  Each K or V fragment read from LDS feeds two MFMAs (one per column
// block), which halves the LDS read bytes per MFMA.  O^T of 64 queries is
// 256 accumulation registers, so the scores must come out in ordinary
// registers: the QK chain of a tile is one asm block (32 MFMAs with the K
// fragment reads and the tile's 16 copy pieces), the rest is compiled code.
// The two key halves of a query row merge through LDS at the end: wave
// (qb, kp) finishes column block kp of its rows.

__global__ void __launch_bounds__(256, 1) attn_prefill64_kernel(PrefillArgs a) {
  constexpr bool VERIFY = false;
  const VerifyArgs vx{};
#include "prefill64_body.inc"
}

// The verify kernel takes the body through an inlined device template: the
// body placed directly in the kernel spills 173 registers there.
template <bool VERIFY>
__device__ __forceinline__ void verify_wide_body(const PrefillArgs& a, const VerifyArgs& vx) {
#include "prefill64_body.inc"
}

__global__ void __launch_bounds__(256, 1) attn_verify_wide_kernel(PrefillArgs a, VerifyArgs vx) {
  verify_wide_body<true>(a, vx);
}

// Launches attn_prefill64_kernel (prefill) or attn_verify_wide_kernel
// (`grid` workgroups of 256 threads).
mi_status launch_prefill64(const PrefillArgs& a, int grid, hipStream_t s) {
  static std::atomic<uint64_t> lds_set{0};
  MI_TRY(mi::set_lds_limit((const void*)attn_prefill64_kernel, LDS64_BYTES, lds_set));
  MI_HIP(mi::launch("attn_prefill", attn_prefill64_kernel, dim3(grid), dim3(256),
                    (size_t)LDS64_BYTES, s, a));
  return MI_OK;
}
mi_status launch_verify_wide(const PrefillArgs& a, const VerifyArgs& v, int grid,
                             hipStream_t s) {
  static std::atomic<uint64_t> lds_set{0};
  MI_TRY(mi::set_lds_limit((const void*)attn_verify_wide_kernel, LDS64_BYTES, lds_set));
  MI_HIP(mi::launch("verify_wide", attn_verify_wide_kernel, dim3(grid), dim3(256),
                    (size_t)LDS64_BYTES, s, a, v));
  return MI_OK;
}

// Whether mi_attn_prefill takes the split-K form (the wide verify's pass and
// merge): up to 1024 new tokens after a past of at least 2048 rows and
// twice the new tokens.  Timed, split-K against the prefill grid (µs):
// past 65536: 16 / 128 / 1024 new tokens 49 / 164 / 1004 against 1434 /
// 1446 / 1489; past 4096: 64 / 256 / 1024 tokens 36 / 47 / 115 against 105 /
// 114 / 136; past 2048, 512 tokens 51 against 70.  It loses where the past
// is short next to n (past 1024, 1024 tokens: 70 against 62; no past, 256
// tokens: 32 against 20) and beyond 1024 tokens (past 32768, 1536 tokens:
// 932 against 846).  MI_ATTN_PREFILL_SPLIT=0 (read at each call) turns it
// off.
bool prefill_split_k(int64_t past, int32_t n) {
  const char* e = getenv("MI_ATTN_PREFILL_SPLIT");
  if (e && *e && atoi(e) == 0) return false;
  return n <= 1024 && past >= 2048 && past >= 2 * (int64_t)n;
}

// Queries per wave of the prefill kernel: 64 (attn_prefill64_kernel, the
// default) or 32 (attn_prefill_kernel, MI_ATTN_PREFILL_QPW=32: the earlier
// form, kept for comparison).  Read at each call.
int prefill_qpw() {
  const char* e = getenv("MI_ATTN_PREFILL_QPW");
  return (e && atoi(e) == 32) ? 32 : 64;
}

}  // namespace

namespace mi {

mi_status verify_wide_split(const mi_kv* kv, int32_t layer, const _Float16* q, int64_t past,
                            int32_t n, int64_t chunk, int32_t nchunks, float* part_o,
                            float* part_ml, hipStream_t stream) {
  const int nrb = (n + 15) / 16;  // row blocks of 16 tokens
  if (n <= 0 || chunk <= 0 || chunk % BK != 0 || nchunks <= 0 ||
      (int64_t)nchunks * chunk < past + n || past + n + 2 * BK >= ((int64_t)1 << 31) ||
      (int64_t)nrb * nchunks * kv->G >= ((int64_t)1 << 31))
    return fail(MI_ERR_INVALID_ARG, "verify split: n=%d chunk=%lld nchunks=%d past=%lld", n,
                (long long)chunk, nchunks, (long long)past);
  PrefillArgs a{};
  a.q = q;
  a.k = kv->k[layer];
  a.v = kv->v[layer];
  a.past = past;
  a.n = n;
  a.H = kv->H;
  a.G = kv->G;
  a.scale_log2e = kLog2e / sqrtf((float)D);
  VerifyArgs vx{};
  vx.chunk = chunk;
  vx.nchunks = nchunks;
  vx.ncols = 8 * n;
  vx.nslots = nchunks;
  vx.part_o = part_o;
  vx.part_ml = part_ml;
  return launch_verify_wide(a, vx, nrb * nchunks * kv->G, stream);
}

}  // namespace mi

extern "C" mi_status mi_attn_prefill(mi_kv* kv, int32_t layer, const mi_f16* q,
                                     const mi_f16* k, const mi_f16* v, const mi_f16* gate,
                                     mi_f16* out, int64_t past_pos, int32_t n,
                                     mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!q || !out) return mi::fail(MI_ERR_INVALID_ARG, "null q/out");
  if (!k != !v) return mi::fail(MI_ERR_INVALID_ARG, "k and v must both be given or both NULL");
  if (n <= 0) return mi::fail(MI_ERR_INVALID_ARG, "n=%d", n);
  if (past_pos < 0) return mi::fail(MI_ERR_OUT_OF_RANGE, "past_pos=%lld", (long long)past_pos);
  if (past_pos + n + 2 * BK >= ((int64_t)1 << 31))
    return mi::fail(MI_ERR_OUT_OF_RANGE, "past_pos + n beyond 2^31 rows");
  // Tiles read up to 64 rows past the last key; capacity is a multiple of 256
  // rows, so it suffices that the rows themselves fit.
  if (k) {
    MI_TRY(mi_kv_append(kv, layer, k, v, past_pos, n, stream));
  } else {
    // rows already in the cache (e.g. from mi_qk_norm_rope_append)
    if (past_pos + n > kv->len[layer])
      return mi::fail(MI_ERR_OUT_OF_RANGE, "k = v = NULL but rows [%lld, %lld) are not in the "
                      "cache (len %lld)", (long long)past_pos, (long long)(past_pos + n),
                      (long long)kv->len[layer]);
    kv->len[layer] = past_pos + n;
  }
  hipStream_t s = (hipStream_t)stream;
  // A few tokens after a long past: the prefill grid (one workgroup per 128
  // queries and head) would leave most CUs idle while each of its
  // workgroups walks the whole past; the split-K form of the same tiles
  // spreads the past over the CUs, then merges.  Not while a graph is being
  // captured unless the workspace already suffices (growing it is refused
  // then).
  if (prefill_split_k(past_pos, n)) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    MI_HIP(hipStreamIsCapturing(s, &cs));
    if (cs == hipStreamCaptureStatusNone ||
        kv->ws_bytes >= mi::wide_workspace_bytes(kv->G, past_pos, n))
      return mi::attend_wide(kv, layer, (const _Float16*)q, (const _Float16*)gate,
                             (_Float16*)out, past_pos, n, s);
  }
  PrefillArgs a;
  a.q = (const _Float16*)q;
  a.k = kv->k[layer];
  a.v = kv->v[layer];
  a.gate = (const _Float16*)gate;
  a.out = (_Float16*)out;
  a.past = past_pos;
  a.n = n;
  a.H = kv->H;
  a.G = kv->G;
  a.ntiles = (n + BQ - 1) / BQ;
  a.work = a.ntiles * kv->G * 8;
  a.scale_log2e = mi::kLog2e / sqrtf((float)D);
  const size_t lds = LDS_BYTES;
  static_assert(LDS_FLAG_OFF * 2 >= (2 * 2 * 8 * 4 * 64 * 4 + 2 * 2 * 32 * 2) * 4,
                "attn_prefill64_kernel's merge area lies below its restart flag");
  const int grid = (a.work + 63) / 64 * 64;
  if (prefill_qpw() == 64) {
    MI_TRY(launch_prefill64(a, grid, s));
  } else {
    static std::atomic<uint64_t> lds_set{0};
    MI_TRY(mi::set_lds_limit((const void*)attn_prefill_kernel, (int)lds, lds_set));
    MI_HIP(mi::launch("attn_prefill", attn_prefill_kernel, dim3(grid), dim3(256), lds, s, a));
  }
  return MI_OK;
}
